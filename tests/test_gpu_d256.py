"""Head dim 256 (Qwen3.5 full-attention layers: 16 query / 4 KV heads) on the GPU.

The reference gates this shape with check_qwen35_math.py: block means, V1 proxy
scores, threshold selection, all-block exact attention against a dense fp32
reference, and the backend's fp_v1 path at alpha 0. The same checks run here with
its tolerances, plus oracle parity for sparse lists and the V1 route at larger
sizes, and the d = 256 tile layouts.
"""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import assert_output_close, to_np

pytestmark = pytest.mark.gpu

SCALE = 256 ** -0.5
Q_HEADS, KV_HEADS, DIM = 16, 4, 256


def qkv(length, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, length, Q_HEADS, DIM, generator=g).to(torch.bfloat16)
    k = torch.randn(1, length, KV_HEADS, DIM, generator=g).to(torch.bfloat16)
    v = torch.randn(1, length, KV_HEADS, DIM, generator=g).to(torch.bfloat16)
    return q, k, v


def dense_reference(q, k, v, scale):
    """fp32 causal attention on the CPU (check_qwen35_math.py:35-44)."""
    group = q.shape[2] // k.shape[2]
    kk = k.float().repeat_interleave(group, dim=2)
    vv = v.float().repeat_interleave(group, dim=2)
    logits = torch.einsum("bqhd,bkhd->bhqk", q.float(), kk) * scale
    pos = torch.arange(q.shape[1])
    logits.masked_fill_(pos[None, :] > pos[:, None], float("-inf"))
    lse = torch.logsumexp(logits, dim=-1).permute(0, 2, 1)
    out = torch.einsum("bhqk,bkhd->bqhd", logits.softmax(dim=-1), vv)
    return out.numpy(), lse.numpy()


class _Layer:
    layer_idx = 3


def _backend_forward(backend, qg, kg, vg):
    out, _ = backend.forward(_Layer(), qg.transpose(1, 2).contiguous(),
                             kg.transpose(1, 2).contiguous(), vg.transpose(1, 2).contiguous(),
                             None, SCALE)
    return out


def test_qwen35_gate(gpu):
    """check_qwen35_math.py:99-164 at its own shape and tolerances."""
    q, k, v = qkv(257, seed=35)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()

    mean_k = up.block_mean_k(kg)
    plain = np.stack([to_np(k)[:, s:s + 128].mean(axis=1) for s in range(0, 257, 128)], axis=1)
    np.testing.assert_allclose(to_np(mean_k), plain, atol=0.003, rtol=0.02)
    expected_mean = ref.block_mean_k(to_np(k))
    assert (np.abs(to_np(mean_k) - expected_mean) <= np.abs(expected_mean) * 2.0 ** -7 + 1e-30).all()

    scores = up.v1_scores(qg, mean_k, SCALE)
    np.testing.assert_allclose(to_np(scores), ref.v1_scores(to_np(q), to_np(mean_k), SCALE),
                               atol=3e-4, rtol=0.008)

    fourth = scores.square().square()
    idx, cnt = up.deal_output_score(fourth, 2, 4, 0.8, 2, 0)
    e_idx, e_cnt = ref.deal_output_score(to_np(fourth), 2, 4, 0.8, 2, 0)
    np.testing.assert_array_equal(to_np(idx), e_idx)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)

    all_idx, all_cnt = up.deal_output_score(torch.zeros_like(scores), 2, 4, 0.0, 2, 0)
    out, lse = up.exact_attention(qg, kg, vg, all_idx, all_cnt, SCALE)
    d_out, d_lse = dense_reference(q, k, v, SCALE)
    np.testing.assert_allclose(to_np(out), d_out, atol=0.03, rtol=0.03)
    np.testing.assert_allclose(to_np(lse), d_lse, atol=0.03, rtol=0.015)

    backend = attention.AttentionBackend(alpha=0.0, register=False)
    backend.configure("fp_v1", 0.0)
    np.testing.assert_allclose(to_np(_backend_forward(backend, qg, kg, vg)), d_out,
                               atol=0.03, rtol=0.03)


def _sparse_selection(length, seed, drop=0.4):
    blocks = ref.num_blocks(length)
    rng = np.random.default_rng(seed)
    sel = ref.protected_selection(np.zeros((1, blocks, blocks, Q_HEADS), np.float32), 0.0, 2, 4, 2)
    t = np.arange(blocks).reshape(1, -1, 1, 1)
    j = np.arange(blocks).reshape(1, 1, -1, 1)
    return sel & ~((rng.random(sel.shape) < drop) & (j < t) & (j >= 1))


@pytest.mark.parametrize("length", (1089, 2200))
def test_exact_attention_sparse_vs_oracle(gpu, length):
    q, k, v = qkv(length, seed=7)
    sel = _sparse_selection(length, seed=3)
    idx, cnt = ref.indices_from_mask(sel)
    out, lse = up.exact_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE,
                                       precision="f32")
    assert_output_close(to_np(out), e_out, what="d256 output")
    np.testing.assert_allclose(to_np(lse), e_lse, atol=0.02, rtol=0.01)   # check_math LSE bar


def test_exact_attention_list_edge_cases(gpu):
    """As in the reference: a listed future block is attended without a mask (only
    the diagonal block is masked), ids outside [0, NB) are skipped (also those whose
    low 32 bits are in range), a block listed n times is attended n times (here by
    both tiles of the pair (4, 3), twice and three times), and a count of 0 gives
    output 0 and LSE -inf."""
    length = 1089
    q, k, v = qkv(length, seed=11)
    blocks = ref.num_blocks(length)
    idx, cnt = ref.indices_from_mask(_sparse_selection(length, seed=5))
    idx, cnt = idx.copy(), cnt.copy()
    for t, h, j in ((3, 0, 5), (4, 2, blocks + 3), (6, 3, -1), (7, 4, (1 << 32) + 2),
                    (8, 5, -(1 << 32) + 3), (4, 6, 0), (3, 6, 0), (3, 6, 0)):
        idx[0, t, cnt[0, t, h], h] = j
        cnt[0, t, h] += 1
    cnt[0, 5, 1] = 0
    out, lse = up.exact_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE,
                                       precision="f32")
    assert_output_close(to_np(out), e_out, what="d256 edge lists")
    np.testing.assert_allclose(to_np(lse), e_lse, atol=0.02, rtol=0.01)
    rows = slice(5 * 128, 6 * 128)
    assert (to_np(out)[0, rows, 1] == 0).all() and np.isneginf(to_np(lse)[0, rows, 1]).all()


@pytest.mark.parametrize("length", (1089, 2200))
def test_fp_v1_route_and_layer_vs_oracle(gpu, length):
    q, k, v = qkv(length, seed=13)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=0.08, register=False)
    backend.configure("fp_v1", 0.08)
    out = _backend_forward(backend, qg, kg, vg)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, "fp_v1", 0.08,
                                   precision="f32")
    record = {"events": {}}
    _, _, _, _, _, _, sel = backend._route_v1(qg, kg, vg, SCALE, record, False, False)
    mism = (to_np(sel) != expected["selected"]).sum()
    assert mism <= max(2, expected["selected"].size // 5000)   # threshold ties only
    # always compared: the oracle layer given the GPU's own selection
    want, _ = ref.attention_from_selection(to_np(q), to_np(k), to_np(v), SCALE, "fp_v1",
                                           to_np(sel), precision="f32")
    assert_output_close(to_np(out), want, what="d256 fp_v1 layer")
    if mism == 0:
        np.testing.assert_array_equal(want, expected["output"])


def test_v1_route_ring_wraps_vs_oracle(gpu):
    """12500 tokens = 98 blocks: the route kernel streams block means in four
    32-block chunks through its 3-slot LDS ring at d = 256, so slots are reused
    and partial sums merged across chunks. Scores against the oracle; the fused
    mask and lists against the selection rule on the kernel's own scores."""
    length, alpha = 12500, 0.08
    q, k, v = qkv(length, seed=19)
    qg, kg = q.cuda(), k.cuda()
    mean_k = up.block_mean_k(kg)
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    record = {"events": {}}
    _, kbar, scores, idx, cnt, sel = backend._v1_selection(qg, kg, SCALE, record, None, True)
    assert torch.equal(kbar, mean_k)
    s = to_np(scores)
    np.testing.assert_allclose(s, ref.v1_scores(to_np(q), to_np(kbar), SCALE, precision="f32"),
                               atol=3e-4, rtol=0.008)   # check_qwen35_math tolerances
    e_idx, e_cnt = ref.deal_output_score(s, 2, 4, alpha, 2, 0)
    np.testing.assert_array_equal(to_np(idx), e_idx)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)
    np.testing.assert_array_equal(to_np(sel), ref.mask_from_indices(e_idx, e_cnt))


def test_dense_hip_vs_reference(gpu):
    q, k, v = qkv(1089, seed=17)
    backend = attention.AttentionBackend(register=False, dense_impl="hip")
    backend.configure("dense")
    out = _backend_forward(backend, q.cuda(), k.cuda(), v.cuda())
    d_out, _ = dense_reference(q, k, v, SCALE)
    assert_output_close(to_np(out), d_out, what="d256 dense hip")


@pytest.mark.parametrize("length", (257, 1089))
def test_attention_tiles_layout_d256(gpu, length):
    """Key tiles [128 keys][256 dims], chunk c of row r at c ^ (r & 15); value tiles
    four 32-key sub-blocks [256 dims][32 slots], chunk c of dim row d at
    c ^ ((d >> 2) & 3), slot -> key permutation inside each 16-key chunk."""
    _, k, v = qkv(length, seed=19)
    kt, vt = (to_np(x) for x in up.attention_tiles(k.cuda(), v.cuda()))
    blocks = kt.shape[2]
    pad = blocks * 128 - length
    kp = np.concatenate([to_np(k), np.zeros((1, pad, KV_HEADS, DIM), np.float32)], axis=1)
    vp = np.concatenate([to_np(v), np.zeros((1, pad, KV_HEADS, DIM), np.float32)], axis=1)
    r = np.arange(128)[:, None]
    c = np.arange(32)[None, :]
    pos = (c & 16) | ((c & 15) ^ (r & 15))
    chunks = kt.reshape(1, KV_HEADS, blocks, 128, 32, 8)
    unswizzled = np.take_along_axis(chunks, pos[None, None, None, :, :, None], axis=4)
    want_k = kp.reshape(1, blocks, 128, KV_HEADS, DIM).transpose(0, 3, 1, 2, 4)
    np.testing.assert_array_equal(unswizzled.reshape(want_k.shape), want_k)

    sub = vt.reshape(1, KV_HEADS, blocks, 4, DIM, 4, 8)
    d = np.arange(DIM)[:, None]
    vc = np.arange(4)[None, :]
    vpos = vc ^ ((d >> 2) & 3)
    sub = np.take_along_axis(sub, vpos[None, None, None, None, :, :, None], axis=5)
    sub = sub.reshape(1, KV_HEADS, blocks, 4, DIM, 32)
    s = np.arange(32)
    key_of_slot = (s // 16) * 16 + 4 * ((s % 16) // 8) + (s % 4) + 8 * ((s % 8) // 4)
    vb = vp.reshape(1, blocks, 4, 32, KV_HEADS, DIM)[:, :, :, key_of_slot]   # [1, NB, 4, slot, g, d]
    want_v = vb.transpose(0, 4, 1, 2, 5, 3)
    np.testing.assert_array_equal(sub, want_v)


def test_unsupported_head_dim_raises(gpu):
    """Head dims other than 128 and 256 are refused with ValueError by every path
    (the kernels' SPX_EUNSUPPORTED), before any launch."""
    g = torch.Generator().manual_seed(23)
    q = torch.randn(1, 257, 8, 64, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(1, 257, 2, 64, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(1, 257, 2, 64, generator=g).to(torch.bfloat16).cuda()
    backend = attention.AttentionBackend(alpha=0.08, register=False)
    for method in ("fp_v1", "mean_native", "cgf_mean", "fp_v1_rescue"):
        backend.configure(method, 0.08)
        with pytest.raises(ValueError, match="head_dim"):
            backend.forward(_Layer(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                            None, 64 ** -0.5)


@pytest.mark.parametrize("tail", ("none", "mean", "rescue_v2"))
def test_random_unsorted_lists(gpu, tail):
    """The head_dim 256 kernel on seeded random lists (random subsets of the causal
    blocks in random order, repeats, empty rows, garbage past the counts): exact
    blocks alone, with the fused block-mean tail, and with the fused rescue tail and
    remainder, against the oracle's exact part, tail and logaddexp merge."""
    from tests.test_gpu_kernels import _random_lists
    length, seed = 1089, 127
    q, k, v = qkv(length, seed=seed)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    idx, cnt = _random_lists(ref.num_blocks(length), seed, heads=Q_HEADS)
    backend = attention.AttentionBackend(register=False)
    _, desc, tiles = backend._pool(kg, vg, False, tail != "none", True)
    ig, cg = torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda()
    x_out, x_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE,
                                       precision="f32")
    sel = ref.mask_from_indices(idx, cnt)
    if tail == "none":
        out, lse = backend._attention(qg, kg, tiles, ig, cg, SCALE, None)
        e_out, e_lse = x_out, x_lse
    elif tail == "mean":
        out, lse = backend._attention(qg, kg, tiles, ig, cg, SCALE, desc)
        e_desc = ref.BlockDescriptors(*(to_np(getattr(desc, n)) for n in
                                        ("mean_k", "mean_v", "var_k", "sigma_v", "counts")))
        m_out, m_lse = ref.mean_tail(to_np(q), e_desc, sel, SCALE)
        e_out, e_lse = ref.merge_exact_mean(x_out, x_lse, m_out, m_lse)
    else:
        choice = kernels.rescue_choice(qg, tiles[0])
        out, lse = backend._attention(qg, kg, tiles, ig, cg, SCALE, None,
                                      rescue=(choice, True, desc, vg))
        r_out, r_lse = ref.rescue_tail(to_np(q), to_np(k), to_np(v), sel, SCALE, remainder=True,
                                       choice=to_np(choice))
        e_out, e_lse = ref.merge_exact_mean(x_out, x_lse, r_out, r_lse)
    finite = np.isfinite(e_lse)   # -inf: tile 0 with an empty list (no key at all)
    a_out, a_lse = to_np(out), to_np(lse)
    assert_output_close(a_out[finite], e_out[finite], what=f"d256 random lists, tail {tail}")
    assert (a_out[~finite] == 0).all()
    np.testing.assert_array_equal(np.isfinite(a_lse), finite)
    np.testing.assert_allclose(a_lse[finite], e_lse[finite], atol=0.02, rtol=0.01)
