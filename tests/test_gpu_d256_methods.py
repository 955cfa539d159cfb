"""The sparse methods at head dim 256 (16 query / 4 KV heads, Qwen3.5's full-attention
layer shape): the reference's kernels.py paths are head-dim generic, and so is the
oracle. Through the backend against the oracle layer (routing masks up to threshold
ties), plus the stand-alone tail and merge entry points.

Q and K are scaled by 4 and alpha is 0.7 so that routing drops blocks and the
block-mean / rescue tails are non-empty; outputs then reach several units, where
one bf16 output step (2^-7 relative) is admitted beyond the 2e-2 bar."""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels, synthetic
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import assert_output_close, masks_equal_except_ties, threshold_ties, to_np

pytestmark = pytest.mark.gpu

LENGTH = 2113   # 17 blocks, the last one 65 rows
ALPHA = 0.7
Q_HEADS, KV_HEADS, DIM = 16, 4, 256
SCALE = DIM ** -0.5
D256_METHODS = attention.METHODS[1:]   # every method but dense (test_gpu_d256.py)


class _Layer:
    layer_idx = 0


def _inputs(length=LENGTH, seed=91):
    q, k, v, _ = synthetic.make_inputs(length, seed=seed, q_heads=Q_HEADS, kv_heads=KV_HEADS,
                                       head_dim=DIM)
    scaled = lambda x: (x.float() * 4.0).to(torch.bfloat16)
    return scaled(q), scaled(k), v


@pytest.mark.parametrize("method", D256_METHODS)
def test_methods_d256_vs_oracle(gpu, method):
    q, k, v = _inputs()
    backend = attention.AttentionBackend(alpha=ALPHA, register=False)
    backend.configure(method, ALPHA)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    out, _ = backend.forward(_Layer(), qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2),
                             None, SCALE)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, ALPHA)
    assert out.shape == (1, LENGTH, Q_HEADS, DIM)
    blocks = ref.num_blocks(LENGTH)
    assert expected["selected"].sum() < Q_HEADS * blocks * (blocks + 1) // 2   # sparse
    record = {"events": {}}
    if method in attention.V1_ROUTED_METHODS:
        _, _, _, _, _, _, sel = backend._route_v1(qg, kg, vg, SCALE, record, False, False)
        unexplained, _, _ = masks_equal_except_ties(to_np(sel), expected["selected"],
                                                     threshold_ties(expected["scores"], ALPHA))
        assert unexplained == 0
    else:
        _, _, _, _, sel = backend._new_selection(qg, kg, vg, SCALE, record)
        ties = threshold_ties(expected["scores"], ALPHA, positive_rule=True)
        unexplained, _, _ = masks_equal_except_ties(to_np(sel), expected["selected"], ties)
        assert unexplained == 0
    # always compared: the oracle layer given the GPU's own selection (and, for the
    # rescue methods, the GPU's rescue tokens: fp32 near-ties may pick another)
    choice = None
    if method in attention.RESCUE_METHODS:
        choice = to_np(kernels.rescue_choice(qg, up.attention_tiles(kg, vg)[0]))
    want, _ = ref.attention_from_selection(to_np(q), to_np(k), to_np(v), SCALE, method,
                                           to_np(sel), choice=choice)
    assert_output_close(to_np(out), want, what=f"{method} d256 (GPU lists)", rel=2.0 ** -7)
    if method not in attention.RESCUE_METHODS:
        assert_output_close(to_np(out), expected["output"], what=f"{method} d256", rel=2.0 ** -7)


@pytest.mark.parametrize("selector", ("mean_balanced", "cgf_mean", "dispersion_mean"))
@pytest.mark.parametrize("length", (1089, 4500))   # 4500: two 32-block chunks per tile
def test_selector_scores_d256_vs_oracle(gpu, selector, length):
    """kernels.py:49-126 at d = 256 (two 128-dim halves per chunk) on unit-scale
    inputs, as check_math runs its selector check, within its 2e-5 tolerance of
    the oracle; rows sum to 1 over j < t."""
    q, k, v, _ = synthetic.make_inputs(length, seed=29, q_heads=Q_HEADS, kv_heads=KV_HEADS,
                                       head_dim=DIM)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    desc = kernels.block_descriptors(kg, vg)
    got = to_np(kernels.selector_scores(qg, desc, SCALE, selector))
    e_desc = ref.block_descriptors(to_np(k), to_np(v))
    want = ref.selector_scores(to_np(q), e_desc, SCALE, selector)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=2e-5)
    if selector != "dispersion_mean":
        rows = got[0, 1:].sum(axis=1)
        np.testing.assert_allclose(rows, 1.0, atol=1e-5)


def _sparse_mask(length, seed):
    blocks = ref.num_blocks(length)
    rng = np.random.default_rng(seed)
    sel = ref.protected_selection(np.zeros((1, blocks, blocks, Q_HEADS), np.float32), 0.0, 2, 4, 2)
    t = np.arange(blocks).reshape(1, -1, 1, 1)
    j = np.arange(blocks).reshape(1, 1, -1, 1)
    return sel & ~((rng.random(sel.shape) < 0.5) & (j < t) & (j >= 1))


def test_mean_tail_and_merge_d256_vs_oracle(gpu):
    """kernels.py:179-230 (mean_tail) and :312-325 (merge_exact_mean) at d = 256 as
    stand-alone entry points, and the fused layer, on a fixed sparse mask."""
    length = 1089
    q, k, v = _inputs(length, seed=7)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    sel = _sparse_mask(length, seed=3)
    sel_g = torch.from_numpy(sel).cuda()
    idx, cnt = ref.indices_from_mask(sel)
    idx_g, cnt_g = torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda()
    desc = kernels.block_descriptors(kg, vg)
    m_out, m_lse = kernels.mean_tail(qg, desc, sel_g, SCALE)
    e_desc = ref.block_descriptors(to_np(k), to_np(v))
    e_out, e_lse = ref.mean_tail(to_np(q), e_desc, sel, SCALE)
    assert_output_close(to_np(m_out), e_out, what="d256 mean_tail", rel=2.0 ** -7)
    finite = np.isfinite(e_lse)
    assert finite.any() and not finite.all()   # tiles 0 and 1 have no tail
    np.testing.assert_array_equal(np.isfinite(to_np(m_lse)), finite)
    np.testing.assert_allclose(to_np(m_lse)[finite], e_lse[finite], atol=0.02, rtol=0.01)

    x_out, x_lse = up.exact_attention(qg, kg, vg, idx_g, cnt_g, SCALE)
    merged, merged_lse = kernels.merge_exact_mean(x_out, x_lse, m_out, m_lse)
    r_out, r_lse = ref.merge_exact_mean(to_np(x_out), to_np(x_lse), to_np(m_out), to_np(m_lse))
    # the merge rounds to bf16 once: within one bf16 step of the float64 merge
    assert (np.abs(to_np(merged) - r_out) <= 2.0 ** -8 * np.abs(r_out) + 1e-6).all()
    np.testing.assert_allclose(to_np(merged_lse), r_lse, atol=1e-5, rtol=1e-6)

    want, _ = ref.attention_from_selection(to_np(q), to_np(k), to_np(v), SCALE, "mean_native",
                                           sel)
    backend = attention.AttentionBackend(alpha=ALPHA, register=False)
    tiles = up.attention_tiles(kg, vg)
    fused, _ = backend._attention(qg, kg, tiles, idx_g, cnt_g, SCALE, desc)
    assert_output_close(to_np(fused), want, what="d256 fused mean layer", rel=2.0 ** -7)
