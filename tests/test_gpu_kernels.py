"""Stage-level parity of the HIP kernels against the CPU oracle (check_math-style).

Each test drives one C-ABI entry point through the reference-named Python
wrapper on the same seeded inputs as the oracle. Bars: bit-exact for selection /
index / mask work; the reference's own check_math tolerances (and the
north-star max-abs 2e-2 / mean-abs 2e-3) for floating point.
"""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels, synthetic
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import (SCALE, assert_output_close, inputs, masks_equal_except_ties,
                           threshold_ties, to_np)

pytestmark = pytest.mark.gpu

LENGTHS = (257, 385, 1089)


def _gpu(*ts):
    return [t.to("cuda") for t in ts]


@pytest.mark.parametrize("length", (257, 1089, 4096))
def test_block_mean_k(gpu, length):
    q, k, v = inputs(length)
    kg, = _gpu(k)
    actual = to_np(up.block_mean_k(kg))
    expected = ref.block_mean_k(to_np(k))
    # bf16 outputs: equal, or one bf16 ulp apart where the fp32 sum order decides rounding
    ulp = np.abs(expected) * 2.0 ** -7 + 1e-30
    diff = np.abs(actual - expected)
    assert (diff <= ulp).all(), float((diff / ulp).max())
    assert (diff == 0).mean() > 0.999
    # check_math.py:292-300 tolerance against the plain fp32 mean
    plain = np.stack([to_np(k)[:, s:s + 128].mean(axis=1) for s in range(0, length, 128)], axis=1)
    np.testing.assert_allclose(actual, plain, atol=0.002, rtol=0.02)


@pytest.mark.parametrize("length", LENGTHS)
def test_block_descriptors(gpu, length):
    q, k, v = inputs(length, seed=3)
    kg, vg = _gpu(k, v)
    d = kernels.block_descriptors(kg, vg)
    e = ref.block_descriptors(to_np(k), to_np(v))
    for name in ("mean_k", "mean_v", "var_k", "sigma_v"):
        np.testing.assert_allclose(to_np(getattr(d, name)), getattr(e, name), atol=2e-6, rtol=2e-5,
                                   err_msg=name)
    np.testing.assert_array_equal(to_np(d.counts), e.counts)


@pytest.mark.parametrize("length", (257, 1089))
def test_attention_tiles_layout(gpu, length):
    """Key tiles hold K rows, value tiles V transposed with the documented key
    permutation; chunk c of row r sits at chunk position c ^ (r & 15); zero past S."""
    q, k, v = inputs(length, seed=5)
    kg, vg = _gpu(k, v)
    kt, vt = (to_np(x) for x in up.attention_tiles(kg, vg))   # [B, Hkv, NB, 128, 128]
    blocks = kt.shape[2]

    def unswizzle(tile):
        out = np.empty_like(tile)
        for r in range(128):
            for c in range(16):
                out[..., r, c * 8:(c + 1) * 8] = tile[..., r, (c ^ (r & 15)) * 8:((c ^ (r & 15)) + 1) * 8]
        return out

    kt, vt = unswizzle(kt), unswizzle(vt)
    kk, vv = to_np(k), to_np(v)
    pad = blocks * 128 - length
    kp = np.concatenate([kk, np.zeros((1, pad) + kk.shape[2:], np.float32)], axis=1)
    vp = np.concatenate([vv, np.zeros((1, pad) + vv.shape[2:], np.float32)], axis=1)
    want_k = kp.reshape(1, blocks, 128, 4, 128).transpose(0, 3, 1, 2, 4)
    np.testing.assert_array_equal(kt, want_k)
    key_of_slot = np.array([(s // 16) * 16 + 4 * ((s % 16) // 8) + (s % 4) + 8 * ((s % 8) // 4)
                            for s in range(128)])
    want_v = vp.reshape(1, blocks, 128, 4, 128)[:, :, key_of_slot].transpose(0, 3, 1, 4, 2)
    np.testing.assert_array_equal(vt, want_v)


@pytest.mark.parametrize("length", (257, 1089, 4096))
def test_v1_scores(gpu, length):
    q, k, v = inputs(length, seed=11)
    qg, kg = _gpu(q, k)
    kbar = up.block_mean_k(kg)
    actual = to_np(up.v1_scores(qg, kbar, SCALE))
    expected = ref.v1_scores(to_np(q), to_np(kbar), SCALE)
    np.testing.assert_allclose(actual, expected, atol=2e-4, rtol=0.005)   # check_math.py:301-303
    rows = actual.sum(axis=2)
    assert np.all(np.isclose(rows, 1.0, atol=1e-5) | np.isclose(rows, 0.0, atol=1e-9))
    upper = np.triu(np.ones((actual.shape[1],) * 2, dtype=bool), k=1)
    assert (actual[:, upper] == 0).all()


@pytest.mark.parametrize("scale", (-SCALE, 0.0))
def test_v1_route_non_positive_scale(gpu, scale):
    """The route kernel's path for a scale that is not positive (every product is
    scaled before the maximum; a positive scale takes the maximum over the raw
    products): V1 scores against the oracle, the fused route's mask equal to the
    selection rule on its own scores, and its lists equal to that mask's. At scale
    0 every valid row has x = 0, so a block's score is its count of valid rows over
    the tile's total (a closed form)."""
    length, alpha = 1089, 0.3
    q, k, v = inputs(length, seed=13)
    qg, kg, vg = _gpu(q, k, v)
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure("fp_v1", alpha)
    record = {"events": {}}
    _, kbar, scores, idx, cnt, sel = backend._v1_selection(qg, kg, scale, record, vg, True)
    g_scores = to_np(scores)
    expected = ref.v1_scores(to_np(q), to_np(kbar), scale)
    np.testing.assert_allclose(g_scores, expected, atol=2e-4, rtol=0.005)
    if scale == 0.0:
        blocks = ref.num_blocks(length)
        rows = np.arange(length)
        valid = rows[:, None] >= (np.arange(blocks)[None, :] + 1) * 128 - 1      # [S, NB]
        per_tile = np.add.reduceat(valid.astype(np.float64), np.arange(0, length, 128), axis=0)
        closed = per_tile / (per_tile.sum(axis=1, keepdims=True) + 1e-9)
        np.testing.assert_allclose(g_scores[0, :, :, 0], closed, atol=1e-6, rtol=1e-5)
    own = ref.mask_from_indices(*ref.deal_output_score(g_scores, 2, 4, alpha, 2, 0))
    np.testing.assert_array_equal(to_np(sel), own)
    e_idx, e_cnt = ref.indices_from_mask(to_np(sel))
    np.testing.assert_array_equal(to_np(idx), e_idx)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)


@pytest.mark.parametrize("sink,window,last,alpha", [(0, 0, 0, 0.3), (1, 6, 3, 0.9), (3, 1, 0, 0.05),
                                                   (0, 2, 1, 1.0), (2, 4, 2, 0.0), (5, 9, 4, 0.5)])
def test_v1_route_protection_parameters(gpu, sink, window, last, alpha):
    """The fused route with the backend's sink / window / last-block settings away
    from the defaults (0 included) and alphas 0 to 1: its mask equals the selection
    rule on its own scores, its lists and counts that mask's, and the scores match
    the oracle's."""
    length = 4096 - 70    # 32 blocks, the last one partial
    q, k, v = inputs(length, seed=17 + sink + 3 * window)
    q = (q.float() * 3).to(torch.bfloat16)
    qg, kg, vg = _gpu(q, k, v)
    backend = attention.AttentionBackend(alpha=alpha, sink_blocks=sink, window_blocks=window,
                                         last_full_blocks=last, register=False)
    backend.configure("fp_v1", alpha)
    record = {"events": {}}
    _, kbar, scores, idx, cnt, sel = backend._v1_selection(qg, kg, SCALE, record, vg, True)
    g_scores = to_np(scores)
    np.testing.assert_allclose(g_scores, ref.v1_scores(to_np(q), to_np(kbar), SCALE),
                               atol=2e-4, rtol=0.005)
    own = ref.mask_from_indices(*ref.deal_output_score(g_scores, sink, window, alpha, last, 0))
    np.testing.assert_array_equal(to_np(sel), own)
    e_idx, e_cnt = ref.indices_from_mask(own)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)
    np.testing.assert_array_equal(to_np(idx), e_idx)


def test_v1_route_head_groups(gpu):
    """The routed form writes each tile's [NB, Hq] index and mask slabs from LDS
    lists, in passes over groups of heads when Hq x NB exceeds its 32768-entry
    list buffer: here 128 q heads x 258 blocks, two passes (127 heads, then 1).
    The fused route's mask equals the selection rule on its own scores, and its
    lists and counts equal that mask's. Inputs are drawn on the GPU (1 GB of Q)."""
    length, q_heads, kv_heads, alpha = 258 * 128 - 100, 128, 8, 0.5
    gen = torch.Generator(device="cuda").manual_seed(29)
    q = (torch.randn(1, length, q_heads, 128, generator=gen, device="cuda") * 4).to(torch.bfloat16)
    k = torch.randn(1, length, kv_heads, 128, generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn(1, length, kv_heads, 128, generator=gen, device="cuda").to(torch.bfloat16)
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure("fp_v1", alpha)
    record = {"events": {}}
    _, _, scores, idx, cnt, sel = backend._v1_selection(q, k, SCALE, record, v, True)
    del q, k, v
    g_scores = to_np(scores)
    assert g_scores.shape == (1, 258, 258, q_heads)
    own = ref.mask_from_indices(*ref.deal_output_score(g_scores, 2, 4, alpha, 2, 0))
    np.testing.assert_array_equal(to_np(sel), own)
    e_idx, e_cnt = ref.indices_from_mask(own)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)
    np.testing.assert_array_equal(to_np(idx), e_idx)


def test_v1_route_eight_chunk_rows(gpu):
    """Rows of 257-512 key blocks take the select kernel's 8-chunk form (40000
    tokens: 313 blocks). V1 scores against the oracle on a sample of tiles, the
    fused mask equal to the selection rule on the kernel's own scores, and the
    lists and counts equal to that mask's."""
    length, q_heads, kv_heads, alpha = 40000, 8, 2, 0.3
    gen = torch.Generator(device="cuda").manual_seed(31)
    q = (torch.randn(1, length, q_heads, 128, generator=gen, device="cuda") * 2).to(torch.bfloat16)
    k = torch.randn(1, length, kv_heads, 128, generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn(1, length, kv_heads, 128, generator=gen, device="cuda").to(torch.bfloat16)
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure("fp_v1", alpha)
    record = {"events": {}}
    _, kbar, scores, idx, cnt, sel = backend._v1_selection(q, k, SCALE, record, v, True)
    g_scores = to_np(scores)
    assert g_scores.shape == (1, 313, 313, q_heads)
    tiles = [0, 1, 150, 255, 312]
    qn, kn = to_np(q), to_np(kbar)
    expected = ref.v1_scores(qn, kn, SCALE)
    np.testing.assert_allclose(g_scores[:, tiles], expected[:, tiles], atol=2e-4, rtol=0.005)
    own = ref.mask_from_indices(*ref.deal_output_score(g_scores, 2, 4, alpha, 2, 0))
    np.testing.assert_array_equal(to_np(sel), own)
    e_idx, e_cnt = ref.indices_from_mask(own)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)
    np.testing.assert_array_equal(to_np(idx), e_idx)


def _adversarial_scores(length, seed):
    """Score tensors that stress the threshold: raised-to-the-4th V1 scores
    (check_math.py:305-311), exact ties with the threshold, zero rows."""
    q, k, v = inputs(length, seed=seed)
    kbar = ref.block_mean_k(to_np(k))
    s = ref.v1_scores(to_np(q), kbar, SCALE)
    s4 = (s * s) * (s * s)
    tied = s.copy()
    tied[:, :, 0, :] = 1.0
    tied[:, :, 1, :] = np.float32(np.float32(1.0) * np.float32(0.08))   # exactly at threshold
    tied[:, :, 2, :] = np.nextafter(tied[:, :, 1, :], np.float32(0))     # one ulp below
    zero = np.zeros_like(s)
    return [(s4.astype(np.float32), 0.8), (s, 0.08), (tied.astype(np.float32), 0.08),
            (zero, 0.08), (s, 0.0)]


@pytest.mark.parametrize("length", (385, 1089))
def test_deal_output_score_bit_exact(gpu, length):
    for scores, alpha in _adversarial_scores(length, seed=23):
        sg = torch.from_numpy(scores).cuda()
        for sink, window, last in ((2, 4, 2), (1, 1, 0), (0, 0, 3)):
            idx, cnt = up.deal_output_score(sg, sink, window, alpha, last, 0)
            e_idx, e_cnt = ref.deal_output_score(scores, sink, window, alpha, last, 0)
            np.testing.assert_array_equal(to_np(idx), e_idx)
            np.testing.assert_array_equal(to_np(cnt), e_cnt)


def test_deal_output_score_min_budget(gpu):
    scores, _ = _adversarial_scores(1089, seed=29)[0]
    sg = torch.from_numpy(scores).cuda()
    idx, cnt = up.deal_output_score(sg, 2, 4, 0.9, 2, 3)
    e_idx, e_cnt = ref.deal_output_score(scores, 2, 4, 0.9, 2, 3)
    np.testing.assert_array_equal(to_np(idx), e_idx)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)


@pytest.mark.parametrize("length", (385, 1089))
def test_protected_selection_bit_exact(gpu, length):
    for scores, alpha in _adversarial_scores(length, seed=31):
        sg = torch.from_numpy(scores).cuda()
        mask = kernels.protected_selection(sg, alpha, 2, 4, 2)
        expected = ref.protected_selection(scores, alpha, 2, 4, 2)
        np.testing.assert_array_equal(to_np(mask), expected)
        idx, cnt = kernels.indices_from_mask(mask)
        e_idx, e_cnt = ref.indices_from_mask(expected)
        np.testing.assert_array_equal(to_np(idx), e_idx)
        np.testing.assert_array_equal(to_np(cnt), e_cnt)
        back = kernels.mask_from_indices(idx, cnt)
        np.testing.assert_array_equal(to_np(back), expected)


@pytest.mark.parametrize("batch,blocks,heads", [
    (1, 100, 4),     # 2 chunks of 64 key blocks per row
    (1, 200, 4),     # 4 chunks
    (2, 313, 8),     # 8 chunks, batch 2
    (1, 700, 4),     # 16 chunks
    (1, 1024, 3),    # 16 chunks at the block limit
    (1, 600, 64),    # 64 heads x 600 blocks > 32768 list entries: two head groups
])
def test_selection_row_kernel_forms_bit_exact(gpu, batch, blocks, heads):
    """Score rows take the per-tile selection kernel in its 1-16-chunk forms (64 key
    blocks per chunk) and, beyond 32768 list entries per tile, in several head
    groups: the protected selection (alpha 0 and 0.3) and the V1 threshold lists
    equal the oracle's bit for bit, with zero rows and exact threshold ties
    planted."""
    rng = np.random.default_rng(37 + blocks)
    scores = rng.random((batch, blocks, blocks, heads), dtype=np.float32) ** 4
    scores[:, 5] = 0.0                                     # a zero row
    scores[:, :, 3, :] = 1.0                               # the max
    scores[:, :, 4, :] = np.float32(np.float32(1.0) * np.float32(0.3))   # exactly at 0.3 x max
    scores[:, :, blocks - 2, :] = np.float32(0.3) * np.float32(1.0)      # a tie at the far end
    sg = torch.from_numpy(scores).cuda()
    for alpha in (0.0, 0.3):
        # the backend's form: mask, indices and counts from one launch
        indices = torch.empty(scores.shape, dtype=torch.int64, device="cuda")
        counts = torch.empty(scores.shape[:2] + scores.shape[3:], dtype=torch.int32, device="cuda")
        mask = kernels.protected_selection(sg, alpha, 2, 4, 2, indices, counts)
        expected = ref.protected_selection(scores, alpha, 2, 4, 2)
        np.testing.assert_array_equal(to_np(mask), expected)
        e_idx, e_cnt = ref.indices_from_mask(expected)
        np.testing.assert_array_equal(to_np(counts), e_cnt)
        np.testing.assert_array_equal(to_np(indices), e_idx)
    idx, cnt = up.deal_output_score(sg, 2, 4, 0.3, 2, 0)
    e_idx, e_cnt = ref.deal_output_score(scores, 2, 4, 0.3, 2, 0)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)
    np.testing.assert_array_equal(to_np(idx), e_idx)
    mask = kernels.mask_from_indices(idx, cnt)
    np.testing.assert_array_equal(to_np(mask), ref.mask_from_indices(e_idx, e_cnt))


@pytest.mark.parametrize("length", (257, 1089, 4500))   # 4500: 36 blocks, two 32-block chunks
@pytest.mark.parametrize("selector", ("mean_balanced", "cgf_mean", "dispersion_mean"))
def test_selector_scores(gpu, length, selector):
    q, k, v = inputs(length, seed=41)
    qg, kg, vg = _gpu(q, k, v)
    desc = kernels.block_descriptors(kg, vg)
    actual = to_np(kernels.selector_scores(qg, desc, SCALE, selector))
    e_desc = ref.BlockDescriptors(*(to_np(getattr(desc, n)) for n in
                                    ("mean_k", "mean_v", "var_k", "sigma_v", "counts")))
    expected = ref.selector_scores(to_np(q), e_desc, SCALE, selector)
    np.testing.assert_allclose(actual, expected, atol=2e-5, rtol=2e-5)   # check_math.py:287-290


# (batch, q heads, kv heads, head dim, length): the selector kernels deal whole tiles to
# XCDs, and the long-row / d=256 kernel one (batch, kv group) stream per XCD pair when
# the streams divide 8, else whole tiles. 40000 tokens (313 blocks) takes d=128 to the
# long-row kernel; layouts with 3, 6 and 9 streams take the whole-tile deal there.
# 32768 tokens (256 blocks) is the longest row of the short-row kernels (8 chunks, the
# last tile's last chunk 31 blocks), 32769 (257 blocks) the shortest of the long-row kernel.
SELECTOR_LAYOUTS = [(1, 6, 3, 128, 40000), (3, 4, 2, 128, 1089), (1, 6, 3, 256, 1089),
                    (3, 6, 3, 256, 600), (2, 8, 2, 128, 40000), (1, 4, 2, 128, 32768),
                    (1, 4, 2, 128, 32769)]


@pytest.mark.parametrize("batch,q_heads,kv_heads,head_dim,length", SELECTOR_LAYOUTS)
@pytest.mark.parametrize("selector", ("mean_balanced", "cgf_mean", "dispersion_mean"))
def test_selector_scores_layouts(gpu, selector, batch, q_heads, kv_heads, head_dim, length):
    q, k, v, _ = synthetic.make_inputs(length, seed=29, q_heads=q_heads, kv_heads=kv_heads,
                                       head_dim=head_dim, batch=batch)
    qg, kg, vg = _gpu(q, k, v)
    desc = kernels.block_descriptors(kg, vg)
    scale = head_dim ** -0.5
    actual = to_np(kernels.selector_scores(qg, desc, scale, selector))
    e_desc = ref.BlockDescriptors(*(to_np(getattr(desc, n)) for n in
                                    ("mean_k", "mean_v", "var_k", "sigma_v", "counts")))
    blocks = ref.num_blocks(length)
    # long sequences: the oracle scores sampled tiles (first, middle, the last two)
    tiles = None if blocks <= 40 else [1, blocks // 2, blocks - 2, blocks - 1]
    expected = ref.selector_scores(to_np(q), e_desc, scale, selector, tiles=tiles)
    if tiles is not None:
        actual, expected = actual[:, tiles], expected[:, tiles]
    np.testing.assert_allclose(actual, expected, atol=2e-5, rtol=2e-5)   # check_math.py:287-290


@pytest.mark.parametrize("selector", ("mean_balanced", "cgf_mean", "dispersion_mean"))
def test_selector_scores_full_size_repeatable(gpu, selector):
    """S=32640 (255 tiles, 8 chunks of 32 blocks): every call gives the same bits,
    also after short sequences that leave other values in LDS, and for the two
    softmax-mean selectors every tile's scores over j < t sum to 1 (mean of softmax
    rows). A cross-wave LDS race once left one tile's first chunk with another
    workgroup's partial sums (row sum 1.22)."""
    q, k, v, _ = synthetic.make_inputs(32640, seed=23, device="cuda")
    desc = kernels.block_descriptors(k, v)
    qs, ks, vs, _ = synthetic.make_inputs(1089, seed=5, device="cuda")
    small = kernels.block_descriptors(ks, vs)
    runs = []
    for _ in range(4):
        kernels.selector_scores(qs, small, SCALE, selector)
        runs.append(kernels.selector_scores(q, desc, SCALE, selector))
    first = runs[0].cpu()
    for r in runs[1:]:
        assert torch.equal(r.cpu(), first)
    s = first[0].double().numpy()                    # [t, j, h]
    blocks = s.shape[0]
    assert np.all(s[np.triu_indices(blocks)[0], np.triu_indices(blocks)[1]] == 0)   # j >= t
    if selector != "dispersion_mean":
        np.testing.assert_allclose(s[1:].sum(axis=1), 1.0, atol=1e-5)


def _fixed_selection(length, seed, drop=0.3):
    """All-causal selection with a random share of full-history blocks removed
    (protected blocks kept), as in check_math.py:245-250."""
    blocks = ref.num_blocks(length)
    rng = np.random.default_rng(seed)
    sel = ref.protected_selection(np.zeros((1, blocks, blocks, 28), np.float32), 0.0, 2, 4, 2)
    drop_mask = rng.random(sel.shape) < drop
    t = np.arange(blocks).reshape(1, -1, 1, 1)
    j = np.arange(blocks).reshape(1, 1, -1, 1)
    droppable = (j < t) & (j >= 1)
    sel = sel & ~(drop_mask & droppable)
    return sel


@pytest.mark.parametrize("length", (257, 1089))
def test_exact_attention_all_selected_vs_dense(gpu, length):
    q, k, v = inputs(length, seed=17)
    qg, kg, vg = _gpu(q, k, v)
    blocks = ref.num_blocks(length)
    sel = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[None, :, :, None],
                          (1, blocks, blocks, 28))
    idx, cnt = ref.indices_from_mask(sel)
    out, lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    d_out, d_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    assert_output_close(to_np(out), d_out)
    np.testing.assert_allclose(to_np(lse), d_lse, atol=0.02, rtol=0.01)   # check_math.py:243


@pytest.mark.parametrize("length", (385, 1089, 4096))
def test_exact_attention_fixed_mask(gpu, length):
    q, k, v = inputs(length, seed=19)
    qg, kg, vg = _gpu(q, k, v)
    sel = _fixed_selection(length, seed=7)
    idx, cnt = ref.indices_from_mask(sel)
    out, lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    assert_output_close(to_np(out), e_out)
    np.testing.assert_allclose(to_np(lse), e_lse, atol=0.02, rtol=0.01)


def test_exact_attention_edge_lists(gpu):
    """Empty list -> output 0 / LSE -inf; a list holding only a future block and
    an out-of-range id follows the kernel's documented semantics."""
    length = 385
    q, k, v = inputs(length, seed=2)
    qg, kg, vg = _gpu(q, k, v)
    blocks = ref.num_blocks(length)
    idx = np.full((1, blocks, blocks, 28), blocks, np.int64)
    cnt = np.zeros((1, blocks, 28), np.int32)
    idx[0, 1, 0, 3] = 2      # future block for tile 1, head 3
    cnt[0, 1, 3] = 1
    idx[0, 2, 0, 5] = 2      # diagonal + an out-of-range id
    idx[0, 2, 1, 5] = 99
    cnt[0, 2, 5] = 2
    # ids whose low 32 bits are in range are still out of range (no narrowing)
    idx[0, 2, :3, 7] = [(1 << 32) + 1, 2, -(1 << 32) + 1]
    cnt[0, 2, 7] = 3
    out, lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    a_out, a_lse = to_np(out), to_np(lse)
    assert_output_close(a_out, e_out)
    finite = np.isfinite(e_lse)
    np.testing.assert_array_equal(np.isfinite(a_lse), finite)
    np.testing.assert_allclose(a_lse[finite], e_lse[finite], atol=0.02, rtol=0.01)
    assert (a_out[~finite] == 0).all()


def test_exact_attention_repeated_list_entries(gpu):
    """A block listed twice is attended twice, as the reference's list walk does
    (upstream:305-340) and the oracle restates: its keys enter the softmax with
    double weight. Lists hold at most NB entries, so repeats go into slots freed by
    dropped blocks: repeats in the full-block path, on the diagonal, one tile of a
    pair repeating a block the other lists once, a block listed three times, and a
    list of one block listed twice."""
    length = 1089
    q, k, v = inputs(length, seed=4)
    qg, kg, vg = _gpu(q, k, v)
    blocks = ref.num_blocks(length)           # 9
    sel = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[None, :, :, None],
                          (1, blocks, blocks, 28)).copy()
    sel[0, 8, [4, 6], 0] = False              # tile 8, head 0: room for 2 repeats
    sel[0, 8, [4, 6], 2] = False
    sel[0, 7, 5, 1] = False                   # tile 7, head 1: room for 2
    idx, cnt = ref.indices_from_mask(sel)

    def append(t, h, *ids):
        for j in ids:
            assert cnt[0, t, h] < blocks
            idx[0, t, cnt[0, t, h], h] = j
            cnt[0, t, h] += 1

    append(8, 0, 3, 3)        # tile 8 lists block 3 three times; tile 7 lists it once
    append(7, 1, 0, 0)        # tile 7: block 0 three times
    append(8, 2, 8, 1)        # the diagonal block twice, block 1 twice
    append(5, 4, 2, 4, 5)     # repeats of history and window blocks, and the diagonal
    idx[0, 3, :, 6] = blocks  # tile 3, head 6: only block 1, listed twice
    idx[0, 3, :2, 6] = 1
    cnt[0, 3, 6] = 2
    out, lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    assert_output_close(to_np(out), e_out, what="repeated entries")
    np.testing.assert_allclose(to_np(lse), e_lse, atol=0.02, rtol=0.01)
    # the repeats matter: the same lists without them give a visibly different answer
    plain_idx, plain_cnt = ref.indices_from_mask(ref.mask_from_indices(idx, cnt))
    p_out, p_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), plain_idx, plain_cnt,
                                       SCALE)
    for t, h in ((8, 0), (7, 1), (8, 2), (5, 4)):
        rows = slice(t * 128, (t + 1) * 128)
        assert np.abs(p_out[0, rows, h] - e_out[0, rows, h]).max() > 0.02, (t, h)
    # one block listed twice: the same softmax, every weight doubled -> LSE + ln 2
    rows = slice(3 * 128, 4 * 128)
    np.testing.assert_allclose(to_np(lse)[0, rows, 6] - p_lse[0, rows, 6], np.log(2.0),
                               atol=0.02)


@pytest.mark.parametrize("length", (257, 1089))
def test_mean_tail_and_merge(gpu, length):
    q, k, v = inputs(length, seed=37)
    qg, kg, vg = _gpu(q, k, v)
    sel = _fixed_selection(length, seed=9, drop=0.5)
    desc = kernels.block_descriptors(kg, vg)
    e_desc = ref.block_descriptors(to_np(k), to_np(v))
    sg = torch.from_numpy(sel).cuda()
    m_out, m_lse = kernels.mean_tail(qg, desc, sg, SCALE)
    e_out, e_lse = ref.mean_tail(to_np(q), e_desc, sel, SCALE)
    np.testing.assert_allclose(to_np(m_out), e_out, atol=2e-3, rtol=2e-2)
    finite = np.isfinite(e_lse)
    np.testing.assert_array_equal(np.isfinite(to_np(m_lse)), finite)
    np.testing.assert_allclose(to_np(m_lse)[finite], e_lse[finite], atol=2e-3, rtol=1e-3)
    idx, cnt = ref.indices_from_mask(sel)
    x_out, x_lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                      torch.from_numpy(cnt).cuda(), SCALE)
    merged, total = kernels.merge_exact_mean(x_out, x_lse, m_out, m_lse)
    r_out, r_total = ref.merge_exact_mean(to_np(x_out), to_np(x_lse), to_np(m_out), to_np(m_lse))
    assert_output_close(to_np(merged), r_out, max_abs=8e-3, mean_abs=1e-4, what="merge")
    np.testing.assert_allclose(to_np(total), r_total, atol=1e-5, rtol=1e-5)


def test_selection_accounting(gpu):
    sel = _fixed_selection(1089, seed=4)
    acct = kernels.selection_accounting(torch.from_numpy(sel).cuda(), 1089, 128, 128,
                                        "mean_native", 32)
    expected = ref.selection_accounting(sel, 1089, 128, 128, "mean_native", 32)
    for key, value in expected.items():
        got = acct[key]
        got = got.item() if isinstance(got, torch.Tensor) else got
        if isinstance(value, float):
            assert got == pytest.approx(value, rel=1e-12), key
        else:
            assert got == value, key


def _selection_params(n=12, seed=31):
    """Deterministic random selection parameters: sink, window and last-full block
    counts (0 included), alpha (0 included), the top-k budget of deal_output_score,
    the score layout."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        out.append((int(rng.integers(1, 3)), int(rng.choice((9, 37, 64, 65, 130))),
                    int(rng.integers(1, 6)), int(rng.integers(0, 4)), int(rng.integers(0, 7)),
                    int(rng.integers(0, 4)), float(rng.choice((0.0, 0.05, 0.3, 0.9, 1.0))),
                    int(rng.choice((0, 0, 3, 10))), 500 + i))
    return out


@pytest.mark.parametrize("batch,blocks,heads,sink,window,last,alpha,budget,seed",
                         _selection_params())
def test_selection_random_parameters_bit_exact(gpu, batch, blocks, heads, sink, window, last,
                                               alpha, budget, seed):
    """protected_selection (mask, indices, counts) and deal_output_score (its top-k
    budget included) over random sink / window / last-block counts, alphas and score
    layouts, with zero rows, repeated maxima and exact threshold ties planted: bit for
    bit against the oracle (kernels.py:129-160, upstream:357-407)."""
    rng = np.random.default_rng(seed)
    scores = rng.random((batch, blocks, blocks, heads), dtype=np.float32) ** 3
    scores[:, min(4, blocks - 1)] = 0.0                          # a zero row
    scores[:, :, 0, :] = scores.max()                            # repeated maxima
    tie = rng.integers(0, blocks, size=3)
    scores[:, :, tie, :] = np.float32(alpha) * scores.max()      # threshold ties
    sg = torch.from_numpy(scores).cuda()
    indices = torch.empty(scores.shape, dtype=torch.int64, device="cuda")
    counts = torch.empty(scores.shape[:2] + scores.shape[3:], dtype=torch.int32, device="cuda")
    mask = kernels.protected_selection(sg, alpha, sink, window, last, indices, counts)
    expected = ref.protected_selection(scores, alpha, sink, window, last)
    np.testing.assert_array_equal(to_np(mask), expected)
    e_idx, e_cnt = ref.indices_from_mask(expected)
    np.testing.assert_array_equal(to_np(counts), e_cnt)
    np.testing.assert_array_equal(to_np(indices), e_idx)
    idx, cnt = up.deal_output_score(sg, sink, window, alpha, last, budget)
    e_idx, e_cnt = ref.deal_output_score(scores, sink, window, alpha, last, budget)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)
    np.testing.assert_array_equal(to_np(idx), e_idx)


def _random_lists(blocks, seed, heads=28):
    """For every (tile, head) a random subset of the causal blocks 0..t in random
    order, some entries repeated, a random count (empty rows included), and garbage
    (out-of-range and negative ids) past the count."""
    rng = np.random.default_rng(seed)
    idx = rng.integers(-3 * blocks, 3 * blocks, size=(1, blocks, blocks, heads)).astype(np.int64)
    cnt = np.zeros((1, blocks, heads), np.int32)
    for t in range(blocks):
        for h in range(heads):
            keep = rng.permutation(t + 1)[: rng.integers(0, t + 2)]
            extra = rng.choice(keep, size=min(len(keep), blocks - len(keep), rng.integers(0, 3)),
                               replace=False) if len(keep) else np.array([], np.int64)
            row = rng.permutation(np.concatenate([keep, extra]).astype(np.int64))
            assert len(row) <= blocks
            idx[0, t, : len(row), h] = row
            cnt[0, t, h] = len(row)
    return idx, cnt


@pytest.mark.parametrize("length,seed", [(1089, 101), (4096, 103)])
def test_exact_attention_random_unsorted_lists(gpu, length, seed):
    """Seeded random lists (``_random_lists``), which must be walked as given: the
    kernel merges each tile pair's lists into one ascending walk and ignores the
    entries past each count; the result must match the oracle's walk of the lists."""
    q, k, v = inputs(length, seed=seed)
    qg, kg, vg = _gpu(q, k, v)
    idx, cnt = _random_lists(ref.num_blocks(length), seed)
    out, lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    a_out, a_lse = to_np(out), to_np(lse)
    assert_output_close(a_out, e_out, what="random unsorted lists")
    finite = np.isfinite(e_lse)
    np.testing.assert_array_equal(np.isfinite(a_lse), finite)
    np.testing.assert_allclose(a_lse[finite], e_lse[finite], atol=0.02, rtol=0.01)
    assert (a_out[~finite] == 0).all()


@pytest.mark.parametrize("length,seed", [(1089, 107), (4096, 109)])
def test_sparse_attention_mean_random_lists(gpu, length, seed):
    """The fused mean-method launch (exact blocks + block-mean tail in one softmax)
    on the same kind of random lists: the tail is every causal block j < t the row
    does not list, whatever the order and repeats of the listed ones; against the
    oracle's exact part, mean tail and logaddexp merge (kernels.py:179-230, 312-325)."""
    q, k, v = inputs(length, seed=seed)
    qg, kg, vg = _gpu(q, k, v)
    idx, cnt = _random_lists(ref.num_blocks(length), seed)
    backend = attention.AttentionBackend(register=False)
    _, desc, tiles = backend._pool(kg, vg, False, True, True)
    out, lse = backend._attention(qg, kg, tiles, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE, desc)
    e_desc = ref.BlockDescriptors(*(to_np(getattr(desc, n)) for n in
                                    ("mean_k", "mean_v", "var_k", "sigma_v", "counts")))
    x_out, x_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    m_out, m_lse = ref.mean_tail(to_np(q), e_desc, ref.mask_from_indices(idx, cnt), SCALE)
    e_out, e_lse = ref.merge_exact_mean(x_out, x_lse, m_out, m_lse)
    # rows with no key at all (tile 0 with an empty list: no listed block, no tail)
    # have LSE -inf; the oracle's merge gives NaN there, the kernel its empty-row 0
    finite = np.isfinite(e_lse)
    a_out, a_lse = to_np(out), to_np(lse)
    assert_output_close(a_out[finite], e_out[finite], what="fused mean, random lists")
    assert (a_out[~finite] == 0).all()
    np.testing.assert_array_equal(np.isfinite(a_lse), finite)
    np.testing.assert_allclose(a_lse[finite], e_lse[finite], atol=0.02, rtol=0.01)


@pytest.mark.parametrize("remainder", (False, True))
def test_sparse_attention_rescue_random_lists(gpu, remainder):
    """The fused rescue launch (exact blocks + one rescue token, and with remainder
    the block's other tokens' mean, per unlisted causal block) on random unsorted
    lists with repeats: against the oracle's exact part, rescue tail (the GPU's token
    choice) and logaddexp merge (kernels.py:233-325)."""
    length, seed = 1089, 113
    q, k, v = inputs(length, seed=seed)
    qg, kg, vg = _gpu(q, k, v)
    idx, cnt = _random_lists(ref.num_blocks(length), seed)
    backend = attention.AttentionBackend(register=False)
    _, desc, tiles = backend._pool(kg, vg, False, remainder, True)
    choice = kernels.rescue_choice(qg, tiles[0])
    out, lse = backend._attention(qg, kg, tiles, torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE, None,
                                  rescue=(choice, remainder, desc, vg))
    x_out, x_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    r_out, r_lse = ref.rescue_tail(to_np(q), to_np(k), to_np(v), ref.mask_from_indices(idx, cnt),
                                   SCALE, remainder=remainder, choice=to_np(choice))
    e_out, e_lse = ref.merge_exact_mean(x_out, x_lse, r_out, r_lse)
    finite = np.isfinite(e_lse)   # -inf: tile 0 with an empty list (no key at all)
    a_out, a_lse = to_np(out), to_np(lse)
    assert_output_close(a_out[finite], e_out[finite], what="fused rescue, random lists")
    assert (a_out[~finite] == 0).all()
    np.testing.assert_array_equal(np.isfinite(a_lse), finite)
    np.testing.assert_allclose(a_lse[finite], e_lse[finite], atol=0.02, rtol=0.01)
