"""End-to-end parity of AttentionBackend.forward (every method) against the oracle,
plus the reference's check_math invariants at the backend level and
size-independent properties at the full 32640-token configuration."""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import (SCALE, assert_output_close, inputs, masks_equal_except_ties,
                           threshold_ties, to_np)

pytestmark = pytest.mark.gpu

SIX = ("dense", "fp_v1", "mean_native", "mean_balanced", "cgf_mean", "dispersion_mean")


class DummyAttention:
    layer_idx = 3


def _forward(backend, q, k, v):
    out, none = backend.forward(DummyAttention(), q.transpose(1, 2), k.transpose(1, 2),
                                v.transpose(1, 2), attention_mask=None, scaling=SCALE)
    assert none is None
    return out


@pytest.mark.parametrize("length", (1089, 4096))
@pytest.mark.parametrize("method", SIX)
def test_backend_methods_vs_oracle(gpu, method, length):
    q, k, v = inputs(length, seed=53)
    alpha = 0.08
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    out = _forward(backend, q.cuda(), k.cuda(), v.cuda())
    precision = "f64" if length <= 1089 else "f32"
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, alpha,
                                   precision=precision)
    assert out.shape == (1, length, 28, 128) and out.dtype == torch.bfloat16
    assert_output_close(to_np(out), expected["output"], what=method)


@pytest.mark.parametrize("method", ("fp_v1", "mean_native", "mean_balanced", "cgf_mean",
                                    "dispersion_mean"))
def test_backend_selection_vs_oracle(gpu, method):
    """Masks from the GPU route equal the oracle's, except entries whose score
    lies within 1e-6 of the threshold (listed on failure)."""
    length, alpha = 4096, 0.08
    q, k, v = inputs(length, seed=59, needles=16)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    record = {"events": {}}
    if method in attention.V1_ROUTED_METHODS:
        desc, kbar, scores, idx, cnt, sel = backend._v1_selection(qg, kg, SCALE, record, vg, True)
        positive = False
    else:
        desc, _, idx, cnt, sel = backend._new_selection(qg, kg, vg, SCALE, record)
        scores = kernels.selector_scores(qg, desc, SCALE, method)
        positive = True
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, alpha,
                                   precision="f32")
    ties = threshold_ties(expected["scores"], alpha, positive)
    bad, differ, listed = masks_equal_except_ties(to_np(sel), expected["selected"], ties)
    assert bad == 0, f"{bad} mask entries differ away from the threshold"
    print(f"{method}: {differ} tie entries differ: {listed}")
    # the GPU mask is exactly the selection rule applied to the GPU's own scores
    g_scores = to_np(scores)
    if positive:
        own = ref.protected_selection(g_scores, alpha, 2, 4, 2)
    else:
        own = ref.mask_from_indices(*ref.deal_output_score(g_scores, 2, 4, alpha, 2, 0))
    np.testing.assert_array_equal(to_np(sel), own)
    e_idx, e_cnt = ref.indices_from_mask(to_np(sel))
    np.testing.assert_array_equal(to_np(idx), e_idx)
    np.testing.assert_array_equal(to_np(cnt), e_cnt)


def test_mean_native_and_fp_v1_masks(gpu):
    """check_math.py:313-320."""
    q, k, v = inputs(257, seed=17)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=0.08, register=False)
    record = {"events": {}}
    _, fi, fc, _ = backend._v1_selection(qg, kg, SCALE, record, None)
    _, mi, mc, _ = backend._v1_selection(qg, kg, SCALE, record, vg)
    assert torch.equal(fi, mi) and torch.equal(fc, mc)


def test_fixed_route_future_kv(gpu):
    """check_math.py:322-329: with a fixed route, K/V after position 200 cannot
    change earlier outputs (exact)."""
    q, k, v = inputs(257, seed=17)
    blocks = 3
    sel = ref.protected_selection(np.zeros((1, blocks, blocks, 28), np.float32), 0.0, 2, 4, 2)
    sel[:, 2, 1, ::2] = False
    idx, cnt = ref.indices_from_mask(sel)
    idx_g, cnt_g = torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda()
    backend = attention.AttentionBackend(register=False)

    def combined(kk, vv):
        qg, kg, vg = q.cuda(), kk.cuda(), vv.cuda()
        _, desc, tiles = backend._pool(kg, vg, False, True, True)
        out, _ = backend._attention(qg, kg, tiles, idx_g, cnt_g, SCALE, desc)
        return to_np(out)

    first = combined(k, v)
    k2, v2 = k.clone(), v.clone()
    k2[:, 200:] *= 19
    v2[:, 200:] += 23
    second = combined(k2, v2)
    np.testing.assert_array_equal(second[:, :200], first[:, :200])
    explicit = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    desc = ref.block_descriptors(to_np(k), to_np(v))
    mean = ref.mean_tail(to_np(q), desc, sel, SCALE)
    merged, _ = ref.merge_exact_mean(*explicit, *mean)
    assert_output_close(first, merged)


@pytest.mark.parametrize("impl", ("sdpa", "hip"))
def test_dense_and_decode(gpu, impl):
    length = 1089
    q, k, v = inputs(length, seed=61)
    backend = attention.AttentionBackend(register=False, dense_impl=impl)
    backend.configure("dense")
    out = _forward(backend, q.cuda(), k.cuda(), v.cuda())
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, "dense")
    assert_output_close(to_np(out), expected["output"], what=f"dense-{impl}")
    # decode step (q_len != kv_len) goes to non-causal SDPA for every method
    backend.configure("mean_native", 0.08)
    step, _ = backend.forward(DummyAttention(), q[:, -1:].cuda().transpose(1, 2),
                              k.cuda().transpose(1, 2), v.cuda().transpose(1, 2),
                              attention_mask=None, scaling=SCALE)
    assert step.shape == (1, 1, 28, 128)
    last = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, "dense")["output"][:, -1:]
    assert_output_close(to_np(step), last, what="decode")


def test_profile_rows(gpu):
    q, k, v = inputs(1089, seed=67)
    backend = attention.AttentionBackend(register=False)
    backend.configure("mean_native", 0.08)
    backend.start_profile()
    _forward(backend, q.cuda(), k.cuda(), v.cuda())
    rows = backend.finish_profile()
    assert len(rows) == 1
    row = rows[0]
    for name in attention.STAGE_NAMES:
        assert row[f"{name}_ms"] >= 0.0
    assert row["exact_ms"] > 0 and row["attention_ms"] > 0
    sel = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, "mean_native")["selected"]
    acct = ref.selection_accounting(sel, 1089, 128, 128, "mean_native", 32)
    assert row["exact_token_pairs"] == acct["exact_token_pairs"]
    assert row["selected_block_entries"] == acct["selected_block_entries"]


def test_full_size_properties(gpu):
    """S = 32640 (BASELINE configs 2/3): size-independent properties plus oracle
    parity on a sample of query tiles."""
    length, alpha = 32640, 0.08
    q, k, v = inputs(length, seed=17, needles=64)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure("mean_native", alpha)
    record = {"events": {}}
    desc, kbar, scores, idx, cnt, sel = backend._v1_selection(qg, kg, SCALE, record, vg, True)
    s = to_np(scores)
    rows = s.sum(axis=2)
    assert np.all(np.isclose(rows, 1.0, atol=1e-4) | (rows == 0))
    counts = to_np(cnt)
    blocks = s.shape[1]
    t = np.arange(blocks).reshape(1, -1, 1)
    assert (counts <= t + 1).all() and (counts >= np.minimum(t + 1, 5)).all()
    assert torch.equal(kernels.mask_from_indices(idx, cnt), sel)
    out = _forward(backend, qg, kg, vg)
    o = to_np(out)
    assert np.isfinite(o).all()
    tiles = [0, 1, 60, blocks - 3, blocks - 1]
    e_idx, e_cnt = to_np(idx), counts
    e_desc = ref.block_descriptors(to_np(k), to_np(v), precision="f32")
    m_out, m_lse = ref.mean_tail(to_np(q), e_desc, to_np(sel), SCALE, precision="f32", tiles=tiles)
    rows_sel = np.concatenate([np.arange(ti * 128, min(length, ti * 128 + 128)) for ti in tiles])
    x_out, x_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), e_idx, e_cnt, SCALE,
                                       precision="f32", tiles=tiles)
    merged, _ = ref.merge_exact_mean(x_out, x_lse, m_out, m_lse)
    assert_output_close(o[:, rows_sel], merged[:, rows_sel], what="32640 sampled tiles")
