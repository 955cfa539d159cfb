"""Batch > 1 on the GPU: every kernel indexes by batch, so each entry point and
every method runs with two independent sequences in one call and is compared
with the oracle on the same two sequences."""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels, synthetic
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import (SCALE, assert_output_close, masks_equal_except_ties, threshold_ties,
                           to_np)

pytestmark = pytest.mark.gpu

LENGTH = 385   # three blocks, the last one partial


def batch_inputs(length=LENGTH, seed=53, **kw):
    q, k, v, _ = synthetic.make_inputs(length, seed=seed, batch=2, **kw)
    return q, k, v


class _Layer:
    layer_idx = 0


def test_pool_and_route_kernels_batch2(gpu):
    q, k, v = batch_inputs()
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    kbar = up.block_mean_k(kg)
    e_kbar = ref.block_mean_k(to_np(k))
    assert (np.abs(to_np(kbar) - e_kbar) <= np.abs(e_kbar) * 2.0 ** -7 + 1e-30).all()
    d = kernels.block_descriptors(kg, vg)
    e = ref.block_descriptors(to_np(k), to_np(v))
    for name in ("mean_k", "mean_v", "var_k", "sigma_v"):
        np.testing.assert_allclose(to_np(getattr(d, name)), getattr(e, name), atol=2e-6, rtol=2e-5,
                                   err_msg=name)
    scores = up.v1_scores(qg, kbar, SCALE)
    np.testing.assert_allclose(to_np(scores), ref.v1_scores(to_np(q), to_np(kbar), SCALE),
                               atol=2e-4, rtol=0.005)
    e_desc = ref.BlockDescriptors(*(to_np(getattr(d, n)) for n in
                                    ("mean_k", "mean_v", "var_k", "sigma_v", "counts")))
    for selector in ("mean_balanced", "cgf_mean", "dispersion_mean"):
        np.testing.assert_allclose(to_np(kernels.selector_scores(qg, d, SCALE, selector)),
                                   ref.selector_scores(to_np(q), e_desc, SCALE, selector),
                                   atol=2e-5, rtol=2e-5, err_msg=selector)
    tiles, _ = up.attention_tiles(kg, vg)
    choice = to_np(kernels.rescue_choice(qg, tiles))
    want = ref.rescue_choice(to_np(q), to_np(k))
    assert (choice != want).mean() < 1e-3   # fp32 near-ties only


def test_exact_attention_batch2(gpu):
    q, k, v = batch_inputs(seed=59)
    blocks = ref.num_blocks(LENGTH)
    rng = np.random.default_rng(7)
    sel = ref.protected_selection(np.zeros((2, blocks, blocks, 28), np.float32), 0.0, 1, 1, 0)
    sel = sel & ~((rng.random(sel.shape) < 0.5) & (np.arange(blocks)[None, None, :, None]
                                                    < np.arange(blocks)[None, :, None, None]))
    sel[:, :, 0] = True   # keep at least block 0 so every row has keys
    idx, cnt = ref.indices_from_mask(sel)
    out, lse = up.exact_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), SCALE)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, SCALE)
    assert_output_close(to_np(out), e_out, what="batch-2 exact")
    np.testing.assert_allclose(to_np(lse), e_lse, atol=0.02, rtol=0.01)


@pytest.mark.parametrize("method", attention.METHODS)
def test_backend_every_method_batch2(gpu, method):
    q, k, v = batch_inputs(seed=61)
    alpha = 0.08
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    out, _ = backend.forward(_Layer(), q.cuda().transpose(1, 2), k.cuda().transpose(1, 2),
                             v.cuda().transpose(1, 2), None, SCALE)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, alpha)
    if expected["scores"] is not None and method in attention.V1_ROUTED_METHODS:
        record = {"events": {}}
        _, _, _, _, _, _, sel = backend._route_v1(q.cuda(), k.cuda(), v.cuda(), SCALE, record,
                                                  False, False)
        unexplained, _, _ = masks_equal_except_ties(to_np(sel), expected["selected"],
                                                     threshold_ties(expected["scores"], alpha))
        assert unexplained == 0
    assert out.shape == (2, LENGTH, 28, 128)
    assert_output_close(to_np(out), expected["output"], what=method)


def test_d256_batch2(gpu):
    q, k, v = batch_inputs(seed=67, q_heads=16, kv_heads=4, head_dim=256)
    scale = 256 ** -0.5
    backend = attention.AttentionBackend(alpha=0.08, register=False)
    backend.configure("fp_v1", 0.08)
    out, _ = backend.forward(_Layer(), q.cuda().transpose(1, 2), k.cuda().transpose(1, 2),
                             v.cuda().transpose(1, 2), None, scale)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), scale, "fp_v1", 0.08)
    assert_output_close(to_np(out), expected["output"], what="batch-2 d256 fp_v1")


@pytest.mark.parametrize("method", ("mean_native", "fp_v1_rescue_v2"))
def test_tails_batch2(gpu, method):
    """Two sequences with sparse V1 selections (Q, K scaled by 8, alpha 0.5: density
    ~0.77), so the block-mean and rescue tails of both batch elements are exercised."""
    q, k, v = batch_inputs(2048, seed=71)
    q = (q.float() * 8).to(torch.bfloat16)
    k = (k.float() * 8).to(torch.bfloat16)
    alpha = 0.5
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    out, _ = backend.forward(_Layer(), qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2),
                             None, SCALE)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, alpha,
                                   precision="f32")
    blocks = ref.num_blocks(2048)
    causal = 2 * 28 * blocks * (blocks + 1) // 2
    assert expected["selected"].sum() < 0.9 * causal          # tails are not empty
    record = {"events": {}}
    _, _, _, _, _, _, sel = backend._route_v1(qg, kg, vg, SCALE, record, False, False)
    unexplained, differ, _ = masks_equal_except_ties(to_np(sel), expected["selected"],
                                                     threshold_ties(expected["scores"], alpha))
    assert unexplained == 0
    # the output is always compared: against the oracle layer given the GPU's own
    # selection, so a mask entry that differs at a threshold tie cannot skip it
    want, _ = ref.attention_from_selection(to_np(q), to_np(k), to_np(v), SCALE, method,
                                           to_np(sel), precision="f32")
    # peaked attention: outputs beyond unit scale, one bf16 step relative on top
    assert_output_close(to_np(out), want, what=method, rel=2.0 ** -7)
    if differ == 0:
        np.testing.assert_array_equal(want, expected["output"])


@pytest.mark.parametrize("length", (1, 100, 128, 129, 256))
@pytest.mark.parametrize("method", attention.METHODS)
def test_short_and_boundary_lengths(gpu, method, length):
    """One token, a partial single block, exact block multiples and one token past
    a block: every method against the oracle layer."""
    q, k, v, _ = synthetic.make_inputs(length, seed=73)
    backend = attention.AttentionBackend(alpha=0.08, register=False)
    backend.configure(method, 0.08)
    out, _ = backend.forward(_Layer(), q.cuda().transpose(1, 2), k.cuda().transpose(1, 2),
                             v.cuda().transpose(1, 2), None, SCALE)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, 0.08)
    assert out.shape == (1, length, 28, 128)
    assert_output_close(to_np(out), expected["output"], what=f"{method} S={length}")


@pytest.mark.parametrize("length", (1, 100))
def test_short_lengths_d256(gpu, length):
    q, k, v, _ = synthetic.make_inputs(length, seed=79, q_heads=16, kv_heads=4, head_dim=256)
    scale = 256 ** -0.5
    for method, impl in (("fp_v1", "sdpa"), ("dense", "hip")):
        backend = attention.AttentionBackend(alpha=0.08, register=False, dense_impl=impl)
        backend.configure(method, 0.08)
        out, _ = backend.forward(_Layer(), q.cuda().transpose(1, 2), k.cuda().transpose(1, 2),
                                 v.cuda().transpose(1, 2), None, scale)
        expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), scale, method, 0.08)
        assert_output_close(to_np(out), expected["output"], what=f"d256 {method} S={length}")
