"""GPU parity of the rescue path (fp_v1_rescue / fp_v1_rescue_v2; kernels.py:233-309,
attention.py:306-331) against the CPU oracle."""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import SCALE, assert_output_close, inputs, to_np
from tests.test_gpu_kernels import _fixed_selection
from tests.test_oracle_pins import explicit_rescue_reference

pytestmark = pytest.mark.gpu


def _choice(qg, kg, vg):
    key_tiles, _ = up.attention_tiles(kg, vg)
    return to_np(kernels.rescue_choice(qg, key_tiles))


@pytest.mark.parametrize("length", (385, 1089, 4500))   # 4500: 245 columns for key block 0
def test_rescue_choice_vs_oracle(gpu, length):
    """Same token as the float64 argmax, except fp32 near-ties (then the GPU's token
    scores within 1e-5 of the maximum)."""
    q, k, v = inputs(length, seed=61)
    got = _choice(q.cuda(), k.cuda(), v.cuda())
    want = ref.rescue_choice(to_np(q), to_np(k))
    blocks = ref.num_blocks(length)
    causal = np.arange(blocks)[None, :, None, None] < np.arange(blocks)[None, None, :, None]
    causal = np.broadcast_to(causal.transpose(0, 2, 1, 3), got.shape)
    assert (got[~causal] == 0).all()
    diff = np.argwhere((got != want) & causal)
    qbar = ref.tile_mean_query(to_np(q)).astype(np.float64)
    kk = to_np(k).astype(np.float64)
    for b, t, j, h in diff:
        scores = kk[b, j * 128:(j + 1) * 128, h // 7] @ qbar[b, t, h]
        assert scores.max() - scores[got[b, t, j, h]] <= 1e-5 * (abs(scores.max()) + 1), (t, j, h)
    assert len(diff) <= max(2, causal.sum() // 1000)


@pytest.mark.parametrize("remainder", (False, True))
@pytest.mark.parametrize("length", (385, 1089))
def test_rescue_tail_vs_oracle(gpu, length, remainder):
    q, k, v = inputs(length, seed=67)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    sel = _fixed_selection(length, seed=11, drop=0.5)
    out, lse = kernels.rescue_tail(qg, kg, vg, torch.from_numpy(sel).cuda(), SCALE,
                                   remainder=remainder)
    e_out, e_lse = ref.rescue_tail(to_np(q), to_np(k), to_np(v), sel, SCALE, remainder=remainder,
                                   choice=_choice(qg, kg, vg))
    # token values are O(1) (not block means): bf16 probabilities leave ~2^-8 |v|
    np.testing.assert_allclose(to_np(out), e_out, atol=1e-2, rtol=2e-2)
    finite = np.isfinite(e_lse)
    assert finite.any() and not finite.all()
    np.testing.assert_array_equal(np.isfinite(to_np(lse)), finite)
    np.testing.assert_allclose(to_np(lse)[finite], e_lse[finite], atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("remainder", (False, True))
def test_exact_plus_rescue_vs_check_math(gpu, remainder):
    """check_math.py:252-287: 385 tokens, the reference's fixed mask, exact + rescue
    tail + merge against the token-level reference (0.03 / 0.025 tolerances), and
    the result of rows < 300 unchanged when K / V change at positions >= 300."""
    q, k, v = inputs(385, seed=71)
    sel = ref.protected_selection(np.zeros((1, 4, 4, 28), np.float32), 0.0, 2, 4, 2)
    sel[:, 2, 0, ::2] = False
    sel[:, 2, 1, 1::2] = False
    sel[:, 3, 1, :] = False
    idx, cnt = ref.indices_from_mask(sel)

    def path(kg, vg):
        qg = q.cuda()
        ex, ex_lse = up.exact_attention(qg, kg, vg, torch.from_numpy(idx).cuda(),
                                        torch.from_numpy(cnt).cuda(), SCALE)
        tail, tail_lse = kernels.rescue_tail(qg, kg, vg, torch.from_numpy(sel).cuda(), SCALE,
                                             chunk_tiles=2, remainder=remainder)
        return kernels.merge_exact_mean(ex, ex_lse, tail, tail_lse)

    out, lse = path(k.cuda(), v.cuda())
    want, want_lse = explicit_rescue_reference(to_np(q), to_np(k), to_np(v), sel, SCALE, remainder)
    np.testing.assert_allclose(to_np(out), want, atol=0.03, rtol=0.03)
    np.testing.assert_allclose(to_np(lse), want_lse, atol=0.025, rtol=0.015)
    k2, v2 = k.clone(), v.clone()
    k2[:, 300:] *= 19
    v2[:, 300:] += 23
    out2, _ = path(k2.cuda(), v2.cuda())
    assert torch.equal(out2[:, :300], out[:, :300])


@pytest.mark.parametrize("length", (1089, 4096))
@pytest.mark.parametrize("method", ("fp_v1_rescue", "fp_v1_rescue_v2"))
def test_backend_rescue_vs_oracle(gpu, method, length):
    """Whole layer against the oracle layer on inputs whose V1 selection is sparse
    (Q and K scaled by 5, alpha 0.5), so the rescue tails are not empty."""
    q, k, v = inputs(length, seed=73)
    q = (q.float() * 5).to(torch.bfloat16)
    k = (k.float() * 5).to(torch.bfloat16)
    alpha = 0.5
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    out, _ = backend.forward(type("L", (), {"layer_idx": 0})(), qg.transpose(1, 2),
                             kg.transpose(1, 2), vg.transpose(1, 2), None, SCALE)
    precision = "f64" if length <= 1089 else "f32"
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, alpha,
                                   precision=precision)
    assert expected["selected"].sum() < expected["selected"].size   # some tail exists
    blocks = ref.num_blocks(length)
    assert expected["counts"].sum() < 28 * blocks * (blocks + 1) // 2
    assert out.shape == (1, length, 28, 128) and out.dtype == torch.bfloat16
    # peaked attention on the scaled inputs gives outputs up to |v| ~ 4-5, where one
    # bf16 step is 2^-5: the absolute bound gets one output rounding step on top
    assert_output_close(to_np(out), expected["output"], what=method, rel=2.0 ** -7)
