"""The V1 capture hook (reference attention.py:239-251, 345-350): a synchronous
callback that fires for fp_v1 prefill only, with the layer's q / k / v, the bf16
block-mean K, the V1 scores, the index lists, counts and mask of that call."""

import numpy as np
import pytest
import torch

from exp3_amd import attention
from oracle import reference_cpu as ref
from tests.helpers import (SCALE, inputs, masks_equal_except_ties, threshold_ties, to_np)

pytestmark = pytest.mark.gpu

KEYS = ("layer", "q", "k", "v", "mean_k", "scores", "indices", "counts", "selected", "scale")


class _Layer:
    layer_idx = 5


def _forward(backend, q, k, v):
    out, _ = backend.forward(_Layer(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                             attention_mask=None, scaling=SCALE)
    return out


def test_capture_fires_for_fp_v1_prefill_only(gpu):
    length, alpha = 1089, 0.08
    q, k, v = inputs(length, seed=83, needles=8)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    calls = []

    def callback(**kwargs):
        # synchronous: the tensors are complete when the callback runs
        calls.append({name: (value.clone() if isinstance(value, torch.Tensor) else value)
                      for name, value in kwargs.items()})

    backend.start_capture(callback)
    for method in ("dense", "mean_native", "mean_balanced", "fp_v1_rescue"):
        backend.configure(method, alpha)
        _forward(backend, qg, kg, vg)
    assert calls == [], "the capture hook fired for a method other than fp_v1"

    backend.configure("fp_v1", alpha)
    out = _forward(backend, qg, kg, vg)
    assert len(calls) == 1
    got = calls[0]
    assert set(got) == set(KEYS)
    assert got["layer"] == 5 and got["scale"] == SCALE
    assert torch.equal(got["q"], qg) and torch.equal(got["k"], kg) and torch.equal(got["v"], vg)
    assert got["q"].shape == (1, length, 28, 128)

    # the captured tensors are _v1_selection's auxiliary outputs for this input
    record = {"events": {}}
    _, kbar, scores, idx, cnt, sel = backend._v1_selection(qg, kg, SCALE, record, None, True)
    for name, want in (("mean_k", kbar), ("scores", scores), ("indices", idx), ("counts", cnt),
                       ("selected", sel)):
        assert got[name].dtype == want.dtype and torch.equal(got[name], want), name

    # ... and the oracle's, up to threshold ties
    qn, kn = to_np(q), to_np(k)
    e_kbar = ref.block_mean_k(kn, precision="f32")
    # bf16 block means: within one bf16 rounding step of the oracle's
    assert (np.abs(to_np(got["mean_k"]) - e_kbar) <= np.abs(e_kbar) * 2.0 ** -7 + 1e-30).all()
    e_scores = ref.v1_scores(qn, e_kbar, SCALE, precision="f32")
    np.testing.assert_allclose(to_np(got["scores"]), e_scores, atol=2e-4, rtol=0.005)
    e_idx, e_cnt = ref.deal_output_score(e_scores, 2, 4, alpha, 2, 0)
    e_sel = ref.mask_from_indices(e_idx, e_cnt)
    bad, _, _ = masks_equal_except_ties(to_np(got["selected"]), e_sel,
                                        threshold_ties(e_scores, alpha))
    assert bad == 0

    # decode steps (q_len != kv_len) never capture; finish_capture detaches
    backend.forward(_Layer(), qg[:, -1:].transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2),
                    attention_mask=None, scaling=SCALE)
    assert len(calls) == 1
    backend.finish_capture()
    again = _forward(backend, qg, kg, vg)
    assert len(calls) == 1
    assert torch.equal(again, out)
