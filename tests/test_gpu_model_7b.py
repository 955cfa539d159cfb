"""BASELINE config 4 in a test: the full 28-layer random-init Qwen2.5-7B architecture
(hidden 3584, FFN 18944, 28 / 4 heads, RMSNorm 1e-6, RoPE theta 1e6, vocab 152064,
QKV bias, bf16) prefilling 32640 token ids through the backend registered as
transformers' "sdpa" attention function (attention.py:57), for dense, fp_v1,
mean_native and cgf_mean:

* the prefill (evaluate.py:323-345: ``model(ids, use_cache=True,
  logits_to_keep=1)``) gives finite logits, and evaluate.py:357-380's
  split-last-token flow (prefill of S - 1 ids, then the last id as one cached
  decode step) gives the same greedy id unless the top two logits are closer than
  the two flows' difference;
* one layer's attention call, captured from inside the model, matches the oracle
  on sampled query tiles (for the sparse methods through the oracle's own routing
  of that layer's q / k / v: scores within check_math's tolerances, the mask equal
  to the oracle's except entries within 1e-6 of the threshold).
"""

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref
from tests.helpers import (V1_METHODS, agreeing_tiles, assert_output_close, gpu_routing,
                           masks_equal_except_ties, oracle_scores, record_ties, select,
                           threshold_ties, tile_rows, to_np)

pytestmark = pytest.mark.gpu

SEQ = 32640
CAPTURED_LAYER = 20
SAMPLE = (0, 1, 90, 180, 252, 254)
SCORE_TOL = {"v1": dict(atol=2e-4, rtol=0.005), "selector": dict(atol=2e-5, rtol=2e-5)}


@pytest.fixture(scope="module")
def qwen7b(gpu):
    transformers = pytest.importorskip("transformers")
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from exp3_amd import attention
    from measure.sweeps import qwen2_7b_config

    saved = ALL_ATTENTION_FUNCTIONS["sdpa"]
    backend = attention.AttentionBackend(alpha=0.08)   # registers as "sdpa"
    torch.manual_seed(17)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = transformers.Qwen2ForCausalLM(qwen2_7b_config(28))
    finally:
        torch.set_default_dtype(torch.float32)
    model.eval()
    ids = torch.randint(0, 152064, (1, SEQ), generator=torch.Generator().manual_seed(17)).cuda()
    try:
        yield model, backend, ids
    finally:
        ALL_ATTENTION_FUNCTIONS["sdpa"] = saved
        del model
        torch.cuda.empty_cache()


class _Capture:
    """Wraps the registered forward; keeps one layer's inputs, scaling and output."""

    def __init__(self, backend, layer):
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        self.functions = ALL_ATTENTION_FUNCTIONS
        self.inner = backend.forward
        self.layer = layer
        self.seen = None

    def __call__(self, module, query, key, value, attention_mask, scaling, dropout=0.0, **kw):
        out, extra = self.inner(module, query, key, value, attention_mask, scaling, dropout, **kw)
        if module.layer_idx == self.layer and query.shape[2] == key.shape[2] and self.seen is None:
            self.seen = {"q": query.transpose(1, 2).clone(), "k": key.transpose(1, 2).clone(),
                         "v": value.transpose(1, 2).clone(), "out": out.clone(),
                         "scale": float(scaling)}
        return out, extra

    def __enter__(self):
        self.functions["sdpa"] = self
        return self

    def __exit__(self, *exc):
        self.functions["sdpa"] = self.inner


@pytest.mark.parametrize("method", ("dense", "fp_v1", "mean_native", "cgf_mean"))
def test_qwen2_7b_prefill_32640(qwen7b, method):
    model, backend, ids = qwen7b
    alpha = 0.08
    backend.configure(method, alpha)
    with torch.no_grad(), _Capture(backend, CAPTURED_LAYER) as capture:
        full = model(ids, use_cache=True, logits_to_keep=1).logits[:, -1].float()
    assert full.shape == (1, 152064) and torch.isfinite(full).all()
    layer = capture.seen
    assert layer is not None and layer["q"].shape == (1, SEQ, 28, 128)
    assert layer["k"].shape == (1, SEQ, 4, 128)

    with torch.no_grad():
        pre = model.model(input_ids=ids[:, :-1], use_cache=True)
        step = model(input_ids=ids[:, -1:], past_key_values=pre.past_key_values, use_cache=True,
                     cache_position=torch.tensor([SEQ - 1], device="cuda"),
                     logits_to_keep=1).logits[:, -1].float()
    del pre
    assert torch.isfinite(step).all()
    diff = (full - step).abs().max().item()
    top2 = full[0].topk(2).values
    print(f"{method}: greedy full {int(full.argmax())} split {int(step.argmax())}, "
          f"max |diff| {diff:.3g}, top-2 gap {(top2[0] - top2[1]).item():.3g}")
    if (top2[0] - top2[1]).item() > 2 * diff:
        assert int(full.argmax()) == int(step.argmax())

    # the captured layer against the oracle, from that layer's own q / k / v
    scale = layer["scale"]
    qn, kn, vn = to_np(layer["q"]), to_np(layer["k"]), to_np(layer["v"])
    blocks = ref.num_blocks(SEQ)
    if method == "dense":
        e_sel = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[None, :, :, None],
                                (1, blocks, blocks, 28))
        tiles = list(SAMPLE)
    else:
        family = "v1" if method in V1_METHODS else "selector"
        g_scores, g_sel = gpu_routing(backend, layer["q"], layer["k"], layer["v"], method, scale)
        e_scores = oracle_scores(qn, kn, vn, method, scale)
        np.testing.assert_allclose(g_scores, e_scores, **SCORE_TOL[family])
        np.testing.assert_array_equal(g_sel, select(g_scores, method, alpha))
        e_sel = select(e_scores, method, alpha)
        ties = threshold_ties(e_scores, alpha, positive_rule=family == "selector")
        bad, differ, listed = masks_equal_except_ties(g_sel, e_sel, ties)
        record_ties(f"config 4 layer {CAPTURED_LAYER} S={SEQ}", method, alpha, ties, differ,
                    listed)
        assert bad == 0
        print(f"layer {CAPTURED_LAYER}: density {g_sel.sum() / (28 * blocks * (blocks + 1) / 2):.4f},"
              f" {differ} tie entries differ: {listed}")
        tiles = agreeing_tiles(SAMPLE, g_sel, e_sel)
    expected, _ = ref.attention_from_selection(qn, kn, vn, scale, method, e_sel,
                                               precision="f32", tiles=tiles)
    rows = tile_rows(tiles, SEQ)
    assert_output_close(to_np(layer["out"][:, rows]), expected[:, rows],
                        what=f"Qwen2.5-7B layer {CAPTURED_LAYER} {method} tiles {tiles}")
