"""The BASELINE configurations at their real sizes, against the oracle's own routing.

* config 2: S = 32640, seed 17, all six methods at alpha 0.08;
* config 3: S = 32640 with 64 planted needles, alpha in {0.04, 0.08, 0.16} for the
  four mean-corrected methods plus fp_v1 at 0.08 and dense;
* config 5: S = 131072 with 256 planted needles, cgf_mean and dispersion_mean at
  alpha 0.04.

Each case runs ``AttentionBackend.forward`` on the GPU and checks:
* the selection mask equals the oracle's routing (scores computed by the oracle
  from the same inputs, the reference's selection rule) except entries within
  1e-6 of the threshold, and equals the rule applied to the GPU's own scores
  exactly;
* the GPU scores are within check_math's tolerances of the oracle's;
* the layer output matches the oracle on sampled query tiles spread over the
  sequence, computed from the oracle's own lists (max-abs 2e-2, mean-abs 2e-3).
At 131072 the oracle scores only the sampled tiles (a tile's selector scores
depend on its own rows only).
"""

import numpy as np
import pytest
import torch

from exp3_amd import attention, synthetic
from oracle import reference_cpu as ref
from tests.helpers import (SCALE, V1_METHODS, agreeing_tiles, assert_output_close,
                           gpu_routing, masks_equal_except_ties, oracle_scores, record_ties,
                           select, threshold_ties, tile_rows, to_np)

pytestmark = pytest.mark.gpu

SEQ = 32640
BLOCKS = 255
SIX = ("dense", "fp_v1", "mean_native", "mean_balanced", "cgf_mean", "dispersion_mean")
SAMPLE = (0, 1, 64, 128, 191, BLOCKS - 3, BLOCKS - 1)
SCORE_TOL = {"v1": dict(atol=2e-4, rtol=0.005), "selector": dict(atol=2e-5, rtol=2e-5)}


class _Layer:
    layer_idx = 0


class _Case:
    """Seeded inputs on the host (numpy, float32 holding bf16 values) and the GPU,
    with the oracle's scores cached per scoring family."""

    def __init__(self, sequence, needles):
        q, k, v, self.needles = synthetic.make_inputs(sequence, seed=17, needles=needles)
        self.q, self.k, self.v = q.cuda(), k.cuda(), v.cuda()
        self.qn, self.kn, self.vn = to_np(q), to_np(k), to_np(v)
        self.sequence = sequence
        self._scores = {}
        self._desc = None

    def scores(self, method, tiles=None):
        key = "v1" if method in V1_METHODS else (method, tuple(tiles) if tiles else None)
        if key not in self._scores:
            self._scores[key] = oracle_scores(self.qn, self.kn, self.vn, method, tiles=tiles)
        return self._scores[key]

    def descriptors(self):
        if self._desc is None:
            self._desc = ref.block_descriptors(self.kn, self.vn, precision="f32")
        return self._desc


@pytest.fixture(scope="module")
def config2():
    return _Case(SEQ, needles=0)


@pytest.fixture(scope="module")
def config3():
    return _Case(SEQ, needles=64)


def _forward(case, method, alpha):
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    out, _ = backend.forward(_Layer(), case.q.transpose(1, 2), case.k.transpose(1, 2),
                             case.v.transpose(1, 2), None, SCALE)
    assert out.shape == (1, case.sequence, 28, 128) and out.dtype == torch.bfloat16
    return backend, out


def _check_layer(case, method, alpha, sample=SAMPLE, name="config"):
    backend, out = _forward(case, method, alpha)
    blocks = ref.num_blocks(case.sequence)
    if method == "dense":
        e_sel = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[None, :, :, None],
                                (1, blocks, blocks, 28))
        tiles = list(sample)
        density = 1.0
    else:
        g_scores, g_sel = gpu_routing(backend, case.q, case.k, case.v, method)
        e_scores = case.scores(method)
        family = "v1" if method in V1_METHODS else "selector"
        np.testing.assert_allclose(g_scores, e_scores, **SCORE_TOL[family])
        # the GPU mask is exactly the rule on the GPU's own scores
        np.testing.assert_array_equal(g_sel, select(g_scores, method, alpha))
        e_sel = select(e_scores, method, alpha)
        ties = threshold_ties(e_scores, alpha, positive_rule=family == "selector")
        bad, differ, listed = masks_equal_except_ties(g_sel, e_sel, ties)
        record_ties(f"{name} S={case.sequence}", method, alpha, ties, differ, listed)
        assert bad == 0, f"{bad} mask entries differ away from the threshold"
        density = g_sel.sum() / (28 * blocks * (blocks + 1) / 2)
        print(f"{method} alpha={alpha}: density {density:.5f} (oracle "
              f"{e_sel.sum() / (28 * blocks * (blocks + 1) / 2):.5f}), {differ} tie entries "
              f"differ: {listed}")
        tiles = agreeing_tiles(sample, g_sel, e_sel)
    desc = case.descriptors() if method in attention.MEAN_METHODS else None
    expected, _ = ref.attention_from_selection(case.qn, case.kn, case.vn, SCALE, method, e_sel,
                                               desc, precision="f32", tiles=tiles)
    rows = tile_rows(tiles, case.sequence)
    assert_output_close(to_np(out[:, rows]), expected[:, rows],
                        what=f"{method} alpha={alpha} S={case.sequence} tiles {tiles}")
    return density


@pytest.mark.parametrize("method", SIX)
def test_config2_six_methods(gpu, config2, method):
    _check_layer(config2, method, 0.08, name="config 2")


CONFIG3 = [(m, a) for a in (0.04, 0.08, 0.16)
           for m in ("mean_native", "mean_balanced", "cgf_mean", "dispersion_mean")]
CONFIG3 += [("fp_v1", 0.08), ("dense", None)]


@pytest.mark.parametrize("method,alpha", CONFIG3)
def test_config3_needles(gpu, config3, method, alpha):
    assert len(config3.needles) == 64
    _check_layer(config3, method, 0.08 if alpha is None else alpha, name="config 3 (64 needles)")


LONG = 131072
LONG_BLOCKS = 1024
LONG_SAMPLE = (1, 300, 700, LONG_BLOCKS - 3, LONG_BLOCKS - 1)


@pytest.fixture(scope="module")
def config5():
    return _Case(LONG, needles=256)


@pytest.mark.parametrize("method", ("cgf_mean", "dispersion_mean"))
def test_config5_long_context(gpu, config5, method):
    """S = 131072 (1024 blocks), 256 needles, alpha 0.04: the selectors' scores on
    sampled tiles against the oracle, the whole mask against the rule on the GPU's
    scores, the sampled tiles' masks against the oracle's, and their outputs."""
    alpha = 0.04
    case = config5
    assert len(case.needles) == 256
    backend, out = _forward(case, method, alpha)
    assert torch.isfinite(out).all()
    g_scores, g_sel = gpu_routing(backend, case.q, case.k, case.v, method)
    np.testing.assert_array_equal(g_sel, select(g_scores, method, alpha))
    sample = list(LONG_SAMPLE)
    e_scores = case.scores(method, tiles=sample)        # rows of the sampled tiles only
    np.testing.assert_allclose(g_scores[:, sample], e_scores[:, sample], **SCORE_TOL["selector"])
    e_sel = select(e_scores, method, alpha)
    ties = threshold_ties(e_scores, alpha, positive_rule=True)
    bad, differ, listed = masks_equal_except_ties(g_sel[:, sample], e_sel[:, sample],
                                                  ties[:, sample])
    sampled_ties = np.zeros_like(ties)
    sampled_ties[:, sample] = ties[:, sample]
    record_ties(f"config 5 (256 needles) S={LONG} tiles {sample}", method, alpha,
                sampled_ties, differ, listed, tiles=sample)
    assert bad == 0, f"{bad} sampled mask entries differ away from the threshold"
    same = (g_sel[:, sample] == e_sel[:, sample]).all(axis=(0, 2, 3))
    tiles = [t for t, ok in zip(sample, same) if ok]
    assert len(tiles) >= 4, f"masks differ at ties on too many sampled tiles: {listed}"
    density = g_sel.sum() / (28 * LONG_BLOCKS * (LONG_BLOCKS + 1) / 2)
    print(f"{method} S={LONG}: density {density:.5f}, sampled tiles {tiles}")
    expected, _ = ref.attention_from_selection(case.qn, case.kn, case.vn, SCALE, method, e_sel,
                                               case.descriptors(), precision="f32", tiles=tiles)
    rows = tile_rows(tiles, LONG)
    assert_output_close(to_np(out[:, rows]), expected[:, rows],
                        what=f"{method} S={LONG} tiles {tiles}")
