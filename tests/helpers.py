"""Shared test helpers: seeded inputs, tolerance checks, tie listing."""

from __future__ import annotations

import json
import os

import numpy as np
import torch

from exp3_amd import synthetic
from oracle import reference_cpu as ref

SCALE = 128 ** -0.5
# North-star output tolerance (bf16): max-abs and mean-abs versus the oracle.
OUT_MAX_ABS = 2e-2
OUT_MEAN_ABS = 2e-3
TIE_EPS = 1e-6


def inputs(sequence, seed=17, needles=0, device="cpu"):
    q, k, v, planted = synthetic.make_inputs(sequence, seed=seed, needles=needles, device=device)
    return q, k, v


def to_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bool:
        return t.cpu().numpy()
    if t.dtype in (torch.int64, torch.int32, torch.uint8):
        return t.cpu().numpy()
    return t.float().cpu().numpy()


def assert_output_close(actual, expected, max_abs=OUT_MAX_ABS, mean_abs=OUT_MEAN_ABS, what="output",
                        rel=0.0):
    """max |a - e| - rel |e| <= max_abs and mean |a - e| <= mean_abs; ``rel`` = 2^-7
    admits one bf16 output rounding step for outputs beyond unit scale."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite values"
    diff = np.abs(a - e)
    worst = float((diff - rel * np.abs(e)).max()) if diff.size else 0.0
    mean = float(diff.mean()) if diff.size else 0.0
    assert worst <= max_abs and mean <= mean_abs, \
        f"{what}: max-abs {worst:.3g} (limit {max_abs}, rel {rel}), mean-abs {mean:.3g} (limit {mean_abs})"
    return worst, mean


def threshold_ties(scores, alpha, positive_rule=False):
    """Entries whose score is within TIE_EPS of their row's threshold."""
    maximum = scores.max(axis=2, keepdims=True)
    thr = (maximum.astype(np.float32) * np.float32(alpha)).astype(np.float32)
    near = np.abs(scores.astype(np.float64) - thr.astype(np.float64)) <= TIE_EPS
    if positive_rule:
        near |= np.abs(scores) <= TIE_EPS
    return near


def routed_entries(shape, sink=2, window=4, last=2):
    """Entries [b, t, j, h] whose selection the threshold decides: causal (j <= t)
    and outside the protected sink, window and last query blocks."""
    t = np.arange(shape[1]).reshape(1, -1, 1, 1)
    j = np.arange(shape[2]).reshape(1, 1, -1, 1)
    routed = (j <= t - window) & (j >= sink) & (t < shape[1] - last)
    return np.broadcast_to(routed, shape)


def record_ties(case, method, alpha, ties, differ, listed, tiles=None):
    """Append one case's threshold-tie count (routed entries within TIE_EPS of the
    threshold, or of 0 under the positive-score rule) and how many of them the GPU
    mask sets differently to the JSON-lines file named by SPX_TIES_LOG, when that
    variable is set."""
    path = os.environ.get("SPX_TIES_LOG")
    if not path:
        return
    routed = routed_entries(ties.shape)
    if tiles is not None:
        routed = routed & np.isin(np.arange(ties.shape[1]), tiles).reshape(1, -1, 1, 1)
    with open(path, "a") as f:
        f.write(json.dumps({"case": case, "method": method, "alpha": alpha,
                            "routed_entries": int(np.count_nonzero(routed)),
                            "tie_entries": int(np.count_nonzero(ties & routed)),
                            "differ": int(differ), "listed": listed}) + "\n")


def masks_equal_except_ties(actual, expected, ties):
    differ = actual != expected
    unexplained = differ & ~ties
    return int(unexplained.sum()), int(differ.sum()), [tuple(int(x) for x in idx)
                                                      for idx in np.argwhere(differ & ties)[:20]]


# ------------------------------------------------------ whole-layer comparisons

V1_METHODS = ("fp_v1", "mean_native", "fp_v1_rescue", "fp_v1_rescue_v2")
SELECTOR_METHODS = ("mean_balanced", "cgf_mean", "dispersion_mean")


def gpu_routing(backend, qg, kg, vg, method, scale=SCALE):
    """The GPU's scores (float32 numpy) and selection mask for ``method``, from the
    same kernels ``forward`` launches (every stage is deterministic)."""
    from exp3_amd import kernels
    record = {"events": {}}
    if method in V1_METHODS:
        values = vg if method in ("mean_native", "fp_v1_rescue_v2") else None
        _, _, scores, _, _, sel = backend._v1_selection(qg, kg, scale, record, values, True)
    else:
        desc, _, _, _, sel = backend._new_selection(qg, kg, vg, scale, record)
        scores = kernels.selector_scores(qg, desc, scale, method)
    return to_np(scores), to_np(sel)


def oracle_scores(qn, kn, vn, method, scale=SCALE, tiles=None):
    """The oracle's routing scores (float32 arithmetic, as the reference's)."""
    if method in V1_METHODS:
        kbar = ref.block_mean_k(kn, precision="f32")
        return ref.v1_scores(qn, kbar, scale, precision="f32")
    desc = ref.block_descriptors(kn, vn, precision="f32")
    return ref.selector_scores(qn, desc, scale, method, precision="f32", tiles=tiles)


def select(scores, method, alpha):
    """The reference's selection rule for ``method`` applied to ``scores``."""
    if method in V1_METHODS:
        return ref.mask_from_indices(*ref.deal_output_score(scores, 2, 4, alpha, 2, 0))
    return ref.protected_selection(scores, alpha, 2, 4, 2)


def agreeing_tiles(wanted, actual_sel, expected_sel, reach=4):
    """Each wanted query tile, or the nearest one within ``reach`` whose masks
    (every head) agree; a tile whose selection differs at a threshold tie would
    compare two different attention problems."""
    blocks = actual_sel.shape[1]
    same = (actual_sel == expected_sel).all(axis=(0, 2, 3))
    chosen = []
    for t in wanted:
        for d in range(reach + 1):
            hit = next((c for c in (t - d, t + d) if 0 <= c < blocks and same[c]), None)
            if hit is not None:
                if hit not in chosen:
                    chosen.append(hit)
                break
        else:
            raise AssertionError(f"no tile near {t} with identical masks")
    return chosen


def tile_rows(tiles, sequence, block_size=128):
    return np.concatenate([np.arange(t * block_size, min(sequence, (t + 1) * block_size))
                           for t in tiles])
