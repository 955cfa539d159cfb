"""Shared test helpers: seeded inputs, tolerance checks, tie listing."""

from __future__ import annotations

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


def masks_equal_except_ties(actual, expected, ties):
    differ = actual != expected
    unexplained = differ & ~ties
    return int(unexplained.sum()), int(differ.sum()), [tuple(int(x) for x in idx)
                                                      for idx in np.argwhere(differ & ties)[:20]]
