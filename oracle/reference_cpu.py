"""CPU restatement (numpy) of exp3's sparse-prefill attention path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, as the checker or the timed CPU
baseline. The product package never imports it.

Every function restates one reference function; the docstring cites the
reference file:line it follows (paths relative to the reference repository).
Conventions:

* Tensors are numpy arrays in the reference's ``[batch, sequence, heads, dim]``
  order. bf16 inputs are passed as float32 arrays holding bf16-exact values
  (``bf16_round`` produces them); outputs the reference stores in bf16 are
  returned rounded with ``bf16_round`` (round-to-nearest-even).
* ``precision="f64"`` (the default, used for parity checks) accumulates dot
  products and sums in float64 and rounds to float32 where the reference
  stores float32. ``precision="f32"`` keeps the reference's float32 arithmetic
  throughout and is what the CPU baseline times.
* Score / mask / index tensors use the reference layout
  ``[batch, query_block, key_block, q_head]``.

Parity pins for every function live in ``tests/test_oracle_pins.py``; the
functions with no pin are named in this header: none.
"""

from __future__ import annotations

import math

import numpy as np

BLOCK_SIZE = 128
LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453
METHODS = (
    "dense",
    "fp_v1",
    "mean_native",
    "mean_balanced",
    "cgf_mean",
    "dispersion_mean",
    "fp_v1_rescue",
    "fp_v1_rescue_v2",
)
V1_ROUTED = {"fp_v1", "mean_native", "fp_v1_rescue", "fp_v1_rescue_v2"}
MEAN_METHODS = {"mean_native", "mean_balanced", "cgf_mean", "dispersion_mean"}
RESCUE_METHODS = {"fp_v1_rescue", "fp_v1_rescue_v2"}
SELECTORS = ("mean_balanced", "cgf_mean", "dispersion_mean")

_F32 = np.float32
_NEG_INF = np.float32(-np.inf)


# ----------------------------------------------------------------- bf16 helpers

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round-to-nearest-even, NaN kept quiet."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    # uint32 sums cannot wrap for non-NaN patterns (at most 0xFF7FFFFF + 0x8000);
    # NaN entries are overwritten below
    rounded = (u >> 16) & np.uint32(1)
    rounded += u
    rounded += np.uint32(0x7FFF)
    rounded >>= np.uint32(16)
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return from_bf16_bits(bf16_bits(x))


def _acc(precision: str):
    if precision not in ("f64", "f32"):
        raise ValueError(f"precision must be 'f64' or 'f32', got {precision!r}")
    return np.float64 if precision == "f64" else np.float32


# ------------------------------------------------------------------- geometry

def num_blocks(sequence: int, block_size: int = BLOCK_SIZE) -> int:
    return (sequence + block_size - 1) // block_size


def block_counts(sequence: int, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Valid tokens per block (kernels.py:33-34)."""
    blocks = num_blocks(sequence, block_size)
    counts = np.full(blocks, block_size, dtype=np.int32)
    counts[-1] = sequence - (blocks - 1) * block_size
    return counts


def _pad_blocks(x: np.ndarray, block_size: int) -> np.ndarray:
    batch, sequence, heads, dim = x.shape
    blocks = num_blocks(sequence, block_size)
    padded = np.zeros((batch, blocks * block_size, heads, dim), dtype=x.dtype)
    padded[:, :sequence] = x
    return padded.reshape(batch, blocks, block_size, heads, dim)


def _expand_heads(x: np.ndarray, q_heads: int, axis: int) -> np.ndarray:
    group = q_heads // x.shape[axis]
    return np.repeat(x, group, axis=axis)


# ------------------------------------------------------------------ pooling

def block_mean_k(k: np.ndarray, block_size: int = BLOCK_SIZE, precision: str = "f64"):
    """bf16 block mean of K over valid tokens.

    upstream/flashprefill_native_forward.py:27-69 (``compute_mean_vector``) and
    :420-442 (``block_mean_k``): float32 sum over the block's valid rows, divided
    by the valid count, stored as bf16.
    """
    acc = _acc(precision)
    counts = block_counts(k.shape[1], block_size).astype(np.float32)
    sums = _pad_blocks(k, block_size).astype(acc).sum(axis=2).astype(np.float32)
    mean = sums / counts.reshape(1, -1, 1, 1)
    return bf16_round(mean.astype(np.float32))


class BlockDescriptors:
    """kernels.py:13-19."""

    def __init__(self, mean_k, mean_v, var_k, sigma_v, counts):
        self.mean_k = mean_k
        self.mean_v = mean_v
        self.var_k = var_k
        self.sigma_v = sigma_v
        self.counts = counts


def block_descriptors(k: np.ndarray, v: np.ndarray, block_size: int = BLOCK_SIZE,
                      precision: str = "f64") -> BlockDescriptors:
    """FP32 block moments per KV head (kernels.py:22-46).

    Keeps the reference's one-pass variance ``E[x^2] - mean^2`` clamped at 0,
    computed in float32 from float32 sums.
    """
    acc = _acc(precision)
    counts = block_counts(k.shape[1], block_size)
    denominator = counts.astype(np.float32).reshape(1, -1, 1, 1)

    def moments(x):
        blocks = _pad_blocks(x, block_size).astype(acc)
        total = blocks.sum(axis=2).astype(np.float32)
        square = (blocks * blocks).sum(axis=2).astype(np.float32)
        mean = (total / denominator).astype(np.float32)
        var = np.maximum(square / denominator - mean * mean, np.float32(0)).astype(np.float32)
        return mean, var

    mean_k, var_k = moments(k)
    mean_v, var_v = moments(v)
    sigma_v = np.sqrt(var_v.astype(acc).sum(axis=-1).astype(np.float32)).astype(np.float32)
    return BlockDescriptors(mean_k, mean_v, var_k, sigma_v, counts)


# ------------------------------------------------------------ V1 block score

def v1_scores_raw(q: np.ndarray, mean_k: np.ndarray, scale: float,
                  block_size: int = BLOCK_SIZE, precision: str = "f64"):
    """Per (query tile, key block, head) max and base-2 mass of the V1 proxy.

    upstream/flashprefill_native_forward.py:89-175 (``compute_block_score``):
    x_ij = fp32(q_i . Kbar_j) * fp32(scale * log2 e); a row i of tile t is valid
    for key block j when i >= (j + 1) * block - 1 and i < S.
    M_tj = max over valid rows, m_tj = sum over valid rows of 2^(x - M_tj).
    Entries with no valid row hold M = -inf, m = 0.
    """
    acc = _acc(precision)
    batch, sequence, q_heads, _ = q.shape
    blocks = mean_k.shape[1]
    c = np.float32(scale * LOG2E)
    kbar = _expand_heads(mean_k, q_heads, axis=2)
    key_end = (np.arange(blocks) + 1) * block_size - 1
    rows = np.arange(sequence)
    valid = rows[:, None] >= key_end[None, :]                      # [S, NB]
    pad = blocks * block_size - sequence
    mass = np.zeros((batch, blocks, blocks, q_heads), dtype=np.float32)
    maximum = np.full((batch, blocks, blocks, q_heads), -np.inf, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for b in range(batch):
            for h in range(q_heads):
                dots = q[b, :, h].astype(acc) @ kbar[b, :, h].astype(acc).T   # [S, NB]
                x = dots.astype(np.float32) * c
                x = np.where(valid, x, _NEG_INF)
                x = np.concatenate([x, np.full((pad, blocks), -np.inf, np.float32)])
                x = x.reshape(blocks, block_size, blocks)
                tile_max = x.max(axis=1)                               # [NB(t), NB(j)]
                finite = np.isfinite(tile_max)
                safe_max = np.where(finite, tile_max, 0).astype(np.float32)
                expo = np.exp2((x - safe_max[:, None, :]).astype(acc))
                tile_mass = np.where(finite, expo.sum(axis=1), 0).astype(np.float32)
                mass[b, :, :, h] = tile_mass
                maximum[b, :, :, h] = tile_max
    return mass, maximum


def normalize_scores(score: np.ndarray, maximum: np.ndarray, precision: str = "f64"):
    """upstream/flashprefill_native_forward.py:410-417.

    w_j = finite(M_j) ? m_j * 2^(M_j - max_j M) : 0 ; score_j = w_j / (sum_j w + 1e-9).
    """
    acc = _acc(precision)
    with np.errstate(invalid="ignore", over="ignore"):
        finite = maximum != -np.inf
        global_max = maximum.max(axis=2, keepdims=True)
        rescale = np.where(finite, np.exp2((maximum - global_max).astype(np.float32)), 1)
        weight = (np.where(finite, score, 0).astype(np.float32) * rescale.astype(np.float32))
        weight = weight.astype(np.float32)
        total = weight.astype(acc).sum(axis=2, keepdims=True).astype(np.float32)
        return (weight / (total + np.float32(1e-9))).astype(np.float32)


def v1_scores(q, mean_k, scale, block_size: int = BLOCK_SIZE, precision: str = "f64"):
    """upstream/flashprefill_native_forward.py:445-475."""
    mass, maximum = v1_scores_raw(q, mean_k, scale, block_size, precision)
    return normalize_scores(mass, maximum, precision)


# ------------------------------------------------------------------ selection

def _threshold(maximum: np.ndarray, alpha: float) -> np.ndarray:
    """fp32(max * fp32(alpha)): the reference multiplies a float32 tensor by a
    Python float, which PyTorch evaluates in float32."""
    return (maximum.astype(np.float32) * np.float32(alpha)).astype(np.float32)


def _protected(query_blocks, key_blocks, sink, window, last):
    query_ids = np.arange(query_blocks).reshape(1, -1, 1, 1)
    key_ids = np.arange(key_blocks).reshape(1, 1, -1, 1)
    distance = query_ids - key_ids
    protected = (
        (key_ids < sink)
        | ((distance >= 0) & (distance < window))
        | (query_ids >= query_blocks - last)
    )
    return protected, distance >= 0


def deal_output_score(score: np.ndarray, attention_sink: int, window: int,
                      alpha: float = 0.1, last_n_blocks_full: int = 2,
                      min_budget: int = 0):
    """V1 threshold + protected selection with sorted indices.

    upstream/flashprefill_native_forward.py:357-407: keep = score >= max_j score *
    alpha; protected = sink | window | last query blocks; active = (keep |
    protected) & causal; indices = ascending active key ids padded with
    key_blocks (int64); counts int32. ``min_budget > 0`` additionally keeps the
    ``min_budget`` largest scores (ties broken toward the lower key id).
    """
    score = np.asarray(score, dtype=np.float32)
    batch, query_blocks, key_blocks, heads = score.shape
    with np.errstate(invalid="ignore"):
        maximum = score.max(axis=2, keepdims=True)
        keep = score >= _threshold(maximum, alpha)
        if min_budget > 0:
            order = np.argsort(-score, axis=2, kind="stable")[:, :, :min_budget]
            np.put_along_axis(keep, order, True, axis=2)
    protected, causal = _protected(query_blocks, key_blocks, attention_sink, window,
                                   last_n_blocks_full)
    active = (keep | protected) & causal
    return indices_from_mask(active)


def protected_selection(scores: np.ndarray, alpha: float, sink_blocks: int,
                        window_blocks: int, last_full_blocks: int) -> np.ndarray:
    """kernels.py:129-151: alpha == 0 selects every causal block; otherwise
    routed = score > 0 & score >= alpha * max, united with the protected set,
    intersected with causality."""
    scores = np.asarray(scores, dtype=np.float32)
    batch, query_blocks, key_blocks, heads = scores.shape
    protected, causal = _protected(query_blocks, key_blocks, sink_blocks, window_blocks,
                                   last_full_blocks)
    if alpha == 0:
        return np.broadcast_to(causal, scores.shape).copy()
    with np.errstate(invalid="ignore"):
        maximum = scores.max(axis=2, keepdims=True)
        routed = (scores > 0) & (scores >= _threshold(maximum, alpha))
    return (routed | protected) & causal


def indices_from_mask(selected: np.ndarray):
    """kernels.py:154-160: ascending key ids with sentinel key_blocks; int32 counts."""
    selected = np.asarray(selected, dtype=bool)
    key_blocks = selected.shape[2]
    key_ids = np.arange(key_blocks, dtype=np.int64).reshape(1, 1, -1, 1)
    indices = np.sort(np.where(selected, key_ids, key_blocks), axis=2).astype(np.int64)
    counts = selected.sum(axis=2).astype(np.int32)
    return indices, counts


def mask_from_indices(indices: np.ndarray, counts: np.ndarray) -> np.ndarray:
    """kernels.py:163-176: mark the first ``counts`` listed key blocks."""
    batch, query_blocks, key_blocks, heads = indices.shape
    positions = np.arange(key_blocks).reshape(1, 1, -1, 1)
    valid = positions < counts[:, :, None, :]
    full = np.zeros((batch, query_blocks, key_blocks + 1, heads), dtype=bool)
    b, t, p, h = np.nonzero(valid)
    full[b, t, indices[b, t, p, h], h] = True
    return full[:, :, :key_blocks]


# -------------------------------------------------------------- new selectors

def selector_scores(q: np.ndarray, descriptors: BlockDescriptors, scale: float,
                    selector: str, block_size: int = BLOCK_SIZE, precision: str = "f64",
                    tiles=None):
    """Balanced / CGF / dispersion block scores (kernels.py:49-126).

    Per real row r of tile t and head h, over visible blocks j < t:
    l0 = scale * q.mu_K + ln n_j ; u = max(0, scale^2 * q^2 . var_K);
    logits = l0 (balanced) or l0 + u / 2 (cgf, dispersion); p = softmax_j;
    contribution = p, or p * sqrt(u) * sigma_V (dispersion); score[t, j] is the
    mean of the contributions over the tile's real rows (0 for j >= t).
    ``tiles`` restricts the work to the rows of the given query tiles: a tile's
    scores depend only on its own rows, so those tiles' scores are exact and the
    other tiles' stay 0.
    """
    if selector not in SELECTORS:
        raise ValueError(f"unsupported selector: {selector}")
    acc = _acc(precision)
    batch, sequence, q_heads, _ = q.shape
    blocks = descriptors.mean_k.shape[1]
    group = q_heads // descriptors.mean_k.shape[2]
    log_counts = np.log(descriptors.counts.astype(np.float32)).astype(acc)
    rows = np.arange(sequence)
    if tiles is not None:
        rows = np.concatenate([np.arange(t * block_size, min(sequence, (t + 1) * block_size))
                               for t in sorted(set(tiles))])
    row_tiles = rows // block_size
    visible = np.arange(blocks)[None, :] < row_tiles[:, None]          # [rows, NB]
    tile_rows = np.bincount(row_tiles, minlength=blocks).astype(acc)
    tile_rows = np.where(tile_rows > 0, tile_rows, 1)
    scores = np.zeros((batch, blocks, blocks, q_heads), dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        for b in range(batch):
            for h in range(q_heads):
                g = h // group
                query = q[b, rows, h].astype(acc)
                ell0 = query @ descriptors.mean_k[b, :, g].astype(acc).T * acc(scale)
                ell0 = ell0 + log_counts[None, :]
                if selector == "mean_balanced":
                    logits, dispersion = ell0, None
                else:
                    u = (query * query) @ descriptors.var_k[b, :, g].astype(acc).T
                    u = np.maximum(u * acc(scale * scale), 0)
                    logits = ell0 + 0.5 * u
                    dispersion = np.sqrt(u) if selector == "dispersion_mean" else None
                masked = np.where(visible, logits, -np.inf)
                row_max = masked.max(axis=1, keepdims=True)
                row_max = np.where(np.isfinite(row_max), row_max, 0)
                expo = np.where(visible, np.exp(masked - row_max), 0)
                probability = expo / np.where(visible.any(axis=1, keepdims=True),
                                              expo.sum(axis=1, keepdims=True), 1)
                if dispersion is not None:
                    contribution = probability * dispersion \
                        * descriptors.sigma_v[b, :, g].astype(acc)[None, :]
                else:
                    contribution = probability
                aggregate = np.zeros((blocks, blocks), dtype=acc)
                np.add.at(aggregate, row_tiles, contribution)
                scores[b, :, :, h] = (aggregate / tile_rows[:, None]).astype(np.float32)
    return scores


# ---------------------------------------------------------- exact attention

def exact_attention(q, k, v, indices, counts, scale, block_size: int = BLOCK_SIZE,
                    precision: str = "f64", tiles=None):
    """Block-sparse causal attention over each (query tile, head)'s index list.

    upstream/flashprefill_native_forward.py:215-354 (``_flash_forward``) and
    :478-521 (``exact_attention``): for query tile t the keys are the listed
    blocks (in list order, first ``counts`` entries); keys past the sequence end
    read as zero; causality is applied only inside the block equal to t. Output
    is rounded to bf16; LSE is the natural-log log-sum-exp (float32). A count
    of zero gives output 0 and LSE -inf (the kernel's denominator starts at 1).
    List entries outside [0, key_blocks) are skipped.

    ``tiles`` restricts the work to the given query tiles (others stay 0 / -inf):
    the CPU baseline uses it to time a bounded sample.
    """
    acc = _acc(precision)
    batch, sequence, q_heads, dim = q.shape
    blocks = num_blocks(sequence, block_size)
    kp = _pad_blocks(k, block_size)
    vp = _pad_blocks(v, block_size)
    kv_heads = k.shape[2]
    group = q_heads // kv_heads
    out = np.zeros(q.shape, dtype=np.float32)
    lse = np.full((batch, sequence, q_heads), -np.inf, dtype=np.float32)
    tile_ids = range(blocks) if tiles is None else tiles
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        for b in range(batch):
            for t in tile_ids:
                row0, row1 = t * block_size, min(sequence, (t + 1) * block_size)
                rows = row1 - row0
                query_pos = np.arange(row0, row1)
                for g in range(kv_heads):
                    # heads of the group that share one list are evaluated together
                    by_list = {}
                    for h in range(g * group, (g + 1) * group):
                        count = max(int(counts[b, t, h]), 0)
                        listed = tuple(int(j) for j in indices[b, t, :count, h]
                                       if 0 <= int(j) < blocks)
                        by_list.setdefault(listed, []).append(h)
                    for listed, heads in by_list.items():
                        if not listed:
                            continue
                        keys = kp[b, list(listed), :, g].reshape(-1, dim).astype(acc)
                        values = vp[b, list(listed), :, g].reshape(-1, dim).astype(acc)
                        key_pos = (np.asarray(listed)[:, None] * block_size
                                   + np.arange(block_size)[None, :]).reshape(-1)
                        diag_cols = np.nonzero(np.repeat(np.asarray(listed) == t, block_size))[0]
                        query = q[b, row0:row1][:, heads].transpose(1, 0, 2).reshape(-1, dim)
                        logits = query.astype(acc) @ keys.T
                        logits *= acc(scale)
                        logits = logits.reshape(len(heads), rows, -1)
                        if diag_cols.size:
                            masked = key_pos[diag_cols][None, :] > query_pos[:, None]
                            sub = logits[:, :, diag_cols]
                            sub[:, masked] = -np.inf
                            logits[:, :, diag_cols] = sub
                        row_max = logits.max(axis=2, keepdims=True)
                        logits -= row_max
                        weights = np.exp(logits, out=logits)
                        total = weights.sum(axis=2, keepdims=True)
                        result = (weights.reshape(-1, weights.shape[2]) @ values).reshape(
                            len(heads), rows, dim) / total
                        out[b, row0:row1][:, heads] = result.transpose(1, 0, 2).astype(np.float32)
                        lse[b, row0:row1][:, heads] = (row_max[..., 0] + np.log(total[..., 0])
                                                       ).T.astype(np.float32)
    return bf16_round(out), lse


# ------------------------------------------------------ mean tail and merge

def mean_tail(q, descriptors: BlockDescriptors, selected, scale,
              block_size: int = BLOCK_SIZE, precision: str = "f64", tiles=None):
    """Unselected full-history block-mean path (kernels.py:179-230).

    Row r of tile t, head h: tail = {j < t : not selected[t, j, h]};
    logits = scale * q.mu_K,j + ln n_j; LSE over the tail (-inf if empty);
    output = softmax-weighted mu_V (0 if empty). Float32 outputs. ``tiles``
    restricts the rows computed (others stay 0 / -inf).
    """
    acc = _acc(precision)
    batch, sequence, q_heads, dim = q.shape
    blocks = descriptors.mean_k.shape[1]
    group = q_heads // descriptors.mean_k.shape[2]
    log_counts = np.log(descriptors.counts.astype(np.float32)).astype(acc)
    rows = np.arange(sequence)
    if tiles is not None:
        rows = np.concatenate([np.arange(t * block_size, min(sequence, (t + 1) * block_size))
                               for t in tiles])
    row_tiles = rows // block_size
    visible = np.arange(blocks)[None, :] < row_tiles[:, None]
    out = np.zeros((batch, sequence, q_heads, dim), dtype=np.float32)
    lse = np.full((batch, sequence, q_heads), -np.inf, dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        for b in range(batch):
            for h in range(q_heads):
                g = h // group
                tail = visible & ~np.asarray(selected[b, row_tiles, :, h], dtype=bool)
                logits = q[b, rows, h].astype(acc) @ descriptors.mean_k[b, :, g].astype(acc).T
                logits = logits * acc(scale) + log_counts[None, :]
                masked = np.where(tail, logits, -np.inf)
                row_max = masked.max(axis=1, keepdims=True)
                finite = np.isfinite(row_max)
                safe = np.where(finite, row_max, 0)
                weights = np.where(tail, np.exp(masked - safe), 0)
                total = weights.sum(axis=1, keepdims=True)
                row_lse = np.where(finite, safe + np.log(np.where(finite, total, 1)), -np.inf)
                weights = weights / np.where(finite, total, 1)
                out[b, rows, h] = (weights @ descriptors.mean_v[b, :, g].astype(acc)).astype(np.float32)
                lse[b, rows, h] = row_lse[:, 0].astype(np.float32)
    return out, lse


def merge_exact_mean(exact_output, exact_lse, mean_output, mean_lse):
    """kernels.py:312-325: logaddexp merge; output rounded to bf16."""
    with np.errstate(invalid="ignore"):
        total = np.logaddexp(exact_lse.astype(np.float32), mean_lse.astype(np.float32))
        exact_weight = np.exp(exact_lse - total)
        mean_weight = np.exp(mean_lse - total)
        output = (exact_output.astype(np.float32) * exact_weight[..., None]
                  + mean_output.astype(np.float32) * mean_weight[..., None])
    return bf16_round(output.astype(np.float32)), total.astype(np.float32)


# ------------------------------------------------------------ rescue tail

def tile_mean_query(q, block_size: int = BLOCK_SIZE, precision: str = "f64"):
    """Mean query of every query tile over its real rows, float32
    ``[B, NB, Hq, D]`` (kernels.py:274-276: sum over the tile / real row count)."""
    acc = _acc(precision)
    batch, sequence, q_heads, dim = q.shape
    blocks = num_blocks(sequence, block_size)
    out = np.zeros((batch, blocks, q_heads, dim), dtype=np.float32)
    for t in range(blocks):
        rows = q[:, t * block_size:min(sequence, (t + 1) * block_size)].astype(acc)
        out[:, t] = (rows.sum(axis=1) / acc(rows.shape[1])).astype(np.float32)
    return out


def rescue_choice(q, k, block_size: int = BLOCK_SIZE, precision: str = "f64"):
    """Rescue token of every (query tile t, key block j < t, q head):
    argmax over the block's 128 positions of qbar_t . k (kernels.py:277-283), the
    first position on ties (torch.argmax). uint8 ``[B, NB, NB, Hq]`` (0 for j >= t).
    Positions past the sequence end hold zero keys, as the reference's padding."""
    acc = _acc(precision)
    batch, sequence, q_heads, dim = q.shape
    kv_heads = k.shape[2]
    group = q_heads // kv_heads
    blocks = num_blocks(sequence, block_size)
    qbar = tile_mean_query(q, block_size, precision).astype(acc)
    kb = _pad_blocks(k, block_size).astype(acc)          # [B, NB, blk, Hkv, D]
    choice = np.zeros((batch, blocks, blocks, q_heads), dtype=np.uint8)
    for b in range(batch):
        for h in range(q_heads):
            g = h // group
            # scores[t, j, pos] = qbar[t] . k[j, pos]
            scores = np.einsum("td,jpd->tjp", qbar[b, :, h], kb[b, :, :, g])
            if precision == "f32":
                scores = scores.astype(np.float32)
            best = scores.argmax(axis=2)                    # first maximum on ties
            causal = np.arange(blocks)[None, :] < np.arange(blocks)[:, None]
            choice[b, :, :, h] = np.where(causal, best, 0).astype(np.uint8)
    return choice


def rescue_tail(q, k, v, selected, scale, block_size: int = BLOCK_SIZE, remainder: bool = False,
                precision: str = "f64", tiles=None, choice=None):
    """Exact attention to one rescue token per unselected full-history block
    (kernels.py:233-309), in float32 outputs.

    Row r of tile t, head h, tail = {j < t : not selected[t, j, h]}: entry j is the
    block's rescue token (``rescue_choice``) with logit scale * q.k_tok and value
    v_tok; with ``remainder`` block j adds a second entry, the mean K / V of its
    other B - 1 tokens, with logit scale * q.k_rest + ln(B - 1). Returns the
    softmax-weighted output and the natural-log LSE over these entries (0 / -inf
    for an empty tail). ``choice`` may be given (the GPU's), to test the attention
    part on identical tokens.
    """
    acc = _acc(precision)
    batch, sequence, q_heads, dim = q.shape
    kv_heads = k.shape[2]
    group = q_heads // kv_heads
    blocks = num_blocks(sequence, block_size)
    if choice is None:
        choice = rescue_choice(q, k, block_size, precision)
    kb = _pad_blocks(k, block_size).astype(acc)
    vb = _pad_blocks(v, block_size).astype(acc)
    rows = np.arange(sequence)
    if tiles is not None:
        rows = np.concatenate([np.arange(t * block_size, min(sequence, (t + 1) * block_size))
                               for t in tiles])
    out = np.zeros((batch, sequence, q_heads, dim), dtype=np.float32)
    lse = np.full((batch, sequence, q_heads), -np.inf, dtype=np.float32)
    log_rest = acc(math.log(block_size - 1))
    for b in range(batch):
        for h in range(q_heads):
            g = h // group
            for t in sorted(set((rows // block_size).tolist())):
                tail = [j for j in range(t) if not selected[b, t, j, h]]
                r = rows[(rows // block_size) == t]
                if not tail:
                    continue
                tok = choice[b, t, tail, h].astype(np.int64)
                keys = kb[b, tail, tok, g]                     # [n, D]
                values = vb[b, tail, tok, g]
                logits = (q[b, r, h].astype(acc) @ keys.T) * acc(scale)
                if remainder:
                    k_rest = (kb[b, tail, :, g].sum(axis=1) - keys) / acc(block_size - 1)
                    v_rest = (vb[b, tail, :, g].sum(axis=1) - values) / acc(block_size - 1)
                    rest = (q[b, r, h].astype(acc) @ k_rest.T) * acc(scale) + log_rest
                    logits = np.concatenate([logits, rest], axis=1)
                    values = np.concatenate([values, v_rest], axis=0)
                row_max = logits.max(axis=1, keepdims=True)
                weights = np.exp(logits - row_max)
                total = weights.sum(axis=1, keepdims=True)
                lse[b, r, h] = (row_max + np.log(total))[:, 0].astype(np.float32)
                out[b, r, h] = ((weights / total) @ values).astype(np.float32)
    return out, lse


# --------------------------------------------------------------- accounting

def selection_accounting(selected, sequence, q_tile_size, k_tile_size, method,
                         score_k_tile_size, block_size: int = BLOCK_SIZE):
    """kernels.py:328-407, as plain integers / floats."""
    selected = np.asarray(selected, dtype=bool)
    batch, blocks, _, heads = selected.shape
    counts = block_counts(sequence, block_size).astype(np.int64)
    query_ids = np.arange(blocks).reshape(-1, 1)
    key_ids = np.arange(blocks).reshape(1, -1)
    history = counts.reshape(-1, 1) * counts.reshape(1, -1)
    diagonal = counts * (counts + 1) // 2
    weights = np.where(key_ids < query_ids, history,
                       np.where(key_ids == query_ids, diagonal.reshape(-1, 1), 0))
    exact_pairs = int((selected.astype(np.int64) * weights.reshape(1, blocks, blocks, 1)).sum())
    total_pairs = batch * heads * sequence * (sequence + 1) // 2
    causal_blocks = batch * heads * blocks * (blocks + 1) // 2
    selected_blocks = int(selected.sum())
    full_history = key_ids < query_ids
    tail = full_history.reshape(1, blocks, blocks, 1) & ~selected
    mean_proxy = int((tail.astype(np.int64) * counts.reshape(1, blocks, 1, 1)).sum())
    selector_proxy = int((full_history.astype(np.int64) * counts.reshape(blocks, 1)).sum()) \
        * batch * heads
    physical = None
    if q_tile_size is not None and k_tile_size is not None:
        q_programs = (counts + q_tile_size - 1) // q_tile_size
        physical = int((selected.astype(np.int64) * q_programs.reshape(1, blocks, 1, 1)
                        * math.ceil(block_size / k_tile_size)).sum())
    mean_method = method in MEAN_METHODS | {"fp_v1_rescue", "fp_v1_rescue_v2"}
    executed_mean = batch * sequence * heads * blocks if mean_method else 0
    selector_executed = 0
    selector_physical = None
    if method in SELECTORS:
        selector_executed = batch * sequence * heads * blocks * (1 if method == "mean_balanced" else 2)
    elif method in V1_ROUTED | {"fp_v1_rescue", "fp_v1_rescue_v2"} and score_k_tile_size is not None:
        selector_physical = sum(math.ceil((t + 1) / score_k_tile_size) for t in range(blocks)) \
            * batch * heads
        selector_executed = selector_physical * score_k_tile_size * block_size
    return {
        "effective_exact_token_pair_ratio": exact_pairs / total_pairs,
        "exact_token_pairs": exact_pairs,
        "causal_token_pairs": total_pairs,
        "legacy_block_density": selected_blocks / causal_blocks,
        "selected_block_entries": selected_blocks,
        "causal_block_entries": causal_blocks,
        "exact_physical_qk_tiles": physical,
        "mean_proxy_entries": mean_proxy,
        "selector_proxy_entries": selector_proxy,
        "mean_executed_logit_entries": executed_mean,
        "mean_executed_value_entries": executed_mean,
        "selector_executed_dot_entries": selector_executed,
        "selector_physical_qk_tiles": selector_physical,
        "q_tile_size": q_tile_size,
        "k_tile_size": k_tile_size,
        "score_k_tile_size": score_k_tile_size,
    }


# -------------------------------------------------------- whole-layer path

def attention_layer(q, k, v, scale, method, alpha=0.08, sink=2, window=4, last=2,
                    block_size: int = BLOCK_SIZE, precision: str = "f64", tiles=None):
    """One prefill attention call for ``method`` (attention.py:154-339).

    Returns a dict with ``output`` (bf16-rounded float32, ``[B, S, Hq, D]``),
    and the intermediate ``indices``, ``counts``, ``selected`` and ``scores``
    (None for dense). ``tiles`` restricts the attention to a sample of query
    tiles (CPU baseline only).
    """
    if method not in METHODS:
        raise ValueError(f"unknown method {method!r}; choose from {METHODS}")
    batch, sequence, q_heads, _ = q.shape
    blocks = num_blocks(sequence, block_size)
    result = {"scores": None, "indices": None, "counts": None, "selected": None}
    if method == "dense":
        selected = np.broadcast_to(
            (np.arange(blocks)[None, :, None, None] >= np.arange(blocks)[None, None, :, None]),
            (batch, blocks, blocks, q_heads))
        indices, counts = indices_from_mask(selected)
        out, lse = exact_attention(q, k, v, indices, counts, scale, block_size, precision, tiles)
        result.update(output=out, lse=lse)
        return result
    descriptors = None
    if method in V1_ROUTED:
        if method == "mean_native":
            descriptors = block_descriptors(k, v, block_size, precision)
        kbar = block_mean_k(k, block_size, precision)
        scores = v1_scores(q, kbar, scale, block_size, precision)
        indices, counts = deal_output_score(scores, sink, window, alpha, last, 0)
        selected = mask_from_indices(indices, counts)
    else:
        descriptors = block_descriptors(k, v, block_size, precision)
        if alpha == 0:
            scores = np.zeros((batch, blocks, blocks, q_heads), dtype=np.float32)
        else:
            scores = selector_scores(q, descriptors, scale, method, block_size, precision)
        selected = protected_selection(scores, alpha, sink, window, last)
        indices, counts = indices_from_mask(selected)
    out, lse = attention_from_selection(q, k, v, scale, method, selected, descriptors,
                                        block_size=block_size, precision=precision, tiles=tiles)
    result.update(output=out, lse=lse, scores=scores, indices=indices, counts=counts,
                  selected=selected)
    return result


def attention_from_selection(q, k, v, scale, method, selected, descriptors=None, choice=None,
                             block_size: int = BLOCK_SIZE, precision: str = "f64", tiles=None):
    """The attention half of a prefill call (attention.py:253-333) for a given
    selection mask: exact attention over ``indices_from_mask(selected)``, then the
    block-mean tail + merge (mean methods; ``descriptors`` computed when None) or
    the rescue tail + merge (rescue methods; ``choice`` computed when None).
    Returns (output, LSE); ``tiles`` restricts the work to those query tiles."""
    indices, counts = indices_from_mask(selected)
    out, lse = exact_attention(q, k, v, indices, counts, scale, block_size, precision, tiles)
    if method in MEAN_METHODS:
        if descriptors is None:
            descriptors = block_descriptors(k, v, block_size, precision)
        mean_out, mean_lse = mean_tail(q, descriptors, selected, scale, block_size, precision,
                                       tiles=tiles)
        out, lse = merge_exact_mean(out, lse, mean_out, mean_lse)
    elif method in RESCUE_METHODS:
        r_out, r_lse = rescue_tail(q, k, v, selected, scale, block_size,
                                   remainder=method == "fp_v1_rescue_v2", precision=precision,
                                   tiles=tiles, choice=choice)
        out, lse = merge_exact_mean(out, lse, r_out, r_lse)
    return out, lse
