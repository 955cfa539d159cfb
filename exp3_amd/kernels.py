"""MI355X implementation of exp3's descriptor / selector / mean-correction stages.

Same names, signatures, dtypes and exceptions as the reference ``kernels.py``;
every tensor function enqueues gfx950 HIP kernels through the C ABI. Tensors
must be on a ROCm GPU; there is no CPU path.
"""

from __future__ import annotations

from dataclasses import dataclass
import math

import torch

from . import _lib

BLOCK_SIZE = 128
SELECTORS = ("mean_balanced", "cgf_mean", "dispersion_mean")
MEAN_ACCOUNTED = {"mean_native", "mean_balanced", "cgf_mean", "dispersion_mean",
                  "fp_v1_rescue", "fp_v1_rescue_v2"}
V1_ACCOUNTED = {"fp_v1", "mean_native", "fp_v1_rescue", "fp_v1_rescue_v2"}


@dataclass
class BlockDescriptors:
    """kernels.py:13-19 (fp32 [B, NB, Hkv, D] moments, [B, NB, Hkv] sigma_v, [NB] counts)."""
    mean_k: torch.Tensor
    mean_v: torch.Tensor
    var_k: torch.Tensor
    sigma_v: torch.Tensor
    counts: torch.Tensor


def _blocks(sequence: int, block_size: int) -> int:
    return (sequence + block_size - 1) // block_size


def _check_descriptors(q: torch.Tensor, d: BlockDescriptors, block_size: int) -> None:
    batch, sequence, q_heads, head_dim = q.shape
    blocks = _blocks(sequence, block_size)
    shape = tuple(d.mean_k.shape)
    if len(shape) != 4 or shape[0] != batch or shape[1] != blocks or shape[3] != head_dim \
            or q_heads % shape[2]:
        raise ValueError(f"descriptor shape {shape} does not match q {tuple(q.shape)}")
    kv = shape[2]
    for name in ("mean_v", "var_k"):
        if tuple(getattr(d, name).shape) != shape:
            raise ValueError(f"descriptor {name} shape {tuple(getattr(d, name).shape)} != {shape}")
    if tuple(d.sigma_v.shape) != (batch, blocks, kv) or tuple(d.counts.shape) != (blocks,):
        raise ValueError("descriptor sigma_v / counts shapes do not match")


def empty_descriptors(batch, blocks, kv_heads, head_dim, device) -> BlockDescriptors:
    f32 = dict(dtype=torch.float32, device=device)
    return BlockDescriptors(
        mean_k=torch.empty(batch, blocks, kv_heads, head_dim, **f32),
        mean_v=torch.empty(batch, blocks, kv_heads, head_dim, **f32),
        var_k=torch.empty(batch, blocks, kv_heads, head_dim, **f32),
        sigma_v=torch.empty(batch, blocks, kv_heads, **f32),
        counts=torch.empty(blocks, dtype=torch.int32, device=device),
    )


@torch.no_grad()
def block_descriptors(k: torch.Tensor, v: torch.Tensor, block_size: int = BLOCK_SIZE):
    """FP32 block moments per KV head (reference kernels.py:22-46)."""
    device = _lib.require_gpu(k, v)
    k = _lib.kernel_view(k)
    v = _lib.kernel_view(v)
    batch, sequence, kv_heads, head_dim = k.shape
    d = empty_descriptors(batch, _blocks(sequence, block_size), kv_heads, head_dim, device)
    _lib.call("spx_block_descriptors", _lib.ptr(k), _lib.strides(k), _lib.ptr(v),
              _lib.strides(v), batch, sequence, kv_heads, head_dim, block_size,
              _lib.ptr(d.mean_k), _lib.ptr(d.mean_v), _lib.ptr(d.var_k), _lib.ptr(d.sigma_v),
              _lib.ptr(d.counts), _lib.stream(device))
    return d


@torch.no_grad()
def selector_scores(q: torch.Tensor, descriptors: BlockDescriptors, scale: float,
                    selector: str, block_size: int = BLOCK_SIZE, chunk_tiles: int = 8):
    """[B, query-block, key-block, Q-head] scores of the three new selectors
    (reference kernels.py:49-126). ``chunk_tiles`` is accepted for signature
    parity; the HIP kernel has no chunk loop."""
    if selector not in SELECTORS:
        raise ValueError(f"unsupported selector: {selector}")
    device = _lib.require_gpu(q, descriptors.mean_k)
    q = _lib.kernel_view(q)
    _check_descriptors(q, descriptors, block_size)
    batch, sequence, q_heads, head_dim = q.shape
    blocks = descriptors.mean_k.shape[1]
    kv_heads = descriptors.mean_k.shape[2]
    mean_k = descriptors.mean_k.contiguous()
    var_k = descriptors.var_k.contiguous()
    sigma_v = descriptors.sigma_v.contiguous()
    counts = descriptors.counts.to(torch.int32).contiguous()
    scores = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.float32, device=device)
    nbytes = _lib.load().spx_selector_workspace_bytes(batch, sequence, kv_heads, head_dim)
    if nbytes < 0:
        raise ValueError(f"selector_scores: unsupported shape {tuple(q.shape)} (head_dim 128 or 256)")
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _lib.call("spx_selector_scores", _lib.ptr(q), _lib.strides(q), _lib.ptr(mean_k),
              _lib.ptr(var_k), _lib.ptr(sigma_v), _lib.ptr(counts), batch, sequence, q_heads,
              kv_heads, head_dim, block_size, _lib.SELECTOR_IDS[selector], float(scale),
              _lib.ptr(workspace), _lib.ptr(scores), _lib.strides(scores), _lib.stream(device))
    return scores


def protected_selection(scores: torch.Tensor, alpha: float, sink_blocks: int,
                        window_blocks: int, last_full_blocks: int,
                        indices: torch.Tensor | None = None,
                        counts: torch.Tensor | None = None) -> torch.Tensor:
    """Threshold + protected regions + causality -> bool mask (kernels.py:129-151).

    Optionally also fills caller-given ``indices`` / ``counts`` (the
    ``indices_from_mask`` lists) in the same launch.
    """
    device = _lib.require_gpu(scores)
    if scores.dtype != torch.float32 or scores.dim() != 4:
        raise ValueError("scores must be a float32 [batch, query_block, key_block, head] tensor")
    batch, query_blocks, key_blocks, heads = scores.shape
    mask = torch.empty(batch, query_blocks, key_blocks, heads, dtype=torch.bool, device=device)
    _lib.call("spx_protected_selection", _lib.ptr(scores), _lib.strides(scores), batch,
              query_blocks, key_blocks, heads, float(alpha), int(sink_blocks),
              int(window_blocks), int(last_full_blocks), _lib.ptr(mask), _lib.ptr(indices),
              _lib.ptr(counts), _lib.stream(device))
    return mask


def indices_from_mask(selected: torch.Tensor):
    """Ascending key ids padded with key_blocks (int64) and int32 counts
    (kernels.py:154-160)."""
    device = _lib.require_gpu(selected)
    selected = selected.contiguous()
    if selected.dtype not in (torch.bool, torch.uint8):
        raise ValueError("selected must be a bool mask")
    batch, query_blocks, key_blocks, heads = selected.shape
    indices = torch.empty(batch, query_blocks, key_blocks, heads, dtype=torch.int64, device=device)
    counts = torch.empty(batch, query_blocks, heads, dtype=torch.int32, device=device)
    _lib.call("spx_indices_from_mask", _lib.ptr(selected), batch, query_blocks, key_blocks, heads,
              _lib.ptr(indices), _lib.ptr(counts), _lib.stream(device))
    return indices, counts


def mask_from_indices(indices: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
    """Bool mask of the first ``counts`` listed key blocks (kernels.py:163-176)."""
    device = _lib.require_gpu(indices, counts)
    indices = indices.to(torch.int64).contiguous()
    counts = counts.to(torch.int32).contiguous()
    batch, query_blocks, key_blocks, heads = indices.shape
    mask = torch.empty(batch, query_blocks, key_blocks, heads, dtype=torch.bool, device=device)
    _lib.call("spx_mask_from_indices", _lib.ptr(indices), _lib.ptr(counts), batch, query_blocks,
              key_blocks, heads, _lib.ptr(mask), _lib.stream(device))
    return mask


@torch.no_grad()
def mean_tail(q: torch.Tensor, descriptors: BlockDescriptors, selected: torch.Tensor,
              scale: float, block_size: int = BLOCK_SIZE, chunk_tiles: int = 8):
    """Unselected full-history block-mean path in FP32 -> (output, LSE)
    (kernels.py:179-230)."""
    device = _lib.require_gpu(q, selected, descriptors.mean_k)
    q = _lib.kernel_view(q)
    _check_descriptors(q, descriptors, block_size)
    batch, sequence, q_heads, head_dim = q.shape
    blocks = _blocks(sequence, block_size)
    if tuple(selected.shape) != (batch, blocks, blocks, q_heads):
        raise ValueError(f"selected shape {tuple(selected.shape)}, expected "
                         f"{(batch, blocks, blocks, q_heads)}")
    indices, counts = indices_from_mask(selected)
    output = torch.empty(batch, sequence, q_heads, head_dim, dtype=torch.float32, device=device)
    lse = torch.empty(batch, sequence, q_heads, dtype=torch.float32, device=device)
    _lib.call("spx_mean_tail", _lib.ptr(q), _lib.strides(q), _lib.ptr(indices),
              _lib.strides(indices), _lib.ptr(counts), _lib.strides(counts),
              _lib.ptr(descriptors.mean_k.contiguous()), _lib.ptr(descriptors.mean_v.contiguous()),
              _lib.ptr(descriptors.counts.to(torch.int32).contiguous()), batch, sequence, q_heads,
              descriptors.mean_k.shape[2], head_dim, block_size, float(scale), _lib.ptr(output),
              _lib.strides(output), _lib.ptr(lse), _lib.strides(lse), _lib.stream(device))
    return output, lse


def _pool_tiles_and_means(k: torch.Tensor, v: torch.Tensor, block_size: int):
    """One spx_block_pool launch -> (key tiles, value tiles, fp32 mean K, fp32 mean V)."""
    device = _lib.require_gpu(k, v)
    k = _lib.kernel_view(k)
    v = _lib.kernel_view(v)
    batch, sequence, kv_heads, head_dim = k.shape
    blocks = _blocks(sequence, block_size)
    key_tiles = torch.empty(batch, kv_heads, blocks, block_size, head_dim, dtype=torch.bfloat16,
                            device=device)
    value_tiles = torch.empty(batch, kv_heads, blocks, head_dim, block_size, dtype=torch.bfloat16,
                              device=device)
    mean_k = torch.empty(batch, blocks, kv_heads, head_dim, dtype=torch.float32, device=device)
    mean_v = torch.empty_like(mean_k)
    _lib.call("spx_block_pool", _lib.ptr(k), _lib.strides(k), _lib.ptr(v), _lib.strides(v), batch,
              sequence, kv_heads, head_dim, block_size, None, _lib.ptr(mean_k), _lib.ptr(mean_v),
              None, None, None, _lib.ptr(key_tiles), _lib.ptr(value_tiles), _lib.stream(device))
    return key_tiles, value_tiles, mean_k, mean_v


def rescue_choice(q: torch.Tensor, key_tiles: torch.Tensor, block_size: int = BLOCK_SIZE):
    """Rescue token of every (query tile t, key block j < t, q head): argmax over the
    block's positions of the tile's mean query . k (kernels.py:274-283), uint8
    ``[B, NB, NB, Hq]`` (0 where j >= t). ``key_tiles`` from the pooling pass."""
    device = _lib.require_gpu(q, key_tiles)
    q = _lib.kernel_view(q)
    batch, sequence, q_heads, head_dim = q.shape
    kv_heads = key_tiles.shape[1]
    blocks = _blocks(sequence, block_size)
    qmean = torch.empty(batch, blocks, q_heads, head_dim, dtype=torch.float32, device=device)
    choice = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.uint8, device=device)
    _lib.call("spx_tile_mean_query", _lib.ptr(q), _lib.strides(q), batch, sequence, q_heads,
              head_dim, block_size, _lib.ptr(qmean), _lib.stream(device))
    _lib.call("spx_rescue_choice", _lib.ptr(qmean), _lib.ptr(key_tiles.contiguous()), batch,
              sequence, q_heads, kv_heads, head_dim, block_size, _lib.ptr(choice),
              _lib.stream(device))
    return choice


@torch.no_grad()
def rescue_tail(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, selected: torch.Tensor,
                scale: float, block_size: int = BLOCK_SIZE, chunk_tiles: int = 8,
                remainder: bool = False):
    """Exact attention to one rescue token per unselected full-history block in
    FP32 -> (output, natural-log LSE) (kernels.py:233-309). Per query tile t and head
    h, the rescue token of block j is argmax_p qbar_{t,h} . k_{j,p}; with
    ``remainder`` the other B-1 tokens of the block also enter through their mean
    K / V with multiplicity B-1. ``chunk_tiles`` is accepted for interface parity
    (the kernel processes every tile in one launch)."""
    device = _lib.require_gpu(q, k, v, selected)
    q = _lib.kernel_view(q)
    batch, sequence, q_heads, head_dim = q.shape
    blocks = _blocks(sequence, block_size)
    if tuple(selected.shape) != (batch, blocks, blocks, q_heads):
        raise ValueError(f"selected shape {tuple(selected.shape)}, expected "
                         f"{(batch, blocks, blocks, q_heads)}")
    key_tiles, value_tiles, mean_k, mean_v = _pool_tiles_and_means(k, v, block_size)
    values = _lib.kernel_view(v)
    choice = rescue_choice(q, key_tiles, block_size)
    indices, counts = indices_from_mask(selected)
    output = torch.empty(batch, sequence, q_heads, head_dim, dtype=torch.float32, device=device)
    lse = torch.empty(batch, sequence, q_heads, dtype=torch.float32, device=device)
    _lib.call("spx_rescue_tail", _lib.ptr(q), _lib.strides(q), _lib.ptr(key_tiles),
              _lib.ptr(value_tiles), _lib.ptr(indices), _lib.strides(indices), _lib.ptr(counts),
              _lib.strides(counts), _lib.ptr(choice), _lib.ptr(values), _lib.strides(values),
              _lib.ptr(mean_k), _lib.ptr(mean_v), int(bool(remainder)), batch, sequence, q_heads,
              k.shape[2], head_dim, block_size,
              float(scale), _lib.ptr(output), _lib.strides(output), _lib.ptr(lse),
              _lib.strides(lse), _lib.stream(device))
    return output, lse


@torch.no_grad()
def merge_exact_mean(exact_output: torch.Tensor, exact_lse: torch.Tensor,
                     mean_output: torch.Tensor, mean_lse: torch.Tensor):
    """logaddexp merge of the exact and mean paths (kernels.py:312-325)."""
    device = _lib.require_gpu(exact_output, exact_lse, mean_output, mean_lse)
    if exact_output.dtype != torch.bfloat16 or mean_output.dtype != torch.float32:
        raise ValueError("exact_output must be bf16 and mean_output float32")
    batch, sequence, heads, head_dim = exact_output.shape
    if tuple(mean_output.shape) != tuple(exact_output.shape) or \
            tuple(exact_lse.shape) != (batch, sequence, heads) or \
            tuple(mean_lse.shape) != (batch, sequence, heads):
        raise ValueError("merge_exact_mean: output / LSE shapes do not match")
    output = torch.empty(batch, sequence, heads, head_dim, dtype=exact_output.dtype, device=device)
    total = torch.empty(batch, sequence, heads, dtype=torch.float32, device=device)
    _lib.call("spx_merge_exact_mean", _lib.ptr(exact_output), _lib.strides(exact_output),
              _lib.ptr(exact_lse), _lib.strides(exact_lse), _lib.ptr(mean_output),
              _lib.strides(mean_output), _lib.ptr(mean_lse), _lib.strides(mean_lse), batch,
              sequence, heads, head_dim, _lib.ptr(output), _lib.strides(output), _lib.ptr(total),
              _lib.strides(total), _lib.stream(device))
    return output, total


def selection_accounting(selected: torch.Tensor, sequence: int, q_tile_size: int | None,
                         k_tile_size: int | None, method: str, score_k_tile_size: int | None,
                         block_size: int = BLOCK_SIZE):
    """Work counters of a selection mask (kernels.py:328-407); scalar GPU tensors,
    read by the caller after its profile forward synchronises."""
    device = _lib.require_gpu(selected)
    selected = selected.contiguous()
    batch, blocks, _, heads = selected.shape
    totals = torch.empty(4, dtype=torch.int64, device=device)
    _lib.call("spx_selection_accounting", _lib.ptr(selected), batch, blocks, heads, int(sequence),
              block_size, int(q_tile_size or 0), _lib.ptr(totals), _lib.stream(device))
    counts = [block_size] * blocks
    counts[-1] = sequence - (blocks - 1) * block_size
    total_pairs = batch * heads * sequence * (sequence + 1) // 2
    causal_blocks = batch * heads * blocks * (blocks + 1) // 2
    selector_proxy = sum(counts[t] * t for t in range(blocks)) * batch * heads
    physical = None
    if q_tile_size is not None and k_tile_size is not None:
        physical = totals[3] * math.ceil(block_size / k_tile_size)
    executed_mean = batch * sequence * heads * blocks if method in MEAN_ACCOUNTED else 0
    selector_executed = 0
    selector_physical = None
    if method in SELECTORS:
        selector_executed = batch * sequence * heads * blocks * (1 if method == "mean_balanced" else 2)
    elif method in V1_ACCOUNTED and score_k_tile_size is not None:
        selector_physical = sum(math.ceil((t + 1) / score_k_tile_size)
                                for t in range(blocks)) * batch * heads
        selector_executed = selector_physical * score_k_tile_size * block_size
    return {
        "effective_exact_token_pair_ratio": totals[0].double() / total_pairs,
        "exact_token_pairs": totals[0],
        "causal_token_pairs": total_pairs,
        "legacy_block_density": totals[1].double() / causal_blocks,
        "selected_block_entries": totals[1],
        "causal_block_entries": causal_blocks,
        "exact_physical_qk_tiles": physical,
        "mean_proxy_entries": totals[2],
        "selector_proxy_entries": selector_proxy,
        "mean_executed_logit_entries": executed_mean,
        "mean_executed_value_entries": executed_mean,
        "selector_executed_dot_entries": selector_executed,
        "selector_physical_qk_tiles": selector_physical,
        "q_tile_size": q_tile_size,
        "k_tile_size": k_tile_size,
        "score_k_tile_size": score_k_tile_size,
    }
