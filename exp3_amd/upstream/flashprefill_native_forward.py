"""MI355X implementation of the FlashPrefill V1 stage functions.

Same names, signatures, dtypes and layouts as the reference module
``upstream/flashprefill_native_forward.py`` (all tensors ``[batch, sequence,
heads, dim]``); each function enqueues hand-written gfx950 HIP kernels through
the C ABI on the current stream. Tensors must be on a ROCm GPU.
"""

from __future__ import annotations

import torch

from .. import _lib

SCORE_IMPL = "v1_kmean_qt_row_reduce"
LSE_IMPL = "natural_log_exact_lse"

# Fixed launch geometry of the HIP kernels (the reference autotunes; these are
# what its introspection helpers report here).
ATTENTION_Q_TILE = 128   # query rows per workgroup
ATTENTION_K_TILE = 128   # keys per LDS tile
SCORE_K_TILE = 32        # key blocks per score MFMA chunk


class LaunchConfig:
    """What a Triton autotuner's ``best_config`` exposes (``kwargs``,
    ``num_warps``, ``num_stages``), describing a fixed HIP launch: ``num_warps``
    is wavefronts (64 lanes) per workgroup, ``num_stages`` the LDS buffers a key
    tile streams through."""

    def __init__(self, num_warps: int, num_stages: int, **kwargs):
        self.kwargs = dict(kwargs)
        self.num_warps = num_warps
        self.num_stages = num_stages

    def __repr__(self):
        return (f"LaunchConfig({self.kwargs}, num_warps={self.num_warps}, "
                f"num_stages={self.num_stages})")


class KernelInfo:
    """Stand-in for a reference Triton kernel object, read only for its
    ``best_config`` (check_qwen35_math.py:134-139, upstream :524-533)."""

    def __init__(self, name: str, best_config: LaunchConfig):
        self.__name__ = name
        self.best_config = best_config


# head dim -> attention kernel geometry: d = 128 runs two 128-row query tiles per
# 8-wave workgroup over 128-key tiles (double-buffered); d = 256 one tile per
# 4-wave workgroup over 32-key sub-blocks (double-buffered)
_ATTENTION_CONFIGS = {
    128: LaunchConfig(8, 2, Q_TILE_SIZE=ATTENTION_Q_TILE, K_TILE_SIZE=ATTENTION_K_TILE),
    256: LaunchConfig(4, 2, Q_TILE_SIZE=ATTENTION_Q_TILE, K_TILE_SIZE=32),
}

# ``best_config`` follows the head dim of the last exact_attention launch (d = 128
# until a d = 256 launch), as the reference's reflects its last autotuned launch.
_flash_forward = KernelInfo("attn_kernel", _ATTENTION_CONFIGS[128])
compute_block_score = KernelInfo(
    "v1_route_kernel", LaunchConfig(4, 4, Q_TILE_SIZE=128, K_TILE_SIZE=SCORE_K_TILE))


def _blocks(sequence: int, block_size: int) -> int:
    return (sequence + block_size - 1) // block_size


@torch.no_grad()
def block_mean_k(k: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """bf16 mean of K over each block's valid tokens, ``[B, NB, Hkv, D]``.

    Reference: upstream/flashprefill_native_forward.py:420-442.
    """
    device = _lib.require_gpu(k)
    k = _lib.kernel_view(k)
    batch, sequence, kv_heads, head_dim = k.shape
    mean = torch.empty(batch, _blocks(sequence, block_size), kv_heads, head_dim,
                       dtype=k.dtype, device=device)
    _lib.call("spx_block_mean_k", _lib.ptr(k), _lib.strides(k), batch, sequence, kv_heads,
              head_dim, block_size, _lib.ptr(mean), _lib.stream(device))
    return mean


@torch.no_grad()
def v1_scores(q: torch.Tensor, mean_k: torch.Tensor, scale: float,
              block_size: int = 128) -> torch.Tensor:
    """Normalised V1 block scores ``[B, NB, NB, Hq]`` (fp32).

    Reference: upstream/flashprefill_native_forward.py:445-475 (the block score
    kernel plus ``normalize_scores``, fused into one HIP kernel).
    """
    device = _lib.require_gpu(q, mean_k)
    q = _lib.kernel_view(q)
    mean_k = _lib.kernel_view(mean_k)
    batch, sequence, q_heads, head_dim = q.shape
    blocks = mean_k.shape[1]
    if blocks != _blocks(sequence, block_size):
        raise ValueError(f"mean_k has {blocks} blocks, expected {_blocks(sequence, block_size)}")
    if mean_k.shape[0] != batch or mean_k.shape[3] != head_dim or q_heads % mean_k.shape[2]:
        raise ValueError(f"mean_k shape {tuple(mean_k.shape)} does not match q {tuple(q.shape)}")
    score = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.float32, device=device)
    _lib.call("spx_v1_scores", _lib.ptr(q), _lib.strides(q), _lib.ptr(mean_k),
              _lib.strides(mean_k), batch, sequence, q_heads, mean_k.shape[2], head_dim,
              block_size, float(scale), _lib.ptr(score), _lib.strides(score),
              _lib.stream(device))
    return score


def deal_output_score(score: torch.Tensor, attention_sink: int, window: int,
                      alpha: float = 0.1, last_n_blocks_full: int = 2, min_budget: int = 0):
    """V1 threshold + protected selection -> (indices int64, counts int32).

    Reference: upstream/flashprefill_native_forward.py:357-407. Outputs are fresh
    tensors (no buffer reuse across calls).
    """
    device = _lib.require_gpu(score)
    if score.dtype != torch.float32 or score.dim() != 4:
        raise ValueError("score must be a float32 [batch, query_block, key_block, head] tensor")
    batch, query_blocks, key_blocks, heads = score.shape
    indices = torch.empty(batch, query_blocks, key_blocks, heads, dtype=torch.int64, device=device)
    counts = torch.empty(batch, query_blocks, heads, dtype=torch.int32, device=device)
    _lib.call("spx_deal_output_score", _lib.ptr(score), _lib.strides(score), batch,
              query_blocks, key_blocks, heads, int(attention_sink), int(window), float(alpha),
              int(last_n_blocks_full), int(min_budget), _lib.ptr(indices), _lib.ptr(counts),
              None, _lib.stream(device))
    return indices, counts


def attention_tiles(k: torch.Tensor, v: torch.Tensor, block_size: int = 128):
    """Per-block K and V tiles the attention kernel copies into LDS verbatim:
    key tiles ``[B, Hkv, NB, 128, D]`` and value tiles ``[B, Hkv, NB, D, 128]``
    (V transposed, keys permuted; at D = 256 four 32-key sub-blocks
    ``[256, 32]`` per block), zero past the sequence end, 16-byte chunks
    XOR-swizzled by row; produced by the pooling pass."""
    device = _lib.require_gpu(k, v)
    k = _lib.kernel_view(k)
    v = _lib.kernel_view(v)
    batch, sequence, kv_heads, head_dim = v.shape
    blocks = _blocks(sequence, block_size)
    key_tiles = torch.empty(batch, kv_heads, blocks, block_size, head_dim, dtype=torch.bfloat16,
                            device=device)
    value_tiles = torch.empty(batch, kv_heads, blocks, head_dim, block_size, dtype=torch.bfloat16,
                              device=device)
    _lib.call("spx_block_pool", _lib.ptr(k), _lib.strides(k), _lib.ptr(v), _lib.strides(v), batch,
              sequence, kv_heads, head_dim, block_size, None, None, None, None, None, None,
              _lib.ptr(key_tiles), _lib.ptr(value_tiles), _lib.stream(device))
    return key_tiles, value_tiles


@torch.no_grad()
def exact_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    indices: torch.Tensor, counts: torch.Tensor, scale: float,
                    block_size: int = 128):
    """Block-sparse causal attention -> (output bf16 ``[B,S,Hq,D]``, natural LSE fp32).

    Reference: upstream/flashprefill_native_forward.py:478-521.
    """
    device = _lib.require_gpu(q, k, v, indices, counts)
    q = _lib.kernel_view(q)
    k = _lib.kernel_view(k)
    if indices.dtype != torch.int64 or counts.dtype != torch.int32:
        raise ValueError("indices must be int64 and counts int32")
    batch, sequence, q_heads, head_dim = q.shape
    check_attention_shapes(q, k, v, indices, counts, block_size)
    key_tiles, value_tiles = attention_tiles(k, v, block_size)
    if head_dim in _ATTENTION_CONFIGS:
        _flash_forward.best_config = _ATTENTION_CONFIGS[head_dim]
    output = torch.empty(batch, sequence, q_heads, head_dim, dtype=q.dtype, device=device)
    lse = torch.empty(batch, sequence, q_heads, dtype=torch.float32, device=device)
    queue = torch.zeros(_lib.WORK_QUEUE_INTS, dtype=torch.int32, device=device)  # work counters
    _lib.call("spx_exact_attention", _lib.ptr(q), _lib.strides(q), _lib.ptr(key_tiles),
              _lib.ptr(value_tiles), _lib.ptr(indices), _lib.strides(indices), _lib.ptr(counts),
              _lib.strides(counts), batch, sequence, q_heads, k.shape[2], head_dim, block_size,
              float(scale), _lib.ptr(output), _lib.strides(output), _lib.ptr(lse),
              _lib.strides(lse), _lib.ptr(queue), _lib.stream(device))
    return output, lse


def check_attention_shapes(q, k, v, indices, counts, block_size=128):
    """Host-side shape validation: the kernels index these buffers by the
    geometry derived from q."""
    batch, sequence, q_heads, head_dim = q.shape
    blocks = _blocks(sequence, block_size)
    if k.dim() != 4 or k.shape[0] != batch or k.shape[1] != sequence or k.shape[3] != head_dim:
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if v is not None and tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"v shape {tuple(v.shape)} does not match k {tuple(k.shape)}")
    if q_heads % k.shape[2]:
        raise ValueError(f"q heads {q_heads} not a multiple of kv heads {k.shape[2]}")
    if indices is not None and tuple(indices.shape) != (batch, blocks, blocks, q_heads):
        raise ValueError(f"indices shape {tuple(indices.shape)}, expected "
                         f"{(batch, blocks, blocks, q_heads)}")
    if counts is not None and tuple(counts.shape) != (batch, blocks, q_heads):
        raise ValueError(f"counts shape {tuple(counts.shape)}, expected {(batch, blocks, q_heads)}")


def attention_tile_sizes():
    """(query tile, key tile) of the attention kernel (upstream :524-528)."""
    config = _flash_forward.best_config
    return config.kwargs["Q_TILE_SIZE"], config.kwargs["K_TILE_SIZE"]


def score_tile_size():
    """Key blocks per score MFMA chunk (upstream :531-533)."""
    return compute_block_score.best_config.kwargs["K_TILE_SIZE"]
