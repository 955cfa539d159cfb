"""Seeded synthetic attention inputs in the Qwen2.5-7B attention shape.

Q/K/V are drawn i.i.d. N(0, 1) from a CPU generator, RoPE (HF Qwen2 convention:
``rotate_half``, ``emb = cat(freqs, freqs)``, ``inv_freq = theta^(-arange(0, d, 2)/d)``,
positions 0..S-1; see transformers models/qwen2/modeling_qwen2.py and the
reference's block_proxy_validation.py:145-160) is applied to Q and K in fp32, and
the tensors are cast to bf16. Layout ``[batch, sequence, heads, dim]``.

Planted retrieval (needles): ``needles`` key positions drawn uniformly outside
the sink blocks and outside the final query tile's window; at each, every KV
head's key is set (after RoPE) to cosine 0.8 with that head group's mean query
of the final query tile (mean over its rows and q heads) and norm 3x the mean
key norm; values stay N(0, 1).
"""

from __future__ import annotations

import math

import torch

Q_HEADS = 28
KV_HEADS = 4
HEAD_DIM = 128
ROPE_THETA = 1.0e6
SEED = 17


def rope_inv_freq(head_dim: int = HEAD_DIM, theta: float = ROPE_THETA) -> torch.Tensor:
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim
    return 1.0 / (theta ** exponent)


def apply_rope(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    """x: [B, S, H, D] fp32."""
    freqs = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos()[None, :, None, :]
    sin = emb.sin()[None, :, None, :]
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rotated * sin


def make_inputs(sequence: int, seed: int = SEED, q_heads: int = Q_HEADS, kv_heads: int = KV_HEADS,
                head_dim: int = HEAD_DIM, batch: int = 1, theta: float = ROPE_THETA,
                needles: int = 0, block_size: int = 128, sink_blocks: int = 2,
                window_blocks: int = 4, device: str | torch.device = "cpu"):
    """Return (q, k, v) bf16 ``[B, S, H, D]`` and the needle positions (list)."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, sequence, q_heads, head_dim, generator=gen)
    k = torch.randn(batch, sequence, kv_heads, head_dim, generator=gen)
    v = torch.randn(batch, sequence, kv_heads, head_dim, generator=gen)
    positions = torch.arange(sequence)
    inv_freq = rope_inv_freq(head_dim, theta)
    q = apply_rope(q, positions, inv_freq)
    k = apply_rope(k, positions, inv_freq)
    planted = []
    if needles:
        planted = plant_needles(q, k, needles, gen, block_size, sink_blocks, window_blocks)
    to = dict(dtype=torch.bfloat16, device=device)
    return q.to(**to), k.to(**to), v.to(**to), planted


def plant_needles(q, k, count, gen, block_size=128, sink_blocks=2, window_blocks=4):
    """In-place planting into fp32 post-RoPE q / k (see the module docstring)."""
    batch, sequence, q_heads, head_dim = q.shape
    kv_heads = k.shape[2]
    group = q_heads // kv_heads
    blocks = math.ceil(sequence / block_size)
    low = sink_blocks * block_size
    high = max(low + 1, (blocks - 1 - window_blocks + 1) * block_size)
    if high - low < count:
        raise ValueError(f"sequence {sequence} too short for {count} needles")
    positions = (torch.randperm(high - low, generator=gen)[:count] + low).sort().values
    last_rows = slice((blocks - 1) * block_size, sequence)
    mean_norm = k.norm(dim=-1).mean()
    for b in range(batch):
        for g in range(kv_heads):
            qbar = q[b, last_rows, g * group:(g + 1) * group].reshape(-1, head_dim).mean(dim=0)
            u = qbar / qbar.norm().clamp_min(1e-12)
            for p in positions.tolist():
                w = torch.randn(head_dim, generator=gen)
                w = w - (w @ u) * u
                w = w / w.norm().clamp_min(1e-12)
                direction = 0.8 * u + 0.6 * w
                k[b, p, g] = 3.0 * mean_norm * direction
    return positions.tolist()
