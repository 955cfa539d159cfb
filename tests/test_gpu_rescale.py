"""Lazy rescale paths of the attention kernels.

The keys of block j are c_j u plus noise and every query is 4 u plus noise (u a
unit direction per kv group), so a key block's scores sit near 0.51 c_j in log2
units. Step patterns of c_j make the running max jump by about 70 to 100 log2
units from one block to the next (rising, rising then falling, alternating),
beyond the kernels' 2^64 lazy headroom, so the full-block pipeline takes its
rare rescale branch at block after block, and the masked diagonal path at the
end sees maxima below, near and above the running one. All causal blocks are
listed; outputs and LSE are compared with the oracle."""

import numpy as np
import pytest
import torch

from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import assert_output_close, to_np

pytestmark = pytest.mark.gpu

LENGTH = 1089   # 9 blocks, the last one partial


def _pattern(name, blocks):
    j = np.arange(blocks)
    if name == "rising":
        return 2.0 + 160.0 * j
    if name == "peak":
        return 2.0 + 192.0 * np.minimum(j, blocks - 1 - j)
    return 2.0 + 192.0 * (j % 2)         # alternating


def _inputs(name, q_heads, kv_heads, dim, seed):
    rng = np.random.default_rng(seed)
    blocks = ref.num_blocks(LENGTH)
    u = rng.standard_normal((kv_heads, dim))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    # same log2 steps at every head dim (the score scale is dim ** -0.5)
    c = np.repeat(_pattern(name, blocks), 128)[:LENGTH] * np.sqrt(dim / 128)
    group = q_heads // kv_heads
    q = 4.0 * np.repeat(u, group, axis=0)[None, None] + 0.3 * rng.standard_normal((1, LENGTH, q_heads, dim))
    k = c[None, :, None, None] * u[None, None] + 0.3 * rng.standard_normal((1, LENGTH, kv_heads, dim))
    v = rng.standard_normal((1, LENGTH, kv_heads, dim))
    to = lambda x: torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    return to(q), to(k), to(v)


@pytest.mark.parametrize("pattern", ("rising", "peak", "alternating"))
@pytest.mark.parametrize("shape", ((28, 4, 128), (16, 4, 256)))
def test_exact_attention_rescale_patterns(gpu, pattern, shape):
    q_heads, kv_heads, dim = shape
    q, k, v = _inputs(pattern, q_heads, kv_heads, dim, seed=101)
    scale = dim ** -0.5
    blocks = ref.num_blocks(LENGTH)
    sel = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[None, :, :, None],
                          (1, blocks, blocks, q_heads))
    idx, cnt = ref.indices_from_mask(sel)
    out, lse = up.exact_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(idx).cuda(),
                                  torch.from_numpy(cnt).cuda(), scale)
    e_out, e_lse = ref.exact_attention(to_np(q), to_np(k), to_np(v), idx, cnt, scale)
    # the jumps are real: neighbouring blocks' score maxima differ by more than the
    # kernels' 2^64 headroom
    x = to_np(q)[0, -1, 0] @ to_np(k)[0, :blocks * 128 - 128 + 1:128, 0].T * scale / np.log(2)
    assert np.abs(np.diff(x)).max() > 64.0
    assert_output_close(to_np(out), e_out, what=f"{pattern} d={dim}")
    np.testing.assert_allclose(to_np(lse), e_lse, atol=0.02, rtol=0.01)
