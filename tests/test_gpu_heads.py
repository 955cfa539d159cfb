"""Head configurations other than Qwen2.5-7B's 28 / 4: multi-head (8 / 8), a wider
GQA group count (32 / 8) and an odd group size (12 / 2, group 6). Every method
through the backend against the oracle layer, and the routing mask against the
oracle's (up to threshold ties), at a length whose last block is partial and
whose tile count is odd (a lone last tile pair).

Q and K are scaled by 4 and alpha is 0.7 so that routing drops blocks: with
unscaled random inputs the block-mean proxy is nearly flat and the sink,
window and last-tile protection at 17 blocks keeps every causal block, which
would leave the sparse lists and the mean / rescue tails of these head layouts
untested. Also seeded random layer shapes (batch, length, head layout, method,
alpha) against the oracle layer."""

import numpy as np
import pytest
import torch

from exp3_amd import attention, synthetic
from oracle import reference_cpu as ref
from tests.helpers import (SCALE, assert_output_close, masks_equal_except_ties, threshold_ties,
                           to_np)

pytestmark = pytest.mark.gpu

LENGTH = 2113   # 17 blocks, the last one 65 rows
ALPHA = 0.7


class _Layer:
    layer_idx = 0


def _inputs(q_heads, kv_heads):
    q, k, v, _ = synthetic.make_inputs(LENGTH, seed=83, q_heads=q_heads, kv_heads=kv_heads)
    scaled = lambda x: (x.float() * 4.0).to(torch.bfloat16)
    return scaled(q), scaled(k), v


@pytest.mark.parametrize("heads", ((8, 8), (32, 8), (12, 2)))
@pytest.mark.parametrize("method", attention.METHODS)
def test_methods_other_head_counts(gpu, heads, method):
    q_heads, kv_heads = heads
    q, k, v = _inputs(q_heads, kv_heads)
    backend = attention.AttentionBackend(alpha=ALPHA, register=False)
    backend.configure(method, ALPHA)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    out, _ = backend.forward(_Layer(), qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2),
                             None, SCALE)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, ALPHA)
    assert out.shape == (1, LENGTH, q_heads, 128)
    if expected["selected"] is not None:
        blocks = ref.num_blocks(LENGTH)
        # the case is sparse: some causal (tile, block, head) entries are dropped
        assert expected["selected"].sum() < q_heads * blocks * (blocks + 1) // 2
    if method in attention.V1_ROUTED_METHODS:
        record = {"events": {}}
        _, _, _, _, _, _, sel = backend._route_v1(qg, kg, vg, SCALE, record, False, False)
        unexplained, _, _ = masks_equal_except_ties(to_np(sel), expected["selected"],
                                                     threshold_ties(expected["scores"], ALPHA))
        assert unexplained == 0
    # peaky softmax: outputs reach several units, where one bf16 rounding step is 2^-5
    assert_output_close(to_np(out), expected["output"], what=f"{method} {q_heads}/{kv_heads}",
                        rel=2.0 ** -7)


def _fuzz_cases(n=16, seed=2024):
    """Deterministic random layer shapes: batch, length (partial last blocks, lone
    tiles), head layout, method and alpha."""
    rng = np.random.default_rng(seed)
    layouts = ((4, 1), (6, 3), (8, 2), (12, 4), (28, 4), (16, 16))
    cases = []
    for i in range(n):
        cases.append((int(rng.integers(1, 4)), int(rng.integers(1, 900)),
                      layouts[int(rng.integers(len(layouts)))],
                      attention.METHODS[int(rng.integers(len(attention.METHODS)))],
                      float(rng.choice((0.08, 0.5, 0.7))), 1000 + i))
    return cases


@pytest.mark.parametrize("batch,length,heads,method,alpha,seed", _fuzz_cases())
def test_random_layer_shapes(gpu, batch, length, heads, method, alpha, seed):
    """Seeded random shapes through the backend against the oracle layer (Q, K x 4 so
    that routing drops blocks)."""
    q_heads, kv_heads = heads
    q, k, v, _ = synthetic.make_inputs(length, seed=seed, q_heads=q_heads, kv_heads=kv_heads,
                                       batch=batch)
    q = (q.float() * 4.0).to(torch.bfloat16)
    k = (k.float() * 4.0).to(torch.bfloat16)
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    out, _ = backend.forward(_Layer(), q.cuda().transpose(1, 2), k.cuda().transpose(1, 2),
                             v.cuda().transpose(1, 2), None, SCALE)
    expected = ref.attention_layer(to_np(q), to_np(k), to_np(v), SCALE, method, alpha)
    assert out.shape == (batch, length, q_heads, 128)
    assert_output_close(to_np(out), expected["output"],
                        what=f"{method} b{batch} S{length} {q_heads}/{kv_heads} a{alpha}",
                        rel=2.0 ** -7)
