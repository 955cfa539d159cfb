"""The attention kernel's dynamic tail (work_queue): the light third of the tile
pairs taken from a zeroed counter by whichever workgroups run first, to even out
the XCDs. Results must be bit-identical to the static schedule (the same items,
each computed by one workgroup with the same arithmetic), every item must be taken
exactly once (the counter ends at the tail's item count plus the surplus
workgroups that found it empty), and layouts with (batch x kv heads) not a proper
divisor of 8 keep the static schedule (d = 128); the d = 256 kernel deals its last
third of tile ranks the same way."""

import numpy as np
import pytest
import torch

from exp3_amd import _lib, attention, synthetic
from tests.helpers import to_np

pytestmark = pytest.mark.gpu



def _call(entry, q, k, tiles, idx, cnt, desc, queue):
    batch, seq, q_heads, head_dim = q.shape
    out = torch.full((batch, seq, q_heads, head_dim), float("nan"), dtype=q.dtype, device=q.device)
    lse = torch.full((batch, seq, q_heads), float("nan"), dtype=torch.float32, device=q.device)
    head = (_lib.ptr(q), _lib.strides(q), _lib.ptr(tiles[0]), _lib.ptr(tiles[1]), _lib.ptr(idx),
            _lib.strides(idx), _lib.ptr(cnt), _lib.strides(cnt))
    tail = (batch, seq, q_heads, k.shape[2], head_dim, 128, head_dim ** -0.5, _lib.ptr(out),
            _lib.strides(out), _lib.ptr(lse), _lib.strides(lse), _lib.ptr(queue),
            _lib.stream(q.device))
    if entry == "mean":
        _lib.call("spx_sparse_attention_mean", *head, _lib.ptr(desc.mean_k), _lib.ptr(desc.mean_v),
                  _lib.ptr(desc.counts), *tail)
    else:
        _lib.call("spx_exact_attention", *head, *tail)
    return out, lse


@pytest.mark.parametrize("layout", ((1, 28, 4, 128, 4500), (1, 28, 4, 128, 32640),
                                    (1, 8, 2, 128, 3000), (2, 28, 4, 128, 2113),
                                    (1, 12, 3, 128, 2113), (1, 16, 4, 256, 4500),
                                    (2, 16, 4, 256, 2113)))
@pytest.mark.parametrize("entry", ("exact", "mean"))
def test_dynamic_tail_matches_static_schedule(gpu, layout, entry):
    batch, q_heads, kv_heads, head_dim, length = layout
    q, k, v, _ = synthetic.make_inputs(length, seed=41, q_heads=q_heads, kv_heads=kv_heads,
                                       head_dim=head_dim, batch=batch, device="cuda")
    q = (q.float() * 4).to(torch.bfloat16)     # sparse lists, non-empty mean tails
    k = (k.float() * 4).to(torch.bfloat16)
    backend = attention.AttentionBackend(alpha=0.7, register=False)
    backend.configure("mean_native", 0.7)
    _, desc, tiles, _, idx, cnt, _ = backend._route_v1(q, k, v, head_dim ** -0.5, {"events": {}},
                                                       True, True)
    if entry == "exact" and length == 32640:
        idx = cnt = None     # dense: every causal block
    static = _call(entry, q, k, tiles, idx, cnt, desc, None)
    queue = torch.zeros(1, dtype=torch.int32, device="cuda")
    dynamic = _call(entry, q, k, tiles, idx, cnt, desc, queue)
    torch.cuda.synchronize()
    assert torch.equal(static[0], dynamic[0]) and torch.equal(static[1], dynamic[1])
    assert not torch.isnan(dynamic[0]).any()
    blocks = (length + 127) // 128
    streams = batch * kv_heads
    taken = int(queue.item())
    if head_dim == 256:
        # one workgroup per (tile, head): the last third of the tile ranks dynamic,
        # 1.25 x as many tail workgroups as items
        items = (blocks - blocks * 2 // 3) * batch * q_heads
        assert taken == (items * 5 + 3) // 4 >= items
        return
    per_stream_xcds = 8 // streams if streams <= 8 and 8 % streams == 0 else 1
    if per_stream_xcds > 1:
        # kernel constants: the first two thirds of the tile pairs static, 1.25 x an even
        # share of tail workgroups per XCD
        np_ = (blocks + 1) // 2
        tp0 = np_ * 2 // 3
        while tp0 > 0 and (tp0 * (q_heads // kv_heads)) % per_stream_xcds:
            tp0 -= 1
        items = (np_ - tp0) * streams * (q_heads // kv_heads)
        workgroups = 8 * int((items * 1.25 + 7) // 8)
        assert taken == workgroups >= items
    else:
        assert taken == 0          # static schedule: the counter is not touched
