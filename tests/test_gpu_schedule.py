"""The attention kernel's work queue (work_queue): with it the d = 128 kernel runs a
persistent grid, one workgroup per CU taking (tile pair, head) items in turn: the
first two thirds of the tile pairs from its own XCD's counter in the static deal's
order, then the light last third: per (batch, kv group) stream when several XCDs
serve each stream (a workgroup drains its own stream's tail, then the others'), from
one shared counter otherwise. Results must be bit-identical to the
one-item-per-workgroup grid (the same items, each computed by one workgroup with the
same arithmetic), and every item must be taken exactly once: each counter ends at
its item count plus one failed draw per workgroup. The d = 256 kernel deals its last
third of tile ranks through the shared counter with 1.25 x as many tail workgroups
as items."""

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
    queue = torch.zeros(_lib.WORK_QUEUE_INTS, dtype=torch.int32, device="cuda")
    dynamic = _call(entry, q, k, tiles, idx, cnt, desc, queue)
    torch.cuda.synchronize()
    assert torch.equal(static[0], dynamic[0]) and torch.equal(static[1], dynamic[1])
    assert not torch.isnan(dynamic[0]).any()
    blocks = (length + 127) // 128
    streams = batch * kv_heads
    group = q_heads // kv_heads
    counters = queue.cpu().numpy().astype(np.int64)
    if head_dim == 256:
        items = (blocks - blocks * 2 // 3) * batch * q_heads
        assert counters[0] == (items * 5 + 3) // 4 >= items
        assert not counters[1:].any()
        return
    # kernel constants: two thirds of the tile pairs on the per-XCD deal (rounded down
    # to whole XCD shares), one workgroup per CU, at most one per static item
    np_ = (blocks + 1) // 2
    xps = 8 // streams if streams <= 8 and 8 % streams == 0 else 1
    tp0 = np_ * 2 // 3
    while tp0 > 0 and xps > 1 and (tp0 * group) % xps:
        tp0 -= 1
    per_xcd = (np_ * group + xps - 1) // xps if xps > 1 else (np_ * streams + 7) // 8 * group
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    grid = 8 * min(cus // 8, per_xcd)
    if xps > 1:
        static_items = 8 * (tp0 * group // xps)
    else:
        static_items = sum(max(0, (tp0 * streams - x + 7) // 8) * group for x in range(8))
    tail_items = (np_ - tp0) * streams * group
    assert static_items + tail_items == np_ * streams * group
    assert counters[1:9].sum() == static_items + grid
    if xps > 1:   # one tail counter per stream (from index 9), each tried by every workgroup
        assert counters[0] == 0
        assert (counters[9:9 + streams] == (np_ - tp0) * group + grid).all()
        assert not counters[9 + streams:].any()
    else:
        assert counters[0] == tail_items + grid
        assert not counters[9:].any()
