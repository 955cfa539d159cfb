"""spx_selector_scores_noalloc: the selector scores with the split workspace in the
library's static device array instead of a caller workspace. Called through the
C ABI, its scores must equal spx_selector_scores' bit for bit, on two calls in a
row (the second with a smaller input, so stale array contents from the first
would show), and shapes beyond the array are refused before any launch."""

import ctypes

import pytest
import torch

from exp3_amd import _lib, kernels, synthetic

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _noalloc(q, desc, selector):
    lib = _lib.load()
    batch, sequence, q_heads, head_dim = q.shape
    blocks = desc.mean_k.shape[1]
    scores = torch.full((batch, blocks, blocks, q_heads), float("nan"), dtype=torch.float32,
                        device=q.device)
    status = lib.spx_selector_scores_noalloc(
        _lib.ptr(q), _lib.strides(q), _lib.ptr(desc.mean_k), _lib.ptr(desc.var_k),
        _lib.ptr(desc.sigma_v), _lib.ptr(desc.counts), batch, sequence, q_heads,
        desc.mean_k.shape[2], head_dim, 128, _lib.SELECTOR_IDS[selector], ctypes.c_float(SCALE),
        _lib.ptr(scores), _lib.strides(scores), _lib.stream(q.device))
    assert status == _lib.SPX_OK, lib.spx_last_error()
    return scores


@pytest.mark.parametrize("head_dim", (128, 256))
@pytest.mark.parametrize("selector", ("mean_balanced", "cgf_mean", "dispersion_mean"))
def test_noalloc_matches_workspace_entry_point(gpu, selector, head_dim):
    heads = {"q_heads": 28, "kv_heads": 4} if head_dim == 128 else {"q_heads": 16, "kv_heads": 4}
    for length, seed in ((4500, 3), (1089, 4)):      # the second call is smaller
        q, k, v, _ = synthetic.make_inputs(length, seed=seed, head_dim=head_dim, device="cuda",
                                           **heads)
        desc = kernels.block_descriptors(k, v)
        want = kernels.selector_scores(q, desc, SCALE, selector)
        got = _noalloc(q, desc, selector)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{selector} S={length} D={head_dim}"


def test_noalloc_refuses_shapes_beyond_the_array(gpu):
    lib = _lib.load()
    # 2 sequences x 8 KV heads x 32 chunks of 32 blocks = 16 MiB of workspace > 8 MiB;
    # refused on the host before any pointer is read
    dummy = torch.zeros(8, device="cuda")
    strides = (ctypes.c_int64 * 4)(8, 8, 8, 1)
    status = lib.spx_selector_scores_noalloc(
        _lib.ptr(dummy), strides, _lib.ptr(dummy), _lib.ptr(dummy), _lib.ptr(dummy),
        _lib.ptr(dummy), 2, 131072, 56, 8, 128, 128, 0, ctypes.c_float(SCALE), _lib.ptr(dummy),
        strides, _lib.stream(dummy.device))
    assert status == _lib.SPX_EUNSUPPORTED
    assert b"static scratch" in lib.spx_last_error()
