"""Maximum size: S = 131072 tokens (NB = 1024, the kernels' block limit).

The oracle cannot run whole layers this long in a test, so the checks are the
size-independent properties (V1 and selector score rows sum to 1 over the
visible blocks) plus oracle parity on sampled query tiles of a full mean_native
layer, given the GPU's own block lists."""

import numpy as np
import pytest
import torch

from exp3_amd import attention, kernels
from exp3_amd.upstream import flashprefill_native_forward as up
from oracle import reference_cpu as ref
from tests.helpers import SCALE, assert_output_close, to_np

pytestmark = pytest.mark.gpu

LENGTH = 131072


@pytest.fixture(scope="module")
def big():
    g = torch.Generator(device="cuda").manual_seed(89)
    q = torch.randn(1, LENGTH, 28, 128, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(1, LENGTH, 4, 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(1, LENGTH, 4, 128, device="cuda", generator=g).to(torch.bfloat16)
    return q, k, v


def test_v1_and_selector_rows_at_max_size(gpu, big):
    q, k, v = big
    blocks = LENGTH // 128
    scores = up.v1_scores(q, up.block_mean_k(k), SCALE)
    rows = scores[0].double().sum(dim=1).cpu().numpy()          # [t, h]
    assert np.allclose(rows, 1.0, atol=5e-5)
    upper = torch.triu(torch.ones(blocks, blocks, dtype=torch.bool, device="cuda"), 1)
    assert (scores[0][upper] == 0).all()
    del scores
    sel = kernels.selector_scores(q, kernels.block_descriptors(k, v), SCALE, "mean_balanced")
    rows = sel[0, 1:].double().sum(dim=1).cpu().numpy()
    assert np.allclose(rows, 1.0, atol=5e-5)
    assert (sel[0][upper | torch.eye(blocks, dtype=torch.bool, device="cuda")] == 0).all()


def test_mean_native_layer_sampled_tiles_at_max_size(gpu, big):
    """Q and K scaled by 8 and alpha 0.5 so V1 selects sparsely and the block-mean
    tail spans hundreds of unselected blocks; tiles 0, 511, 1021 (the last tile
    routed by score) and 1023 (protected: every block) against the oracle, given
    the GPU's own descriptors and selection."""
    q, k, v = big
    q = (q.float() * 8).to(torch.bfloat16)
    k = (k.float() * 8).to(torch.bfloat16)
    backend = attention.AttentionBackend(alpha=0.5, register=False)
    backend.configure("mean_native", 0.5)
    out, _ = backend.forward(type("L", (), {"layer_idx": 0})(), q.transpose(1, 2),
                             k.transpose(1, 2), v.transpose(1, 2), None, SCALE)
    assert torch.isfinite(out).all()
    record = {"events": {}}
    _, desc, _, _, idx, cnt, sel = backend._route_v1(q, k, v, SCALE, record, True, False)
    tiles = [0, 511, 1021, 1023]
    sel_n = to_np(sel)
    assert sel_n[0, 1021].mean() < 0.9                  # the tail is not empty
    assert sel_n[0, 1023].all()                         # last tiles are protected
    e_desc = ref.BlockDescriptors(*(to_np(getattr(desc, n)) for n in
                                    ("mean_k", "mean_v", "var_k", "sigma_v", "counts")))
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    ex_out, ex_lse = ref.exact_attention(qn, kn, vn, to_np(idx), to_np(cnt), SCALE,
                                         precision="f32", tiles=tiles)
    m_out, m_lse = ref.mean_tail(qn, e_desc, sel_n, SCALE, precision="f32", tiles=tiles)
    for t in tiles:
        rows = slice(t * 128, (t + 1) * 128)
        merged, _ = ref.merge_exact_mean(ex_out[:, rows], ex_lse[:, rows], m_out[:, rows],
                                         m_lse[:, rows])
        # peaked attention: outputs beyond unit scale, one bf16 step relative on top
        assert_output_close(to_np(out[:, rows]), merged, what=f"S=131072 tile {t}",
                            rel=2.0 ** -7)
