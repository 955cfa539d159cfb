"""A whole prefill layer captured in a HIP graph (torch.cuda.CUDAGraph on ROCm):
the C entry points allocate nothing and never synchronise, and the per-call work
counters are cleared by a fill kernel, so the layer can be captured once and
replayed. Every replay, with other eager layers run between them, must give the
eager output bit for bit (all kernels are deterministic)."""

import pytest
import torch

from exp3_amd import attention, synthetic

pytestmark = pytest.mark.gpu


class DummyAttention:
    layer_idx = 0


def _sharpened(length, seed):
    # Q and K x 4: at alpha 0.7 the routing keeps a fraction of the blocks, so the
    # block-mean and rescue tails are non-empty
    q, k, v, _ = synthetic.make_inputs(length, seed=seed, device="cuda")
    q = (q.float() * 4).to(torch.bfloat16)
    k = (k.float() * 4).to(torch.bfloat16)
    return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)


@pytest.mark.parametrize("method", ("mean_native", "cgf_mean", "fp_v1_rescue_v2", "dense"))
def test_prefill_layer_replayed_from_a_graph(gpu, method):
    alpha = 0.7
    backend = attention.AttentionBackend(alpha=alpha, register=False, dense_impl="hip")
    backend.configure(method, alpha)
    q, k, v = _sharpened(2000, seed=83)
    q2, k2, v2 = _sharpened(1500, seed=89)

    def layer(a, b, c):
        return backend.forward(DummyAttention(), a, b, c, None, 128 ** -0.5)[0]

    eager = layer(q, k, v).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            layer(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = layer(q, k, v)
    torch.cuda.synchronize()
    for replay in range(3):
        other = layer(q2, k2, v2)          # eager work between the replays
        torch.cuda.synchronize()
        assert torch.isfinite(other.float()).all()
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"{method}: replay {replay} differs from the eager layer"
