"""Host-side checks that need no GPU: the C-ABI library loads and exports every
symbol the header declares, its argument validation returns the documented
error codes, and the Python mirror keeps the reference's interface."""

import ctypes
import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from exp3_amd import _lib, attention, kernels, synthetic
from exp3_amd.upstream import flashprefill_native_forward as up

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sparse_prefill.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(spx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declared_symbols()
    assert len(declared) >= 21
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    assert lib.spx_abi_version() == _lib.ABI_VERSION


def test_c_abi_argument_validation_without_gpu():
    lib = _lib.load()
    s4 = (ctypes.c_int64 * 4)(4096, 512, 128, 1)
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: validation fails first
    assert lib.spx_block_mean_k(fake, s4, 1, 256, 4, 64, 128, fake, None) == _lib.SPX_EUNSUPPORTED
    assert b"head_dim" in lib.spx_last_error()
    assert lib.spx_block_mean_k(fake, s4, 1, 256, 4, 128, 64, fake, None) == _lib.SPX_EUNSUPPORTED
    assert lib.spx_block_mean_k(fake, s4, 0, 256, 4, 128, 128, fake, None) == _lib.SPX_EINVAL
    bad = (ctypes.c_int64 * 4)(4096, 512, 128, 2)          # non-unit dim stride
    assert lib.spx_block_mean_k(fake, bad, 1, 256, 4, 128, 128, fake, None) == _lib.SPX_EINVAL
    odd = ctypes.c_void_p((1 << 20) + 2)                    # misaligned base
    assert lib.spx_block_mean_k(odd, s4, 1, 256, 4, 128, 128, fake, None) == _lib.SPX_EINVAL
    assert lib.spx_selector_scores(fake, s4, fake, fake, fake, fake, 1, 256, 28, 4, 128, 128, 7,
                                   ctypes.c_float(0.1), fake, fake, s4, None) == _lib.SPX_EINVAL
    # a null workspace is rejected; workspace bytes = B Hkv ceil(NB / 32) (D / 128) 32 KB
    assert lib.spx_selector_scores(fake, s4, fake, fake, fake, fake, 1, 256, 28, 4, 128, 128, 1,
                                   ctypes.c_float(0.1), None, fake, s4, None) == _lib.SPX_EINVAL
    assert lib.spx_selector_workspace_bytes(1, 32640, 4, 128) == 4 * 8 * 32768
    assert lib.spx_selector_workspace_bytes(2, 4097, 4, 128) == 2 * 4 * 2 * 32768
    assert lib.spx_selector_workspace_bytes(1, 32640, 4, 256) == 2 * 4 * 8 * 32768
    assert lib.spx_selector_workspace_bytes(1, 256, 4, 64) == -1
    # 28 q heads over 3 kv heads is not a GQA grouping
    assert lib.spx_exact_attention(fake, s4, fake, fake, None, None, None, None, 1, 256, 28, 3,
                                   128, 128, ctypes.c_float(0.1), fake, s4, None, None, None,
                                   None) == _lib.SPX_EINVAL
    # 131073 tokens exceed the 1024-block limit of the routing kernels
    assert lib.spx_v1_scores(fake, s4, fake, s4, 1, 131073, 28, 4, 128, 128, ctypes.c_float(0.1),
                             fake, s4, None) == _lib.SPX_EUNSUPPORTED
    assert lib.spx_mean_tail(fake, s4, None, None, None, None, fake, fake, fake, 1, 256, 28, 4, 128,
                             128, ctypes.c_float(0.1), fake, s4, None, None, None) == _lib.SPX_EINVAL
    # the routed V1 form: at most 256 q heads, an 8-byte-aligned index output (its
    # per-block partials live there between the route's two kernels)
    def route(heads, kv_heads, indices):
        return lib.spx_v1_route(fake, s4, fake, s4, 1, 256, heads, kv_heads, 128, 128,
                                ctypes.c_float(0.1), ctypes.c_float(0.08), 2, 4, 2, None, indices,
                                fake, None, None)
    assert route(264, 8, fake) == _lib.SPX_EUNSUPPORTED
    assert b"q_heads" in lib.spx_last_error()
    assert route(28, 4, ctypes.c_void_p((1 << 20) + 4)) == _lib.SPX_EINVAL


def test_call_maps_status_to_exceptions():
    s4 = (ctypes.c_int64 * 4)(4096, 512, 128, 1)
    fake = ctypes.c_void_p(1 << 20)
    with pytest.raises(ValueError, match="head_dim"):
        _lib.call("spx_block_mean_k", fake, s4, 1, 256, 4, 64, 128, fake, None)


def test_reference_interface():
    assert attention.METHODS == ("dense", "fp_v1", "mean_native", "mean_balanced", "cgf_mean",
                                 "dispersion_mean", "fp_v1_rescue", "fp_v1_rescue_v2")
    assert attention.MEAN_METHODS == {"mean_native", "mean_balanced", "cgf_mean", "dispersion_mean"}
    b = attention.AttentionBackend(register=False)
    assert (b.alpha, b.sink_blocks, b.window_blocks, b.last_full_blocks, b.block_size,
            b.selector_chunk_tiles) == (0.08, 2, 4, 2, 128, 8)
    with pytest.raises(ValueError, match="unknown method"):
        b.configure("topk")
    b.configure("cgf_mean")
    assert b.alpha == 0.08
    b.configure("fp_v1", 0.16)
    assert (b.method, b.alpha) == ("fp_v1", 0.16)
    assert up.attention_tile_sizes() == (128, 128) and up.score_tile_size() == 32
    # check_qwen35_math.py:134-139 reads the exact-attention launch through
    # _flash_forward.best_config; attention_tile_sizes() reports the same values
    config = up._flash_forward.best_config
    launch = {**config.kwargs, "num_warps": config.num_warps, "num_stages": config.num_stages}
    assert launch == {"Q_TILE_SIZE": 128, "K_TILE_SIZE": 128, "num_warps": 8, "num_stages": 2}
    assert up.compute_block_score.best_config.kwargs["K_TILE_SIZE"] == up.score_tile_size()
    with pytest.raises(ValueError, match="unsupported selector"):
        kernels.selector_scores(torch.zeros(1, 8, 1, 128), None, 0.1, "bogus")
    with pytest.raises(ValueError, match="ROCm GPU"):
        kernels.rescue_tail(torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16),
                            torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16),
                            torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16),
                            torch.zeros(1, 1, 1, 1, dtype=torch.bool), 0.1)


def test_backend_registers_as_sdpa():
    tf = pytest.importorskip("transformers.modeling_utils")
    b = attention.AttentionBackend()
    assert tf.ALL_ATTENTION_FUNCTIONS["sdpa"] == b.forward


def test_wrappers_refuse_cpu_tensors():
    k = torch.zeros(1, 256, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        up.block_mean_k(k)
    with pytest.raises(ValueError, match="ROCm GPU"):
        kernels.block_descriptors(k, k)
    b = attention.AttentionBackend(register=False)
    b.configure("mean_native")

    class L:
        layer_idx = 0

    q = torch.zeros(1, 28, 256, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        b.forward(L(), q, k.transpose(1, 2), k.transpose(1, 2), None, 0.1)
    b.configure("fp_v1_rescue")
    with pytest.raises(ValueError, match="ROCm GPU"):
        b.forward(L(), q, k.transpose(1, 2), k.transpose(1, 2), None, 0.1)


def test_kernel_view_keeps_transposed_layout():
    base = torch.zeros(1, 300, 28, 128, dtype=torch.bfloat16)
    view = base.transpose(1, 2).transpose(1, 2)
    assert _lib.kernel_view(view).data_ptr() == base.data_ptr()
    assert _lib.kernel_view(base[..., :64].contiguous()).shape[-1] == 64
    strided = torch.zeros(1, 300, 28, 256, dtype=torch.bfloat16)[..., ::2]
    assert _lib.kernel_view(strided).stride()[-1] == 1
    with pytest.raises(ValueError):
        _lib.kernel_view(torch.zeros(1, 8, 1, 128))
    with pytest.raises(ValueError, match="bfloat16"):   # the kernels read bf16 only
        _lib.kernel_view(torch.zeros(1, 8, 1, 128, dtype=torch.float16))


def test_rope_matches_transformers_qwen2():
    modeling = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    x = torch.randn(1, 64, 3, 128)
    pos = torch.arange(64)
    ours = synthetic.apply_rope(x, pos, synthetic.rope_inv_freq())
    inv = synthetic.rope_inv_freq()
    freqs = pos[:, None].float() * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    hf_q, _ = modeling.apply_rotary_pos_emb(x.transpose(1, 2), x.transpose(1, 2),
                                            emb.cos()[None], emb.sin()[None])
    torch.testing.assert_close(ours, hf_q.transpose(1, 2), atol=1e-6, rtol=1e-6)


def test_synthetic_needles():
    q, k, v, positions = synthetic.make_inputs(4096, seed=5, needles=16)
    assert len(positions) == 16 and min(positions) >= 256 and max(positions) < (32 - 4) * 128
    qf, kf = q.float(), k.float()
    last = qf[0, 31 * 128:, 0:7].reshape(-1, 128).mean(0)
    for p in positions[:4]:
        cos = torch.nn.functional.cosine_similarity(kf[0, p, 0], last, dim=0)
        assert abs(cos.item() - 0.8) < 0.02
    mean_norm = kf[0, :, 0].norm(dim=-1).median()
    assert 2.5 < (kf[0, positions[0], 0].norm() / mean_norm).item() < 3.5
    q2, k2, v2, _ = synthetic.make_inputs(4096, seed=5, needles=16)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2 and "one GPU" in proc.stdout
