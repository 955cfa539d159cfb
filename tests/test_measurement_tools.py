"""CPU checks of the measurement helpers: the rocprofv3 traffic reduction and the
full-model sweep's Qwen2.5-7B-shaped config (no GPU needed)."""

import csv
import json

import pytest

from measure import profiling


def _counter_csv(directory, rows):
    directory.mkdir(parents=True)
    with open(directory / "p_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for did, kernel, counter, value in rows:
            w.writerow({"Dispatch_Id": did, "Kernel_Name": kernel, "Counter_Name": counter,
                        "Counter_Value": value})


def test_traffic_reduction_scales_by_copy_calibration(tmp_path):
    gib_kib = 1 << 20
    # the copy reads 1 GiB but FETCH_SIZE reports half; WRITE_SIZE reports it exactly
    _counter_csv(tmp_path / "cf", [(1, "rand", "FETCH_SIZE", 10), (2, "__amd_rocclr_copyBuffer",
                                    "FETCH_SIZE", gib_kib / 2), (3, "__amd_rocclr_copyBuffer",
                                    "FETCH_SIZE", gib_kib / 2)])
    _counter_csv(tmp_path / "cw", [(2, "__amd_rocclr_copyBuffer", "WRITE_SIZE", gib_kib)])
    # attention: two dispatches, FETCH split over two counter instances per dispatch
    _counter_csv(tmp_path / "af", [(3, "spx::attn_kernel<true>", "FETCH_SIZE", 100.0),
                                   (3, "spx::attn_kernel<true>", "FETCH_SIZE", 150.0),
                                   (6, "spx::attn_kernel<true>", "FETCH_SIZE", 250.0),
                                   (7, "spx::v1_route_kernel", "FETCH_SIZE", 9999.0)])
    _counter_csv(tmp_path / "aw", [(3, "spx::attn_kernel<true>", "WRITE_SIZE", 40.0),
                                   (6, "spx::attn_kernel<true>", "WRITE_SIZE", 40.0)])
    out = tmp_path / "traffic.json"

    class Args:
        attn_fetch, attn_write = tmp_path / "af", tmp_path / "aw"
        copy_fetch, copy_write = tmp_path / "cf", tmp_path / "cw"
        copy_gib, attn_kernel, copy_kernel = 1.0, r"attn_kernel", r"copyBuffer"
        key = "mean_native:32640"

    Args.out = str(out)
    entry = profiling.traffic(Args)
    assert entry["fetch_size_scale"] == pytest.approx(2.0)
    assert entry["write_size_scale"] == pytest.approx(1.0)
    assert entry["read_bytes"] == 250 * 1024 * 2
    assert entry["write_bytes"] == 40 * 1024
    assert entry["bytes_per_launch"] == entry["read_bytes"] + entry["write_bytes"]
    assert json.loads(out.read_text())["mean_native:32640"] == entry


def test_qwen2_7b_config_matches_the_model_shape():
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    from measure import sweeps
    cfg = sweeps.qwen2_7b_config(28)
    assert (cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers) == (3584, 18944, 28)
    assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.vocab_size) == (28, 4, 152064)
    rope = getattr(cfg, "rope_parameters", None) or {}
    assert rope.get("rope_theta", getattr(cfg, "rope_theta", None)) == 1e6
    assert cfg.rms_norm_eps == 1e-6
    with torch.device("meta"):
        model = transformers.Qwen2ForCausalLM(cfg)
    assert sum(p.numel() for p in model.parameters()) == 7_615_616_512   # Qwen2.5-7B
    assert model.model.layers[0].self_attn.q_proj.bias is not None       # QKV bias


@pytest.mark.parametrize("method", ("dense", "fp_v1", "mean_native", "mean_balanced", "cgf_mean",
                                    "dispersion_mean", "fp_v1_rescue", "fp_v1_rescue_v2"))
def test_bench_cpu_baseline_layer_equals_oracle_layer(method):
    """bench.py's CPU baseline splits the oracle layer into routing and per-tile
    attention; the two halves over all tiles give exactly the oracle's layer."""
    import numpy as np
    import bench
    from oracle import reference_cpu as ref
    from tests.helpers import inputs, to_np, SCALE
    q, k, v = inputs(385, seed=29)
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    route = bench._oracle_route(ref, qn, kn, vn, SCALE, method, 0.08)
    out = bench._oracle_tiles(ref, qn, kn, vn, SCALE, method, route, None)
    expected = ref.attention_layer(qn, kn, vn, SCALE, method, 0.08, precision="f32")
    np.testing.assert_array_equal(out, expected["output"])
    sampled = bench._oracle_tiles(ref, qn, kn, vn, SCALE, method, route, [1])
    np.testing.assert_array_equal(sampled[:, 128:256], expected["output"][:, 128:256])
