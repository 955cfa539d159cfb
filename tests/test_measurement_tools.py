"""CPU checks of the measurement helpers: the rocprofv3 traffic reduction, the
full-model sweep's Qwen2.5-7B-shaped config and the CPU mirror of the attention
grid's XCD mapping (no GPU needed)."""

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


@pytest.mark.parametrize("batch,kv_heads,group,blocks", [(1, 4, 7, 255), (1, 4, 7, 9), (2, 4, 7, 17),
                                                         (1, 1, 8, 33), (1, 8, 4, 12), (3, 2, 6, 5)])
@pytest.mark.parametrize("alternating", (False, True))
def test_attention_grid_items_cover_every_item_once(batch, kv_heads, group, blocks, alternating):
    """The CPU mirror of the attention kernel's workgroup -> (tile pair, head) mapping
    deals every item to exactly one XCD, and when the number of (batch, kv group)
    streams divides 8, XCD x serves stream x mod streams only."""
    from measure import sweeps
    per_xcd = sweeps.attention_grid_items(batch, kv_heads, group, blocks, alternating)
    items = [it for lst in per_xcd for it in lst]
    pairs = (blocks + 1) // 2
    assert sorted(items) == sorted((tp, b, g, hg) for tp in range(pairs) for b in range(batch)
                                   for g in range(kv_heads) for hg in range(group))
    streams = batch * kv_heads
    if 8 % streams == 0:
        for xcd, lst in enumerate(per_xcd):
            assert all((b * kv_heads + g) == xcd % streams for tp, b, g, hg in lst)


def test_alternating_mapping_splits_tile_pairs_and_balances_xcds():
    """With 4 kv groups the heads of each tile pair alternate between XCDs g and g + 4,
    and on the dense lists every XCD gets the same work (the earlier mapping gave
    XCDs 0-3 the heavier pair of every two)."""
    import numpy as np
    from measure import sweeps
    per_xcd = sweeps.attention_grid_items(1, 4, 7, 255, True)
    heads_of_pair0 = {x: sorted(hg for tp, b, g, hg in per_xcd[x] if tp == 0 and g == 0)
                      for x in (0, 4)}
    assert heads_of_pair0 == {0: [0, 2, 4, 6], 4: [1, 3, 5]}
    dense = np.broadcast_to(np.tril(np.ones((255, 255), bool))[:, :, None], (255, 255, 28))
    span_old, loads_old, ideal = sweeps.simulate_xcds(dense, 4, (12.6, 3.45, 2.02), False)
    span_new, loads_new, ideal2 = sweeps.simulate_xcds(dense, 4, (12.6, 3.45, 2.02), True)
    assert ideal == pytest.approx(ideal2)
    assert max(loads_new) - min(loads_new) < 0.01 * ideal < max(loads_old) - min(loads_old)
    assert span_new < span_old
