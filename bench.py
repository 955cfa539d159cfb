#!/usr/bin/env python3
"""Sparse-prefill attention benchmark on one MI355X.

Headline (BASELINE.json metric "sparse-prefill attn ms/layer @32K Qwen2.5-7B
shape"): one prefill attention layer, method mean_native alpha=0.08, block 128,
sink 2, window 4, last 2 exact query blocks, at S=32640 tokens with 28 query /
4 KV heads, head_dim 128, bf16, through
``AttentionBackend.forward`` exactly as a Qwen2 attention layer calls it. A
"step" is one such layer over synthetic seeded N(0,1)+RoPE inputs already
resident in HBM. ``value`` = ms per layer (lower is better).

Also reported on the same line:
  roofline      the attention kernel's algorithmic FLOP rate (8,388,608 x selected
                128x128 tiles / its HIP-event duration inside the timed region)
                against the 2.5 PFLOP/s bf16 dense MFMA peak, plus its HBM bytes per
                launch (profiles/hbm_traffic.json, from rocprofv3 FETCH/WRITE_SIZE);
  achievable    measured ceilings on the same box: a 16384^3 bf16 GEMM (hipBLASLt
                through torch, N(0,1) data) and a 1 GiB device copy;
  methods       ms/layer and selected-block density of all eight methods (the six of
                the headline table plus fp_v1_rescue and fp_v1_rescue_v2);
  stages        per-stage kernel times with their roofline fractions;
  full_model    the metric's second half: random-init Qwen2.5-7B (28 layers) prefill of
                32640 ids, median of rotated repeats as evaluate.py times it, with peak
                allocated / reserved memory, for every method (dense through torch SDPA
                under the reference's backend pin) and dense through the HIP kernel;
  cpu_baseline  the CPU oracle (numpy restatement of the reference path) on a
                bounded sample of the same workload, scaled to ms per layer, with the
                GPU routing's threshold ties against the oracle's; the same for every
                method (per_method); BASELINE config 1 (S=4096) through the oracle in
                full beside the same layer on the GPU; BASELINE config 5 (S=131072,
                cgf_mean) on sampled query tiles beside the GPU layer.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FLOPS_PER_TILE = 4 * 128 * 128 * 128   # QK^T + PV of one 128x128 tile at d=128
METHOD_NAMES = ("dense", "fp_v1", "mean_native", "mean_balanced", "cgf_mean", "dispersion_mean",
                "fp_v1_rescue", "fp_v1_rescue_v2")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--seq", type=int, default=32640)
    p.add_argument("--method", default="mean_native", choices=METHOD_NAMES)
    p.add_argument("--alpha", type=float, default=0.08)
    p.add_argument("--seed", type=int, default=17)
    p.add_argument("--no-methods", action="store_true", help="skip the methods table")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample-tiles", type=int, default=4, help="minimum sampled query tiles")
    p.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of sampled attention")
    p.add_argument("--cpu-headline-only", action="store_true",
                   help="time the CPU oracle for the headline method only (not every method "
                        "and not config 5)")
    p.add_argument("--cpu-method-budget", type=float, default=8.0,
                   help="seconds of sampled attention per method in the per-method CPU baseline")
    p.add_argument("--cpu-config5-budget", type=float, default=15.0,
                   help="seconds of sampled tiles in the config-5 CPU baseline")
    p.add_argument("--traffic-file", default=str(ROOT / "profiles" / "hbm_traffic.json"))
    p.add_argument("--no-full-model", action="store_true",
                   help="skip the full-model 32K prefill (second half of the metric)")
    p.add_argument("--model-repeats", type=int, default=3)
    return p.parse_args()


class Layer:
    layer_idx = 0


def progress(message):
    """One progress line on stderr (the JSON result line goes to stdout)."""
    print(f"bench: {message}", file=sys.stderr, flush=True)


def timed_forward(backend, q, k, v, scale, steps, warmup, torch):
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    for _ in range(warmup):
        backend.forward(Layer(), qt, kt, vt, None, scale)
    torch.cuda.synchronize()
    if backend.kernel_events is not None:
        backend.kernel_events.clear()
    start = time.perf_counter()
    for _ in range(steps):
        backend.forward(Layer(), qt, kt, vt, None, scale)
    torch.cuda.synchronize()
    return (time.perf_counter() - start) * 1000.0 / steps


def selection_stats(backend, q, k, v, scale, method, torch):
    """Selected 128x128 tiles (N_sel) and exact token pairs of one call."""
    from exp3_amd import attention, kernels
    if method == "dense":
        blocks = math.ceil(q.shape[1] / 128)
        n_sel = blocks * (blocks + 1) // 2 * q.shape[2] * q.shape[0]
        seq = q.shape[1]
        return n_sel, q.shape[0] * q.shape[2] * seq * (seq + 1) // 2, 1.0
    record = {"events": {}}
    if method in attention.V1_ROUTED_METHODS:
        _, _, cnt, sel = backend._v1_selection(q, k, scale, record, v)
    else:
        _, _, _, cnt, sel = backend._new_selection(q, k, v, scale, record)
    acct = kernels.selection_accounting(sel, q.shape[1], 128, 128, method, 32)
    torch.cuda.synchronize()
    return int(cnt.sum().item()), int(acct["exact_token_pairs"].item()), \
        float(acct["legacy_block_density"].item())


def stage_profile(backend, q, k, v, scale, torch):
    backend.start_profile()
    for _ in range(3):
        backend.forward(Layer(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                        None, scale)
    rows = backend.finish_profile()
    out = {}
    for name in ("descriptor", "selector", "indices", "exact"):
        out[name] = sorted(r[f"{name}_ms"] for r in rows)[len(rows) // 2]
    return out


def achievable_peaks(torch):
    """Measured ceilings on this box: a large bf16 GEMM through torch (hipBLASLt)
    on N(0,1) data and a device-to-device copy, for context next to the nominal
    peaks (random data keeps the MFMA clock below the nominal 2.5 PFLOP/s one)."""
    n = 16384
    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    for _ in range(3):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    reps = 10
    for _ in range(reps):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    gemm = 2 * n ** 3 * reps / (time.perf_counter() - t0) / 1e12
    del a, b
    x = torch.empty(1 << 29, device="cuda", dtype=torch.bfloat16)   # 1 GiB
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        y.copy_(x)
    torch.cuda.synchronize()
    copy = 2 * x.numel() * 2 * 10 / (time.perf_counter() - t0) / 1e9
    return {"gemm_bf16_16384_tflops": round(gemm, 1), "copy_1gib_gbs": round(copy, 1)}


def _cpu_threads():
    try:
        from threadpoolctl import threadpool_info
        return max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover
        return os.cpu_count() or 1


def _cpu_model():
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _oracle_route(ref, qn, kn, vn, scale, method, alpha):
    """The oracle's routing for ``method`` (attention_layer's first half):
    (indices, counts, selected, descriptors, rescue choice, routing scores)."""
    import numpy as np
    batch, seq, heads, _ = qn.shape
    blocks = ref.num_blocks(seq)
    desc = scores = None
    if method == "dense":
        sel = np.broadcast_to(np.arange(blocks)[None, :, None, None]
                              >= np.arange(blocks)[None, None, :, None], (batch, blocks, blocks, heads))
        idx, cnt = ref.indices_from_mask(sel)
    elif method in ref.V1_ROUTED:
        if method == "mean_native":
            desc = ref.block_descriptors(kn, vn, precision="f32")
        kbar = ref.block_mean_k(kn, precision="f32")
        scores = ref.v1_scores(qn, kbar, scale, precision="f32")
        idx, cnt = ref.deal_output_score(scores, 2, 4, alpha, 2, 0)
        sel = ref.mask_from_indices(idx, cnt)
    else:
        desc = ref.block_descriptors(kn, vn, precision="f32")
        scores = ref.selector_scores(qn, desc, scale, method, precision="f32")
        sel = ref.protected_selection(scores, alpha, 2, 4, 2)
        idx, cnt = ref.indices_from_mask(sel)
    choice = ref.rescue_choice(qn, kn, precision="f32") if method in ref.RESCUE_METHODS else None
    return idx, cnt, sel, desc, choice, scores


def _oracle_tiles(ref, qn, kn, vn, scale, method, route, tiles):
    """The oracle's attention part of the layer for the given query tiles (all
    tiles for None); rows outside the tiles are left as the exact part's zeros."""
    import numpy as np
    idx, cnt, sel, desc, choice = route[:5]
    out, lse = ref.exact_attention(qn, kn, vn, idx, cnt, scale, precision="f32", tiles=tiles)
    if method in ref.MEAN_METHODS:
        t_out, t_lse = ref.mean_tail(qn, desc, sel, scale, precision="f32", tiles=tiles)
    elif method in ref.RESCUE_METHODS:
        t_out, t_lse = ref.rescue_tail(qn, kn, vn, sel, scale, remainder=method == "fp_v1_rescue_v2",
                                       precision="f32", tiles=tiles, choice=choice)
    else:
        return out
    rows = slice(None) if tiles is None else np.concatenate(
        [np.arange(t * 128, min(qn.shape[1], t * 128 + 128)) for t in tiles])
    merged, _ = ref.merge_exact_mean(out[:, rows], lse[:, rows], t_out[:, rows], t_lse[:, rows])
    out[:, rows] = merged
    return out


def full_model_prefill(seq, alpha, seed, repeats, probe, torch):
    """Second half of the metric ("full-model prefill ms"):
    random-init Qwen2.5-7B (28 layers, bf16) prefilling ``seq`` seeded token ids with
    the backend registered as transformers' "sdpa" attention, timed as the
    reference's evaluate.py:323-345 / 630-663 (warm-up per case, ``repeats``
    rotated rounds, median, peak allocated / reserved memory per prefill) inside
    the SDPA backend pin of evaluate.py:630. Cases: every method at ``alpha``
    (dense through torch SDPA, the reference's dense) and dense through the HIP
    attention kernel (like for like)."""
    from exp3_amd import attention
    from measure import sweeps
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    saved = ALL_ATTENTION_FUNCTIONS["sdpa"]
    context, sdpa_name = sweeps.dense_sdpa_context(probe)
    backend = attention.AttentionBackend(alpha=alpha)   # registers as "sdpa"
    try:
        t0 = time.perf_counter()
        model = sweeps.build_qwen2_7b(28, seed)
        build_s = time.perf_counter() - t0
        ids = sweeps.prompt_ids(seq, seed, model.config.vocab_size)
        cases = [(m, m, "sdpa") for m in attention.METHODS] + [("dense_hip", "dense", "hip")]
        times, tokens, peaks = sweeps.time_prefills(model, backend, ids, cases, repeats, alpha,
                                                    context)
    finally:
        ALL_ATTENTION_FUNCTIONS["sdpa"] = saved
    med = {label: sweeps.median(v) for label, v in times.items()}
    per_method = {
        label: {"prefill_ms": round(med[label], 1),
                "speedup_vs_dense": round(med["dense"] / med[label], 3),
                "peak_allocated_gib": round(max(p[0] for p in peaks[label]), 3),
                "peak_reserved_gib": round(max(p[1] for p in peaks[label]), 3),
                "all_ms": [round(x, 1) for x in times[label]],
                "first_token_id": tokens[label]}
        for label in times}
    result = {
        "seq": seq, "layers": 28, "model": "random-init Qwen2.5-7B architecture, bf16",
        "alpha": alpha, "repeats": repeats, "median_of": "rotated repeats (evaluate.py:646-663)",
        "dense_sdpa_backend": sdpa_name,
        "dense_ms": round(med["dense"], 1),
        "fp_v1_ms": round(med["fp_v1"], 1),
        "mean_native_ms": round(med["mean_native"], 1),
        "dense_hip_ms": round(med["dense_hip"], 1),
        "speedup": round(med["dense"] / med["mean_native"], 3),
        "speedup_vs_dense_hip": round(med["dense_hip"] / med["mean_native"], 3),
        "methods": per_method,
        "model_build_s": round(build_s, 1),
    }
    del model
    torch.cuda.empty_cache()
    return result


def routing_ties(gpu_scores, gpu_sel, scores, sel, alpha, positive_rule, eps=1e-6, tiles=None):
    """Threshold ties of one routing against the oracle's: routed entries (causal,
    outside the sink / window / last query blocks) whose oracle score lies within
    ``eps`` of its row's threshold fp32(max * alpha) (or of 0 under the selectors'
    positive-score rule), how many of those the GPU mask sets differently, and how
    many entries differ anywhere else (0 when the masks agree up to ties)."""
    import numpy as np
    shape = sel.shape
    t = np.arange(shape[1]).reshape(1, -1, 1, 1)
    j = np.arange(shape[2]).reshape(1, 1, -1, 1)
    routed = (j <= t - 4) & (j >= 2) & (t < shape[1] - 2)
    if tiles is not None:
        routed = routed & np.isin(np.arange(shape[1]), tiles).reshape(1, -1, 1, 1)
    routed = np.broadcast_to(routed, shape)
    thr = (scores.max(axis=2, keepdims=True).astype(np.float32) * np.float32(alpha))
    near = np.abs(scores.astype(np.float64) - thr.astype(np.float64)) <= eps
    if positive_rule:
        near |= np.abs(scores) <= eps
    rows = slice(None) if tiles is None else tiles
    differ = np.zeros(shape, bool)
    differ[:, rows] = gpu_sel[:, rows] != sel[:, rows]
    ties = near & routed
    return {"routed_entries": int(np.count_nonzero(routed)),
            "tie_entries": int(np.count_nonzero(ties)),
            "differ_at_ties": int(np.count_nonzero(differ & near)),
            "differ_elsewhere": int(np.count_nonzero(differ & ~near)),
            "max_abs_score_diff": float(np.abs(gpu_scores[:, rows].astype(np.float64)
                                               - scores[:, rows]).max()),
            "eps": eps}


def gpu_routing(qg, kg, vg, scale, method, alpha):
    """The GPU's routing scores and selection mask (numpy) for ``method``, from the
    kernels ``forward`` launches."""
    from exp3_amd import attention, kernels
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    record = {"events": {}}
    if method in attention.V1_ROUTED_METHODS:
        values = vg if method in ("mean_native", "fp_v1_rescue_v2") else None
        _, _, scores, _, _, sel = backend._v1_selection(qg, kg, scale, record, values, True)
    else:
        desc, _, _, _, sel = backend._new_selection(qg, kg, vg, scale, record)
        scores = kernels.selector_scores(qg, desc, scale, method)
    return scores.float().cpu().numpy(), sel.cpu().numpy()


def cpu_baseline(q, k, v, scale, method, alpha, sample_tiles, budget_s, gpu=None):
    """Time the CPU oracle (reference semantics in numpy float32) on the full
    routing stages plus a sample of query tiles of the attention stages; scale
    the sampled part by selected-block work to a whole layer. With ``gpu`` (the
    same inputs on the device) the GPU routing is compared with the oracle's and
    its threshold ties are recorded."""
    import numpy as np
    from oracle import reference_cpu as ref
    qn, kn, vn = (x.float().cpu().numpy() for x in (q, k, v))
    blocks = ref.num_blocks(qn.shape[1])
    t0 = time.perf_counter()
    route = _oracle_route(ref, qn, kn, vn, scale, method, alpha)
    routing_s = time.perf_counter() - t0
    ties = None
    if gpu is not None and route[5] is not None:
        g_scores, g_sel = gpu_routing(*gpu, scale, method, alpha)
        ties = routing_ties(g_scores, g_sel, route[5], route[2], alpha,
                            positive_rule=method not in ref.V1_ROUTED)
    # query tiles in a stratified order (coarse to fine over the sequence) until the
    # time budget is spent, so the sample is spread over short and long tiles
    order = []
    step = blocks
    while step >= 1 and len(order) < blocks:
        for t in range(0, blocks, step):
            if t not in order:
                order.append(t)
        step //= 2
    tiles = []
    t1 = time.perf_counter()
    for t in order:
        _oracle_tiles(ref, qn, kn, vn, scale, method, route, [t])
        tiles.append(t)
        if len(tiles) >= sample_tiles and time.perf_counter() - t1 >= budget_s:
            break
    attention_s = time.perf_counter() - t1
    work = route[1].sum(axis=(0, 2)).astype(np.float64) + 1.0   # per tile (+1: the tail row pass)
    scale_up = work.sum() / work[tiles].sum()
    total_ms = (routing_s + attention_s * scale_up) * 1000.0
    result = {
        "value": round(total_ms, 1),
        "unit": "ms",
        "cores": int(_cpu_threads()),
        "kind": "port",
        "sample": (f"{method} alpha={alpha} S={qn.shape[1]}: routing over all {blocks} query tiles "
                   f"({routing_s:.1f} s), attention (exact blocks + tail + merge) over {len(tiles)} "
                   f"query tiles spread over the sequence ({attention_s:.1f} s) scaled x{scale_up:.1f} "
                   f"by selected-block work; numpy float32 oracle (reference's own harness pins "
                   f"1 thread, evaluate.py:793)"),
        "routing_s": round(routing_s, 2),
        "attention_sample_s": round(attention_s, 2),
        "sampled_tiles": len(tiles),
        "cpu": _cpu_model(),
    }
    if ties is not None:
        result["ties"] = ties
    return result


def cpu_config5(seed, alpha, budget_s, torch, method="cgf_mean", seq=131072, needles=256):
    """BASELINE config 5 on the CPU: S=131072 with 256 planted needles, ``method`` at
    ``alpha``. The oracle runs the descriptors over the whole sequence, then scores,
    selects and attends (exact blocks + mean tail + merge) sampled query tiles, one
    at a time in the order 255, 511, 767, 1023, 127, 383, ... until ``budget_s``: a
    tile's selector scores depend on its own rows only, and its attention on the
    sequence up to its last row, so each tile runs on the prefix that ends with it.
    The layer estimate scales the sampled per-tile time by causal work (t + 1 blocks
    per tile; selection density is 1.0 on these inputs). The same layer runs on the
    GPU beside it; the sampled tiles' GPU scores, masks and outputs are compared
    with the oracle's."""
    import numpy as np
    from oracle import reference_cpu as ref
    from exp3_amd import attention, synthetic
    q, k, v, _ = synthetic.make_inputs(seq, seed=seed, needles=needles)
    scale = 128 ** -0.5
    qn, kn, vn = (x.float().numpy() for x in (q, k, v))
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    gpu_ms = timed_forward(backend, qg, kg, vg, scale, 3, 1, torch)
    out, _ = backend.forward(Layer(), qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2),
                             None, scale)
    out = out.float().cpu().numpy()
    g_scores, g_sel = gpu_routing(qg, kg, vg, scale, method, alpha)
    del qg, kg, vg
    torch.cuda.empty_cache()
    blocks = ref.num_blocks(seq)
    order, step = [], 256
    while step >= 1 and len(order) < blocks:
        for t in range(step - 1, blocks, step):
            if t not in order:
                order.append(t)
        step //= 2
    t0 = time.perf_counter()
    desc = ref.block_descriptors(kn, vn, precision="f32")
    desc_s = time.perf_counter() - t0
    scores = np.zeros((1, blocks, blocks, qn.shape[2]), np.float32)
    tiles, tile_s, max_abs, mean_abs = [], 0.0, 0.0, []
    for t in order:
        end = min(seq, (t + 1) * 128)
        prefix = ref.BlockDescriptors(desc.mean_k[:, :t + 1], desc.mean_v[:, :t + 1],
                                      desc.var_k[:, :t + 1], desc.sigma_v[:, :t + 1],
                                      desc.counts[:t + 1])
        t1 = time.perf_counter()
        row = ref.selector_scores(qn[:, :end], prefix, scale, method, precision="f32",
                                  tiles=[t])[:, t]
        scores[:, t, :t + 1] = row
        sel = ref.protected_selection(scores, alpha, 2, 4, 2)   # row t's rule needs NB
        expected, _ = ref.attention_from_selection(qn[:, :end], kn[:, :end], vn[:, :end], scale,
                                                   method, sel[:, :t + 1, :t + 1], prefix,
                                                   precision="f32", tiles=[t])
        tile_s += time.perf_counter() - t1
        tiles.append(t)
        if (g_sel[:, t] == sel[:, t]).all():
            diff = np.abs(out[:, t * 128:end] - expected[:, t * 128:end])
            max_abs = max(max_abs, float(diff.max()))
            mean_abs.append(float(diff.mean()))
        if len(tiles) >= 2 and tile_s >= budget_s:
            break
    sel = ref.protected_selection(scores, alpha, 2, 4, 2)
    ties = routing_ties(g_scores, g_sel, scores, sel, alpha, positive_rule=True, tiles=tiles)
    work = np.arange(1, blocks + 1, dtype=np.float64)
    scale_up = work.sum() / work[tiles].sum()
    cpu_ms = (desc_s + tile_s * scale_up) * 1000.0
    return {"config": "BASELINE config 5", "method": method, "alpha": alpha, "seq": seq,
            "needles": needles, "cpu_ms": round(cpu_ms, 1), "cpu_cores": int(_cpu_threads()),
            "kind": "port",
            "sample": (f"descriptors over all {seq} tokens ({desc_s:.1f} s); selector scores, "
                       f"protected selection and attention (exact + mean tail + merge) of "
                       f"{len(tiles)} query tiles {tiles}, each on its prefix ({tile_s:.1f} s), "
                       f"scaled x{scale_up:.1f} by causal work (t + 1 blocks per tile)"),
            "gpu_ms": round(gpu_ms, 3), "ties": ties,
            "max_abs_gpu_vs_cpu": max_abs,
            "mean_abs_gpu_vs_cpu": float(np.mean(mean_abs)) if mean_abs else None,
            "compared_tiles": len(mean_abs)}


def cpu_config1(method, alpha, seed, torch):
    """S=4096, the whole layer through the CPU oracle (no
    sampling), beside the same layer on the GPU, with their max / mean abs
    difference."""
    import numpy as np
    from oracle import reference_cpu as ref
    from exp3_amd import attention, synthetic
    q, k, v, _ = synthetic.make_inputs(4096, seed=seed)
    scale = 128 ** -0.5
    qn, kn, vn = (x.float().numpy() for x in (q, k, v))
    t0 = time.perf_counter()
    route = _oracle_route(ref, qn, kn, vn, scale, method, alpha)
    expected = _oracle_tiles(ref, qn, kn, vn, scale, method, route, None)
    cpu_ms = (time.perf_counter() - t0) * 1000.0
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    backend = attention.AttentionBackend(alpha=alpha, register=False)
    backend.configure(method, alpha)
    gpu_ms = timed_forward(backend, qg, kg, vg, scale, 10, 3, torch)
    out, _ = backend.forward(Layer(), qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2),
                             None, scale)
    diff = np.abs(out.float().cpu().numpy() - expected)
    return {"config": "BASELINE config 1", "method": method, "alpha": alpha, "seq": 4096,
            "cpu_ms": round(cpu_ms, 1), "cpu_cores": int(_cpu_threads()), "kind": "port",
            "gpu_ms": round(gpu_ms, 4), "max_abs_gpu_vs_cpu": float(diff.max()),
            "mean_abs_gpu_vs_cpu": float(diff.mean())}


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the sparse-prefill path "
                                   "is single-GPU (bench.py --gpus 1); multi-GPU sharding is a "
                                   "design note (KV-head groups), not built"}), flush=True)
        sys.exit(2)

    import torch
    from exp3_amd import _lib, attention, synthetic

    from measure import sweeps

    _lib.load()
    device = torch.device("cuda:0")
    # the reference pins torch SDPA to FLASH_ATTENTION around every prefill
    # (evaluate.py:630); the same pin (or, if that backend refuses the GQA call
    # on this GPU, the first accepting one) wraps every timing below
    sdpa_probe = sweeps.probe_sdpa_backends()
    sdpa_context, sdpa_name = sweeps.dense_sdpa_context(sdpa_probe)
    sdpa_context.__enter__()
    scale = 128 ** -0.5
    q, k, v, _ = synthetic.make_inputs(args.seq, seed=args.seed)
    qg, kg, vg = q.to(device), k.to(device), v.to(device)

    backend = attention.AttentionBackend(alpha=args.alpha, register=False)
    backend.configure(args.method, args.alpha)
    backend.kernel_events = []
    ms = timed_forward(backend, qg, kg, vg, scale, args.steps, args.warmup, torch)
    kernel_ms = sum(a.elapsed_time(b) for a, b in backend.kernel_events) / len(backend.kernel_events)
    backend.kernel_events = None
    n_sel, exact_pairs, density = selection_stats(backend, qg, kg, vg, scale, args.method, torch)
    flops = FLOPS_PER_TILE * n_sel
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    head_dim = q.shape[3]

    traffic = None
    tf = Path(args.traffic_file)
    if tf.exists():
        try:
            entry = json.loads(tf.read_text()).get(f"{args.method}:{args.seq}")
            if entry:
                traffic = entry.get("bytes_per_launch")
        except (ValueError, OSError):
            traffic = None

    stages = stage_profile(backend, qg, kg, vg, scale, torch)
    kv_bytes = 2 * args.seq * k.shape[2] * head_dim * 2
    blocks = math.ceil(args.seq / 128)
    # pool: K and V read once; key and value tiles written (padded to whole blocks);
    # bf16 mean K plus fp32 mean K / mean V / var K descriptors
    tile_bytes = 2 * blocks * 128 * k.shape[2] * head_dim * 2
    pool_bytes = kv_bytes + tile_bytes + blocks * k.shape[2] * head_dim * (2 + 4 * 3)
    route_bytes = args.seq * q.shape[2] * head_dim * 2 + blocks * blocks * q.shape[2] * (8 + 1)
    stage_report = {
        "pool": {"ms": round(stages["descriptor"], 4),
                 "gbs": round(pool_bytes / (stages["descriptor"] * 1e-3) / 1e9, 1),
                 "frac_hbm": round(pool_bytes / (stages["descriptor"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)},
        "route": {"ms": round(stages["selector"], 4),
                  "gbs": round(route_bytes / (stages["selector"] * 1e-3) / 1e9, 1),
                  "frac_hbm": round(route_bytes / (stages["selector"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)},
        # stage events bracket the whole launch call (host-side setup included when
        # the GPU has caught up); kernel_ms brackets the attention kernel alone
        "attention": {"ms": round(stages["exact"], 4), "kernel_ms": round(kernel_ms, 4)},
    }

    methods = {}
    if not args.no_methods:
        for name in attention.METHODS:
            b = attention.AttentionBackend(alpha=args.alpha, register=False)
            b.configure(name, args.alpha)
            m_ms = timed_forward(b, qg, kg, vg, scale, 5, 2, torch)
            m_sel, m_pairs, m_density = selection_stats(b, qg, kg, vg, scale, name, torch)
            methods[name] = {"ms_per_layer": round(m_ms, 3), "block_density": round(m_density, 5),
                             "effective_tflops": round(4 * head_dim * m_pairs / (m_ms * 1e-3) / 1e12, 1)}
        b = attention.AttentionBackend(alpha=args.alpha, register=False, dense_impl="hip")
        b.configure("dense")
        methods["dense_hip"] = {"ms_per_layer": round(timed_forward(b, qg, kg, vg, scale, 5, 2, torch), 3),
                                "block_density": 1.0}

    progress("layer, stages and methods timed")
    achievable = achievable_peaks(torch)
    sdpa_context.__exit__(None, None, None)

    full_model = None
    if not args.no_full_model:
        progress("full-model prefills")
        full_model = full_model_prefill(args.seq, args.alpha, args.seed, args.model_repeats,
                                        sdpa_probe, torch)
        full_model["sdpa_probe"] = sdpa_probe

    baseline = None
    if not args.no_cpu_baseline:
        progress("CPU baseline")
        baseline = cpu_baseline(q, k, v, scale, args.method, args.alpha, args.cpu_sample_tiles,
                                args.cpu_budget, gpu=(qg, kg, vg))
        baseline["config1"] = cpu_config1(args.method, args.alpha, args.seed, torch)
        if not args.cpu_headline_only:
            per_method = {}
            for name in attention.METHODS:
                if name == args.method:
                    entry = {key: val for key, val in baseline.items() if key != "config1"}
                else:
                    entry = cpu_baseline(q, k, v, scale, name, args.alpha, 2,
                                         args.cpu_method_budget, gpu=(qg, kg, vg))
                if name in methods:
                    entry["gpu_ms"] = methods[name]["ms_per_layer"]
                per_method[name] = entry
                progress(f"CPU baseline {name}: {entry['value']} ms")
            baseline["per_method"] = per_method
            del qg, kg, vg
            torch.cuda.empty_cache()
            progress("CPU baseline config 5")
            baseline["config5"] = cpu_config5(args.seed, 0.04, args.cpu_config5_budget, torch)

    line = {
        "metric": "sparse-prefill attn ms/layer @32K Qwen2.5-7B shape; full-model prefill ms",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"single prefill attention layer, {args.method} alpha={args.alpha}, "
                         f"S={args.seq}, 28 q / 4 kv heads, head_dim 128, block 128, sink 2, "
                         f"window 4, last 2 (BASELINE config 2)"),
            "seq_len": args.seq, "batch": 1, "q_heads": 28, "kv_heads": 4, "head_dim": 128,
            "method": args.method, "alpha": args.alpha, "seed": args.seed,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "kernel": ("attn_kernel (spx_sparse_attention_mean)" if args.method in attention.MEAN_METHODS
                       else "attn_kernel (spx_sparse_attention_rescue)"
                       if args.method in attention.RESCUE_METHODS
                       else "attn_kernel (spx_exact_attention)"),
            "kernel_ms": round(kernel_ms, 4),
            "selected_tiles": n_sel,
            "flops_per_launch": flops,
            "frac_of_achievable_gemm": round(achieved / achievable["gemm_bf16_16384_tflops"], 4),
        },
        "achievable": achievable,
        "effective_tflops": round(4 * head_dim * exact_pairs / (ms * 1e-3) / 1e12, 1),
        "block_density": round(density, 5),
        "stages": stage_report,
        "methods": methods,
        "dense_sdpa_backend": sdpa_name,
        "full_model": full_model,
        "cpu_baseline": baseline,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
