"""Measurement runs beyond the headline bench line (one GPU, synthetic data).

  python -m measure.sweeps needles [--seq 32640] [--needles 64]
      planted-retrieval inputs; alpha in {0.04, 0.08, 0.16} for the four mean
      methods, fp_v1 at 0.08 and dense: ms/layer, selected-block density
      counts.sum() / (H NB (NB + 1) / 2) and the exact-pair ratio
      (kernels.py:338-353 accounting)
  python -m measure.sweeps long [--seq 131072] [--needles 256]
      long context: cgf_mean and dispersion_mean at alpha 0.04 (plus mean_native
      at 0.04 for reference), same columns
  python -m measure.sweeps sparse [--seq 32640] [--qk-scale 4]
      sparse selections (not a BASELINE config): the seeded inputs with Q and K
      multiplied by --qk-scale (bf16) sharpen the block scores, and alpha in
      {0.08, 0.3, 0.5, 0.7} gives densities well below 1, exercising the block-mean
      and rescue tails; mean_native, fp_v1, cgf_mean, fp_v1_rescue_v2 and dense
  python -m measure.sweeps d256 [--seq 32640]
      head_dim 256 with 16 query / 4 KV heads (Qwen3.5 full-attention layer shape,
      check_qwen35_math.py): dense (torch SDPA and the HIP kernel) and every sparse
      method at alpha 0.08, and four methods on Q, K x 4 at alpha 0.7 (sparse
      lists, non-empty tails); ms/layer, the attention kernel's HIP-event time and
      its rate over the selected 128 x 128 tiles (4 x 128 x 128 x 256 FLOP each)
  python -m measure.sweeps pair-overlap [--seq 32640] [--qk-scale 4] [--alpha 0.7]
      fp_v1 on sharpened inputs: the attention kernel on the routed lists and on
      lists where each tile pair's lists coincide (tile t - 1 takes tile t's routed
      blocks), the cost of pairing tiles whose lists differ
  python -m measure.sweeps cost-model [--seq 32640]
      the attention kernel on synthetic lists (unscaled inputs): every list empty,
      then k blocks per tile pair listed by both tiles or by one tile only; prints
      each case's time and the fitted per-workgroup and per-step costs
  python -m measure.sweeps xcd-balance [--seq 32640] [--qk-scale 4] [--alpha 0.7]
      routes the fp_v1 layer on the GPU, then simulates on the CPU how the
      attention grid's work items land on the 8 XCDs (workgroup i on XCD i % 8,
      greedy dispatch to each XCD's CUs in grid order) under the shipped mapping
      and the earlier one-tile-pair-per-XCD mapping, with per-item costs from
      the cost model; also for the dense (all causal blocks) lists
  python -m measure.sweeps route [--cases 32640:128:28,32640:256:16,131072:128:28]
      the fused V1 route (spx_v1_route: block products, then the per-tile
      normalisation and selection) on the seeded inputs, seq:head_dim:q_heads per
      case with 4 KV heads, alpha 0.08: HIP events around 50 back-to-back calls
      after 5 warm-up calls; microseconds per call and the rate over its
      algorithmic bytes (Q read once, int64 indices and the mask written)
  python -m measure.sweeps model [--seq 32640] [--layers 28] [--repeats 3]
      full prefill of a random-init Qwen2.5-7B-shaped model built from a local
      config (28 layers, hidden 3584, FFN 18944, 28/4 heads, RMSNorm 1e-6,
      theta 1e6, vocab 152064, QKV bias, bf16) with the attention backend
      registered as transformers' "sdpa" function. Timing follows
      evaluate.py:323-345: ids already on the GPU, sync, timer, model(ids,
      use_cache=True, logits_to_keep=1), argmax, sync; each method warmed up
      first (evaluate.py:634-644), repeats with rotated method order
      (evaluate.py:646-663), median reported (report.py:33-42); then 128 greedy
      dense decode tokens (not timed) to exercise the decode path. With
      --split-last-token, each method also runs evaluate.py:357-380's RULER flow:
      prefill of the first S - 1 ids through the backend, then the last id as one
      cached decode step; its first greedy id is printed beside the full
      prefill's.

Every run prints one JSON object per measured case.
"""

from __future__ import annotations

import argparse
import json
import math
import sys
import time

MEAN_FOUR = ("mean_native", "mean_balanced", "cgf_mean", "dispersion_mean")


class _Layer:
    layer_idx = 0


def _layer_case(torch, attention, kernels, q, k, v, method, alpha, steps=5, warmup=2,
                dense_impl="sdpa", scale=None):
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    backend = attention.AttentionBackend(alpha=alpha, register=False, dense_impl=dense_impl)
    backend.configure(method, alpha)
    backend.kernel_events = []
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    for _ in range(warmup):
        backend.forward(_Layer(), qt, kt, vt, None, scale)
    torch.cuda.synchronize()
    backend.kernel_events.clear()
    t0 = time.perf_counter()
    for _ in range(steps):
        backend.forward(_Layer(), qt, kt, vt, None, scale)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    kernel_ms = (sum(x.elapsed_time(y) for x, y in backend.kernel_events)
                 / len(backend.kernel_events)) if backend.kernel_events else None
    seq, heads, dim = q.shape[1], q.shape[2], q.shape[3]
    blocks = math.ceil(seq / 128)
    selected_tiles = heads * blocks * (blocks + 1) // 2
    if method == "dense":
        density, pair_ratio = 1.0, 1.0
    else:
        record = {"events": {}}
        if method in attention.V1_ROUTED_METHODS:
            _, _, cnt, sel = backend._v1_selection(q, k, scale, record, v)
        else:
            _, _, _, cnt, sel = backend._new_selection(q, k, v, scale, record)
        acct = kernels.selection_accounting(sel, seq, 128, 128, method, 32)
        selected_tiles = int(cnt.sum().item())
        density = selected_tiles / (heads * blocks * (blocks + 1) / 2)
        pair_ratio = float(acct["effective_exact_token_pair_ratio"].item())
    row = {"method": method, "alpha": alpha if method != "dense" else None, "seq": seq,
           "ms_per_layer": round(ms, 3), "block_density": round(density, 5),
           "exact_pair_ratio": round(pair_ratio, 5)}
    if kernel_ms:
        flops = 4.0 * 128 * 128 * dim * selected_tiles
        row.update({"kernel_ms": round(kernel_ms, 3),
                    "kernel_tflops": round(flops / (kernel_ms * 1e-3) / 1e12, 1)})
    return row


def run_layer_sweep(seq, needles, seed, cases, label):
    import torch
    from exp3_amd import _lib, attention, kernels, synthetic
    _lib.load()
    q, k, v, positions = synthetic.make_inputs(seq, seed=seed, needles=needles, device="cuda")
    for method, alpha in cases:
        row = _layer_case(torch, attention, kernels, q, k, v, method, alpha)
        row.update({"sweep": label, "needles": needles, "seed": seed})
        print(json.dumps(row), flush=True)


def run_sparse(seq, seed, qk_scale):
    import torch
    from exp3_amd import _lib, attention, kernels, synthetic
    _lib.load()
    q, k, v, _ = synthetic.make_inputs(seq, seed=seed, device="cuda")
    q = (q.float() * qk_scale).to(torch.bfloat16)
    k = (k.float() * qk_scale).to(torch.bfloat16)
    cases = [(m, a) for a in (0.08, 0.3, 0.5, 0.7)
             for m in ("mean_native", "fp_v1", "cgf_mean", "fp_v1_rescue_v2")]
    cases.append(("dense", 0.08))
    for method, alpha in cases:
        row = _layer_case(torch, attention, kernels, q, k, v, method, alpha)
        row.update({"sweep": "sparse", "qk_scale": qk_scale, "seed": seed})
        print(json.dumps(row), flush=True)


def run_d256(seq, seed):
    import torch
    from exp3_amd import _lib, attention, kernels, synthetic
    _lib.load()
    q, k, v, _ = synthetic.make_inputs(seq, seed=seed, q_heads=16, kv_heads=4, head_dim=256,
                                       device="cuda")
    cases = [("dense", "sdpa", 0.08, 1.0), ("dense", "hip", 0.08, 1.0)]
    cases += [(m, "sdpa", 0.08, 1.0) for m in attention.METHODS[1:]]
    # sharpened inputs (Q, K x 4) at alpha 0.7: sparse lists, non-empty tails
    cases += [(m, "sdpa", 0.7, 4.0) for m in ("fp_v1", "mean_native", "cgf_mean",
                                             "fp_v1_rescue_v2")]
    for method, dense_impl, alpha, qk in cases:
        qq, kk = q, k
        if qk != 1.0:
            qq = (q.float() * qk).to(torch.bfloat16)
            kk = (k.float() * qk).to(torch.bfloat16)
        row = _layer_case(torch, attention, kernels, qq, kk, v, method, alpha, steps=5, warmup=2,
                          dense_impl=dense_impl, scale=256 ** -0.5)
        row.update({"sweep": "d256", "q_heads": 16, "kv_heads": 4, "head_dim": 256,
                    "qk_scale": qk, "impl": dense_impl if method == "dense" else "hip"})
        print(json.dumps(row), flush=True)


def run_pair_overlap(seq, seed, qk_scale, alpha):
    """fp_v1 on sharpened inputs: the attention kernel's time on the routed lists and
    on lists where tile t - 1 takes tile t's routed blocks below it (its diagonal
    added), so that each tile pair's lists coincide; bounds what pairing tiles on
    list overlap can give."""
    import numpy as np
    import torch
    from exp3_amd import _lib, attention, kernels, synthetic
    _lib.load()
    q, k, v, _ = synthetic.make_inputs(seq, seed=seed, device="cuda")
    q = (q.float() * qk_scale).to(torch.bfloat16)
    k = (k.float() * qk_scale).to(torch.bfloat16)
    scale = 128 ** -0.5
    b = attention.AttentionBackend(alpha=alpha, register=False)
    b.configure("fp_v1", alpha)
    _, _, tiles, _, idx, cnt, sel = b._route_v1(q, k, v, scale, {"events": {}}, False, True)
    blocks = sel.shape[1]

    def timed(i, c, n=10):
        for _ in range(3):
            b._attention(q, k, tiles, i, c, scale, None, want_lse=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            b._attention(q, k, tiles, i, c, scale, None, want_lse=False)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def union_efficiency(m):
        union = 0
        for tp in range((blocks + 1) // 2):
            t1, t2 = blocks - 1 - 2 * tp, blocks - 2 - 2 * tp
            union += (m[t1] | (m[t2] if t2 >= 0 else np.zeros_like(m[t1]))).sum()
        return m.sum() / (2 * union)

    m = sel.cpu().numpy()[0]
    aligned = m.copy()
    for tp in range((blocks + 1) // 2):
        t1, t2 = blocks - 1 - 2 * tp, blocks - 2 - 2 * tp
        if t2 >= 0:
            row = m[t1].copy()
            row[t2 + 1:] = False
            row[t2] = True
            aligned[t2] = row
    i2, c2 = kernels.indices_from_mask(torch.from_numpy(aligned[None]).cuda())
    for label, lists, mask in (("routed", (idx, cnt), m), ("pair-aligned", (i2, c2), aligned)):
        ms = timed(*lists)
        n_sel = int(mask.sum())
        print(json.dumps({"sweep": "pair-overlap", "lists": label, "seq": seq, "alpha": alpha,
                          "qk_scale": qk_scale, "ms": round(ms, 3), "selected_tiles": n_sel,
                          "union_efficiency": round(float(union_efficiency(mask)), 3),
                          "pflops_on_selected": round(8388608 * n_sel / ms / 1e12, 3)}),
              flush=True)


def _attention_timer(torch, backend, q, k, tiles, scale):
    def timed(indices, counts, n=10):
        for _ in range(3):
            backend._attention(q, k, tiles, indices, counts, scale, None, want_lse=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            backend._attention(q, k, tiles, indices, counts, scale, None, want_lse=False)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n
    return timed


def run_route(cases, seed):
    """spx_v1_route alone, per (seq, head_dim, q_heads) case (see the module docstring)."""
    import torch
    from exp3_amd import _lib, synthetic
    from exp3_amd.upstream import flashprefill_native_forward as up
    _lib.load()
    for seq, head_dim, q_heads in cases:
        q, k, _, _ = synthetic.make_inputs(seq, seed=seed, q_heads=q_heads, kv_heads=4,
                                           head_dim=head_dim, device="cuda")
        kbar = up.block_mean_k(k)
        batch, _, heads, dim = q.shape
        blocks = kbar.shape[1]
        idx = torch.empty(batch, blocks, blocks, heads, dtype=torch.int64, device="cuda")
        cnt = torch.empty(batch, blocks, heads, dtype=torch.int32, device="cuda")
        sel = torch.empty(batch, blocks, blocks, heads, dtype=torch.bool, device="cuda")

        def route():
            _lib.call("spx_v1_route", _lib.ptr(q), _lib.strides(q), _lib.ptr(kbar),
                      _lib.strides(kbar), batch, seq, heads, k.shape[2], dim, 128,
                      dim ** -0.5, 0.08, 2, 4, 2, None, _lib.ptr(idx), _lib.ptr(cnt),
                      _lib.ptr(sel), _lib.stream(q.device))

        for _ in range(5):
            route()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        reps = 50
        e0.record()
        for _ in range(reps):
            route()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        nbytes = q.numel() * 2 + idx.numel() * 9 + cnt.numel() * 4
        print(json.dumps({"sweep": "route", "seq": seq, "head_dim": head_dim, "q_heads": q_heads,
                          "us": round(us, 1), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                          "frac_hbm": round(nbytes / (us * 1e-6) / 8e12, 3)}), flush=True)
        del q, k, kbar, idx, cnt, sel
        torch.cuda.empty_cache()


def run_cost_model(seq, seed):
    """Per-workgroup and per-step costs of the attention kernel from synthetic lists:
    every list empty (fixed cost: Q in, O out, list merge), then for each tile pair
    (t, t - 1) the k most recent history blocks below t - 1 listed by both tiles
    (shared steps) or by tile t only (one-sided steps), diagonals as routing lists
    them. Per-step costs are the slope between k = 16 and k = 32."""
    import numpy as np
    import torch
    from exp3_amd import _lib, attention, synthetic
    _lib.load()
    q, k, v, _ = synthetic.make_inputs(seq, seed=seed, device="cuda")
    scale = 128 ** -0.5
    b = attention.AttentionBackend(alpha=0.08, register=False)
    b.configure("fp_v1", 0.08)
    _, _, tiles, _, _, _, sel = b._route_v1(q, k, v, scale, {"events": {}}, False, True)
    blocks, heads = sel.shape[1], sel.shape[3]
    timed = _attention_timer(torch, b, q, k, tiles, scale)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    workgroups = (blocks + 1) // 2 * heads

    def lists(kk, mode):
        ind = np.full((blocks, blocks, heads), blocks, dtype=np.int64)
        cnt = np.zeros((blocks, heads), dtype=np.int32)
        union = 0
        for tp in range((blocks + 1) // 2):
            t1, t2 = blocks - 1 - 2 * tp, blocks - 2 - 2 * tp
            lim = max(t2, 0)
            hist = list(range(lim - min(kk, lim), lim))
            l1 = [] if mode == "empty" else hist + ([t2] if t2 >= 0 else []) + [t1]
            l2 = [] if mode == "empty" else (hist if mode == "shared" else []) + [t2]
            ind[t1, :len(l1)] = np.array(l1, dtype=np.int64)[:, None] if l1 else blocks
            cnt[t1] = len(l1)
            if t2 >= 0:
                ind[t2, :len(l2)] = np.array(l2, dtype=np.int64)[:, None] if l2 else blocks
                cnt[t2] = len(l2)
            union += heads * len(set(l1) | (set(l2) if t2 >= 0 else set()))
        return torch.from_numpy(ind[None]).cuda(), torch.from_numpy(cnt[None]).cuda(), union

    rows = {}
    for mode, kk in (("empty", 0), ("shared", 16), ("shared", 32), ("one-sided", 16),
                     ("one-sided", 32)):
        i, c, union = lists(kk, mode)
        ms = timed(i, c, 20)
        rows[(mode, kk)] = (ms, union)
        print(json.dumps({"sweep": "cost-model", "lists": mode, "k": kk, "ms": round(ms, 4),
                          "steps": union, "selected_tiles": int(c.sum().item())}), flush=True)
    slope = lambda m: ((rows[(m, 32)][0] - rows[(m, 16)][0])
                       / (rows[(m, 32)][1] - rows[(m, 16)][1]) * 1e6)   # ns per step, GPU-wide
    fit = {"sweep": "cost-model-fit", "cus": cus, "workgroups": workgroups,
           "fixed_us_per_workgroup": round(rows[("empty", 0)][0] * 1e3 * cus / workgroups, 2),
           "shared_step_ns": round(slope("shared"), 2),
           "one_sided_step_ns": round(slope("one-sided"), 2)}
    fit["shared_step_us_per_cu"] = round(fit["shared_step_ns"] * cus / 1e3, 3)
    fit["one_sided_step_us_per_cu"] = round(fit["one_sided_step_ns"] * cus / 1e3, 3)
    print(json.dumps(fit), flush=True)


def attention_grid_items(batch, kv_heads, group, blocks, alternating=True):
    """Work items (tile pair, batch, kv group, head in group) of the d = 128 attention
    grid per XCD, in grid order, as the kernel maps workgroup i (XCD i % 8): with
    ``alternating`` the shipped mapping (a (batch, kv group) stream on 8 / (B Hkv)
    XCDs, its items dealt over them in turn), else pair p on XCD p % 8 with all its
    heads."""
    pairs_per_stream = (blocks + 1) // 2
    streams = batch * kv_heads
    num_pairs = pairs_per_stream * streams
    per_stream = 8 // streams if alternating and streams <= 8 and 8 % streams == 0 else 1
    if per_stream > 1:
        per_xcd = (pairs_per_stream * group + per_stream - 1) // per_stream
    else:
        per_xcd = (num_pairs + 7) // 8 * group
    out = [[] for _ in range(8)]
    for p in range(8 * per_xcd):
        xcd, local = p & 7, p >> 3
        if per_stream > 1:
            kk = local * per_stream + xcd // streams
            pair, hg = (kk // group) * streams + xcd % streams, kk % group
        else:
            pair, hg = (local // group) * 8 + xcd, local % group
        if pair < num_pairs:
            tp, s = pair // streams, pair % streams
            out[xcd].append((tp, s // kv_heads, s % kv_heads, hg))
    return out


def simulate_xcds(mask, kv_heads, costs, alternating, cus_per_xcd=32):
    """Greedy dispatch of each XCD's items to its CUs in grid order; returns
    (makespan, per-XCD work per CU, ideal) in the unit of ``costs`` (fixed per
    item, per shared step, per one-sided step)."""
    import heapq
    import numpy as np
    blocks, _, heads = mask.shape
    group = heads // kv_heads
    fixed, shared, one = costs
    loads, spans = [], []
    for items in attention_grid_items(1, kv_heads, group, blocks, alternating):
        heap = [0.0] * cus_per_xcd
        total = 0.0
        for tp, _, g, hg in items:
            h = g * group + hg
            t1, t2 = blocks - 1 - 2 * tp, blocks - 2 - 2 * tp
            a = mask[t1, :, h]
            bb = mask[t2, :, h] if t2 >= 0 else np.zeros(blocks, bool)
            c = fixed + shared * int((a & bb).sum()) + one * int((a ^ bb).sum())
            total += c
            heapq.heappush(heap, heapq.heappop(heap) + c)
        loads.append(total / cus_per_xcd)
        spans.append(max(heap))
    return max(spans), loads, sum(loads) / 8


def run_xcd_balance(seq, seed, qk_scale, alpha, costs):
    import numpy as np
    import torch
    from exp3_amd import _lib, attention, synthetic
    _lib.load()
    q, k, v, _ = synthetic.make_inputs(seq, seed=seed, device="cuda")
    q = (q.float() * qk_scale).to(torch.bfloat16)
    k = (k.float() * qk_scale).to(torch.bfloat16)
    b = attention.AttentionBackend(alpha=alpha, register=False)
    b.configure("fp_v1", alpha)
    _, _, _, _, _, _, sel = b._route_v1(q, k, v, 128 ** -0.5, {"events": {}}, False, False)
    routed = sel.cpu().numpy()[0]
    blocks, _, heads = routed.shape
    dense = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[:, :, None],
                            routed.shape)
    kv_heads = k.shape[2]
    for label, mask in (("fp_v1 routed", routed), ("dense", dense)):
        for alternating in (False, True):
            span, loads, ideal = simulate_xcds(mask, kv_heads, costs, alternating)
            print(json.dumps({"sweep": "xcd-balance", "lists": label, "alpha": alpha,
                              "qk_scale": qk_scale,
                              "mapping": "alternating heads" if alternating else "pair per XCD",
                              "makespan_ms": round(span / 1e3, 3), "ideal_ms": round(ideal / 1e3, 3),
                              "per_xcd_ms": [round(x / 1e3, 3) for x in loads]}), flush=True)


def qwen2_7b_config(layers):
    from transformers import Qwen2Config
    return Qwen2Config(vocab_size=152064, hidden_size=3584, intermediate_size=18944,
                       num_hidden_layers=layers, num_attention_heads=28, num_key_value_heads=4,
                       rms_norm_eps=1e-6, rope_theta=1e6, max_position_embeddings=32768,
                       tie_word_embeddings=False, use_sliding_window=False,
                       attn_implementation="sdpa", torch_dtype="bfloat16")


SDPA_ORDER = ("FLASH_ATTENTION", "EFFICIENT_ATTENTION", "MATH")


def probe_sdpa_backends(head_dim=128, q_heads=28, kv_heads=4):
    """Which torch SDPA backends accept the reference's dense prefill call
    (attention.py:179-189: causal, ``enable_gqa=True``, bf16) on this GPU, each
    tried alone under ``sdpa_kernel``: name -> "ok" or the error's first line."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    q = torch.randn(1, q_heads, 256, head_dim, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, kv_heads, 256, head_dim, device="cuda", dtype=torch.bfloat16)
    result = {}
    for name in SDPA_ORDER:
        try:
            with sdpa_kernel(getattr(SDPBackend, name)):
                F.scaled_dot_product_attention(q, k, k, is_causal=True, scale=head_dim ** -0.5,
                                               enable_gqa=True)
            torch.cuda.synchronize()
            result[name] = "ok"
        except RuntimeError as exc:
            result[name] = str(exc).strip().splitlines()[0][:160]
    return result


def dense_sdpa_context(probe):
    """The reference's contract is ``sdpa_kernel(SDPBackend.FLASH_ATTENTION)``
    around every prefill (evaluate.py:630); when that backend refuses the GQA call
    on this GPU, the first accepting backend in torch's priority order is pinned
    instead. Returns (context manager, backend name)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for name in SDPA_ORDER:
        if probe.get(name) == "ok":
            return sdpa_kernel(getattr(SDPBackend, name)), name
    raise RuntimeError(f"no SDPA backend accepts the dense GQA call: {probe}")


def build_qwen2_7b(layers=28, seed=17):
    """Random-init Qwen2.5-7B architecture in bf16 on the GPU (no checkpoint)."""
    import torch
    from transformers import Qwen2ForCausalLM
    cfg = qwen2_7b_config(layers)
    torch.manual_seed(seed)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(torch.float32)
    model.eval()
    return model


def prompt_ids(seq, seed=17, vocab=152064):
    import torch
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (1, seq), generator=gen).to("cuda")


def time_prefills(model, backend, ids, cases, repeats, alpha, context):
    """evaluate.py:323-345 and 630-663: every case warmed up once, then ``repeats``
    rounds in rotated case order, each prefill timed from a synchronised start
    through ``model(ids, use_cache=True, logits_to_keep=1)`` and the argmax to a
    synchronised end, all inside ``context`` (the SDPA backend pin) and inference
    mode, with the peak allocated / reserved device memory of each timed prefill
    (torch's counters reset at its start, evaluate.py:328, 338-339). ``cases``:
    (label, method, dense_impl). Returns label -> list of ms, label -> first greedy
    id and label -> list of (peak allocated GiB, peak reserved GiB)."""
    import torch

    def prefill(method, dense_impl):
        backend.configure(method, alpha)
        backend.dense_impl = dense_impl
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
        token = out.logits[:, -1].argmax(dim=-1)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1000.0
        peak = (torch.cuda.max_memory_allocated() / 2 ** 30,
                torch.cuda.max_memory_reserved() / 2 ** 30)
        del out
        return ms, int(token.item()), peak

    times = {label: [] for label, _, _ in cases}
    peaks = {label: [] for label, _, _ in cases}
    tokens = {}
    with torch.inference_mode(), context:
        for label, method, impl in cases:           # warm-up (evaluate.py:634-644)
            _, tokens[label], _ = prefill(method, impl)
        for r in range(repeats):                     # rotated order (evaluate.py:646-663)
            order = cases[r % len(cases):] + cases[:r % len(cases)]
            for label, method, impl in order:
                ms, _, peak = prefill(method, impl)
                times[label].append(ms)
                peaks[label].append(peak)
    return times, tokens, peaks


def median(values):
    v = sorted(values)
    return v[len(v) // 2]


def run_model(seq, layers, repeats, seed, methods, alpha, decode_tokens, split_last=False):
    import torch
    from exp3_amd import _lib, attention
    _lib.load()
    backend = attention.AttentionBackend(alpha=alpha)   # registers as transformers' "sdpa"
    probe = probe_sdpa_backends()
    context, sdpa_name = dense_sdpa_context(probe)
    print(json.dumps({"sweep": "model-sdpa", "probe": probe, "dense_backend": sdpa_name}),
          flush=True)
    model = build_qwen2_7b(layers, seed)
    params = sum(p.numel() for p in model.parameters())
    ids = prompt_ids(seq, seed, model.config.vocab_size)
    cases = [(m, m, "sdpa") for m in methods]
    if "dense" in methods:
        cases.append(("dense_hip", "dense", "hip"))
    times, tokens, peaks = time_prefills(model, backend, ids, cases, repeats, alpha, context)
    dense_ms = median(times["dense"]) if "dense" in times else None
    for label, method, impl in cases:
        med = median(times[label])
        print(json.dumps({"sweep": "model", "method": label,
                          "alpha": alpha if method != "dense" else None,
                          "dense_backend": (sdpa_name if impl == "sdpa" else "hip attn_kernel")
                          if method == "dense" else None,
                          "seq": seq, "layers": layers, "params": params,
                          "prefill_ms_median": round(med, 1),
                          "prefill_ms_all": [round(x, 1) for x in times[label]],
                          "first_token_id": tokens[label],
                          "peak_allocated_gib": round(max(p[0] for p in peaks[label]), 3),
                          "peak_reserved_gib": round(max(p[1] for p in peaks[label]), 3),
                          "speedup_vs_dense": round(dense_ms / med, 3) if dense_ms else None}),
              flush=True)
    backend.dense_impl = "sdpa"

    def prefill(method):
        backend.configure(method, alpha)
        with torch.no_grad():
            out = model(ids, use_cache=True, logits_to_keep=1)
        return out, out.logits[:, -1].argmax(-1)

    if split_last:   # evaluate.py:357-380, split_last_prompt_token=True (not timed)
        for m in methods:
            _, full_token = prefill(m)
            with torch.no_grad():
                pre = model.model(input_ids=ids[:, :-1], use_cache=True)
                step = model(input_ids=ids[:, -1:], past_key_values=pre.past_key_values,
                             use_cache=True, logits_to_keep=1,
                             cache_position=torch.tensor([seq - 1], device="cuda"))
                split_token = step.logits[:, -1].argmax(-1)
            del pre, step
            print(json.dumps({"sweep": "model-split-last-token", "method": m, "seq": seq,
                              "full_prefill_id": int(full_token.item()),
                              "split_id": int(split_token.item())}), flush=True)
    # greedy dense decode (not timed): exercises the backend's decode branch
    out, token = prefill("dense")
    cache = out.past_key_values
    generated = [int(token.item())]
    with torch.no_grad():
        for _ in range(decode_tokens):
            step = model(token[:, None], past_key_values=cache, use_cache=True, logits_to_keep=1)
            cache = step.past_key_values
            token = step.logits[:, -1].argmax(-1)
            generated.append(int(token.item()))
    print(json.dumps({"sweep": "model-decode", "tokens": decode_tokens,
                      "cache_len": seq + decode_tokens, "first_ids": generated[:8]}), flush=True)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description="measurement sweeps (one GPU)")
    sub = p.add_subparsers(dest="cmd", required=True)
    n = sub.add_parser("needles")
    n.add_argument("--seq", type=int, default=32640)
    n.add_argument("--needles", type=int, default=64)
    n.add_argument("--seed", type=int, default=17)
    lo = sub.add_parser("long")
    lo.add_argument("--seq", type=int, default=131072)
    lo.add_argument("--needles", type=int, default=256)
    lo.add_argument("--seed", type=int, default=17)
    sp = sub.add_parser("sparse")
    sp.add_argument("--seq", type=int, default=32640)
    sp.add_argument("--seed", type=int, default=17)
    sp.add_argument("--qk-scale", type=float, default=4.0)
    d2 = sub.add_parser("d256")
    d2.add_argument("--seq", type=int, default=32640)
    d2.add_argument("--seed", type=int, default=17)
    po = sub.add_parser("pair-overlap")
    po.add_argument("--seq", type=int, default=32640)
    po.add_argument("--seed", type=int, default=17)
    po.add_argument("--qk-scale", type=float, default=4.0)
    po.add_argument("--alpha", type=float, default=0.7)
    cm = sub.add_parser("cost-model")
    cm.add_argument("--seq", type=int, default=32640)
    cm.add_argument("--seed", type=int, default=17)
    xb = sub.add_parser("xcd-balance")
    xb.add_argument("--seq", type=int, default=32640)
    xb.add_argument("--seed", type=int, default=17)
    xb.add_argument("--qk-scale", type=float, default=4.0)
    xb.add_argument("--alpha", type=float, default=0.7)
    xb.add_argument("--costs", default="12.6,3.45,2.02",
                    help="microseconds per CU: fixed per workgroup, shared step, one-sided step")
    ro = sub.add_parser("route")
    ro.add_argument("--cases", default="32640:128:28,32640:256:16,131072:128:28")
    ro.add_argument("--seed", type=int, default=17)
    mo = sub.add_parser("model")
    mo.add_argument("--seq", type=int, default=32640)
    mo.add_argument("--layers", type=int, default=28)
    mo.add_argument("--repeats", type=int, default=3)
    mo.add_argument("--seed", type=int, default=17)
    mo.add_argument("--alpha", type=float, default=0.08)
    mo.add_argument("--decode-tokens", type=int, default=128)
    mo.add_argument("--split-last-token", action="store_true")
    mo.add_argument("--methods", default="dense,fp_v1,mean_native,mean_balanced,cgf_mean,dispersion_mean")
    args = p.parse_args(argv)
    if args.cmd == "needles":
        cases = [(m, a) for a in (0.04, 0.08, 0.16) for m in MEAN_FOUR]
        cases += [("fp_v1", 0.08), ("dense", 0.08)]
        run_layer_sweep(args.seq, args.needles, args.seed, cases, "needles")
    elif args.cmd == "sparse":
        run_sparse(args.seq, args.seed, args.qk_scale)
    elif args.cmd == "d256":
        run_d256(args.seq, args.seed)
    elif args.cmd == "pair-overlap":
        run_pair_overlap(args.seq, args.seed, args.qk_scale, args.alpha)
    elif args.cmd == "route":
        run_route([tuple(int(x) for x in c.split(":")) for c in args.cases.split(",")], args.seed)
    elif args.cmd == "cost-model":
        run_cost_model(args.seq, args.seed)
    elif args.cmd == "xcd-balance":
        run_xcd_balance(args.seq, args.seed, args.qk_scale, args.alpha,
                        tuple(float(x) for x in args.costs.split(",")))
    elif args.cmd == "long":
        cases = [("cgf_mean", 0.04), ("dispersion_mean", 0.04), ("mean_native", 0.04)]
        run_layer_sweep(args.seq, args.needles, args.seed, cases, "long")
    else:
        run_model(args.seq, args.layers, args.repeats, args.seed, args.methods.split(","),
                  args.alpha, args.decode_tokens, args.split_last_token)
    return 0


if __name__ == "__main__":
    sys.exit(main())
