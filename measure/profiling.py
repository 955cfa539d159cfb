"""Profiling helpers: workloads to run under ``rocprofv3`` and the HBM-traffic
reduction that ``bench.py`` reports as ``roofline.traffic``.

Workloads (run as the program after ``rocprofv3 ... --``):
  python -m measure.profiling attention [--seq 32640] [--method mean_native] [--repeats 2]
                                        [--qk-scale 4 --alpha 0.7]  (sparse selections)
                                         [--q-heads 28 --kv-heads 4 --head-dim 128] [--dense-impl sdpa]
      one prefill attention layer (pool, route, attention) per repeat, as bench.py runs it
  python -m measure.profiling gemm [--n 16384] [--repeats 3]
      the hipBLASLt bf16 GEMM bench.py reports as the achievable MFMA ceiling
  python -m measure.profiling copy [--gib 1]
      a plain device copy of known size (torch copy_), the calibration for the
      FETCH_SIZE / WRITE_SIZE counters

Reduction:
  python -m measure.profiling traffic --attn-fetch DIR --attn-write DIR \
      --copy-fetch DIR --copy-write DIR [--copy-gib 1] [--key mean_native:32640] \
      [--out profiles/hbm_traffic.json]
      reads the counter_collection CSVs of four ``rocprofv3 --pmc FETCH_SIZE`` /
      ``--pmc WRITE_SIZE`` runs, scales each attention counter by (known copy
      bytes / what the counter read for the copy) and stores the attention
      kernel's HBM bytes per launch under ``key``.
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
KIB = 1024


def counter_per_dispatch(directory: str | Path, kernel_regex: str, counter: str) -> list[float]:
    """Values of ``counter`` (summed over its instances) for every dispatch of a
    kernel matching ``kernel_regex`` in a rocprofv3 --pmc output directory."""
    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {directory}")
    per = defaultdict(float)
    pattern = re.compile(kernel_regex)
    for row in csv.DictReader(open(files[0])):
        if row["Counter_Name"] != counter or not pattern.search(row["Kernel_Name"]):
            continue
        per[row["Dispatch_Id"]] += float(row["Counter_Value"])
    return [per[d] for d in sorted(per, key=int)]


def _median(values: list[float]) -> float:
    if not values:
        raise ValueError("no matching dispatches")
    v = sorted(values)
    return v[len(v) // 2]


def traffic(args) -> dict:
    copy_bytes = args.copy_gib * (1 << 30)
    fetch_copy = _median(counter_per_dispatch(args.copy_fetch, args.copy_kernel, "FETCH_SIZE")) * KIB
    write_copy = _median(counter_per_dispatch(args.copy_write, args.copy_kernel, "WRITE_SIZE")) * KIB
    fetch_scale = copy_bytes / fetch_copy
    write_scale = copy_bytes / write_copy
    fetch = _median(counter_per_dispatch(args.attn_fetch, args.attn_kernel, "FETCH_SIZE")) * KIB
    write = _median(counter_per_dispatch(args.attn_write, args.attn_kernel, "WRITE_SIZE")) * KIB
    entry = {
        "bytes_per_launch": int(round(fetch * fetch_scale + write * write_scale)),
        "read_bytes": int(round(fetch * fetch_scale)),
        "write_bytes": int(round(write * write_scale)),
        "fetch_size_scale": round(fetch_scale, 4),
        "write_size_scale": round(write_scale, 4),
        "kernel": args.attn_kernel,
        "calibration": f"{args.copy_gib} GiB device copy ({args.copy_kernel})",
    }
    out = Path(args.out)
    data = json.loads(out.read_text()) if out.exists() else {}
    data[args.key] = entry
    out.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")
    return entry


def run_attention(args) -> None:
    import torch
    from exp3_amd import _lib, attention, synthetic
    _lib.load()
    q, k, v, _ = synthetic.make_inputs(args.seq, seed=args.seed, q_heads=args.q_heads,
                                       kv_heads=args.kv_heads, head_dim=args.head_dim, device="cuda")
    if args.qk_scale != 1.0:   # sharpened scores: sparse selections (the sparse sweep's inputs)
        q = (q.float() * args.qk_scale).to(torch.bfloat16)
        k = (k.float() * args.qk_scale).to(torch.bfloat16)
    backend = attention.AttentionBackend(alpha=args.alpha, register=False,
                                         dense_impl=args.dense_impl)
    backend.configure(args.method, args.alpha)

    class Layer:
        layer_idx = 0

    # the reference's SDPA backend pin (evaluate.py:630), as bench.py applies it
    from measure.sweeps import dense_sdpa_context, probe_sdpa_backends
    context, sdpa_name = dense_sdpa_context(
        probe_sdpa_backends(args.head_dim, args.q_heads, args.kv_heads))
    with context:
        for _ in range(args.repeats):
            backend.forward(Layer(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                            None, args.head_dim ** -0.5)
    torch.cuda.synchronize()
    print(f"attention {args.method} S={args.seq} x{args.repeats} done (SDPA pinned to "
          f"{sdpa_name})", flush=True)


def run_gemm(args) -> None:
    """The achievable-peak reference bench.py times: a bf16 GEMM (hipBLASLt through
    torch.matmul) on N(0,1) operands, ``repeats`` times."""
    import torch
    n = args.n
    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    for _ in range(args.repeats):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    print(f"gemm {n}^3 x{args.repeats} done", flush=True)


def run_copy(args) -> None:
    import torch
    n = int(args.gib * (1 << 30)) // 2
    a = torch.randn(n, dtype=torch.bfloat16, device="cuda")
    b = torch.empty_like(a)
    for _ in range(args.repeats):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copy {args.gib} GiB x{args.repeats} done", flush=True)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description="profiling workloads and HBM-traffic reduction")
    sub = p.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("attention")
    a.add_argument("--seq", type=int, default=32640)
    a.add_argument("--method", default="mean_native")
    a.add_argument("--alpha", type=float, default=0.08)
    a.add_argument("--seed", type=int, default=17)
    a.add_argument("--repeats", type=int, default=2)
    a.add_argument("--q-heads", type=int, default=28)
    a.add_argument("--kv-heads", type=int, default=4)
    a.add_argument("--head-dim", type=int, default=128)
    a.add_argument("--dense-impl", default="sdpa", choices=("sdpa", "hip"))
    a.add_argument("--qk-scale", type=float, default=1.0,
                   help="multiply Q and K (bf16) to sharpen the routing, as the sparse sweep")
    g = sub.add_parser("gemm")
    g.add_argument("--n", type=int, default=16384)
    g.add_argument("--repeats", type=int, default=3)
    c = sub.add_parser("copy")
    c.add_argument("--gib", type=float, default=1.0)
    c.add_argument("--repeats", type=int, default=3)
    t = sub.add_parser("traffic")
    t.add_argument("--attn-fetch", required=True)
    t.add_argument("--attn-write", required=True)
    t.add_argument("--copy-fetch", required=True)
    t.add_argument("--copy-write", required=True)
    t.add_argument("--copy-gib", type=float, default=1.0)
    t.add_argument("--attn-kernel", default=r"attn_kernel")
    t.add_argument("--copy-kernel", default=r"copyBuffer|copy")
    t.add_argument("--key", default="mean_native:32640")
    t.add_argument("--out", default=str(ROOT / "profiles" / "hbm_traffic.json"))
    args = p.parse_args(argv)
    if args.cmd == "attention":
        run_attention(args)
    elif args.cmd == "copy":
        run_copy(args)
    elif args.cmd == "gemm":
        run_gemm(args)
    else:
        print(json.dumps(traffic(args), indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
