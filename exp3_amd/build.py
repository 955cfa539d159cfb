"""In-tree build of the gfx950 HIP library ``exp3_amd/_C/libexp3_amd.so``.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 only and links one shared
library exporting the C ABI declared in ``include/sparse_prefill.h``. Packed
FP32 instructions are disabled for all device code.

Usage: ``python -m exp3_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
REPO = PACKAGE.parent
CSRC = PACKAGE / "csrc"
OUT_DIR = PACKAGE / "_C"
LIBRARY = OUT_DIR / "libexp3_amd.so"
BUILD_DIR = REPO / "_build"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
]


# Per-source additions. attn256.hip: the d = 256 attention kernel's O accumulator
# (128 registers) plus Q (64) fill the 256 VGPRs; in the default AGPR form of the
# MFMA accumulators the register allocator then keeps O in AGPRs across the loop
# and copies all 128 registers in and out every iteration (8 extra instructions per
# MFMA). The VGPR form keeps O where it is accumulated: 12.1 -> 8.2 ms per
# 32640-token layer.
# route.hip: the V1 score reduction reads every MFMA result with VALU instructions;
# in the VGPR form they read the accumulators in place instead of copying them out
# of AGPRs first (16 copies per 32-block chunk and wave).
# selectors.hip: the MFMAs accumulate in VGPRs so that the AGPR file is free to hold
# the parked logits of up to 12 chunks (192 registers); the stored-chunk loop must
# be unrolled in full (its register array indexed by constants), which a 12-chunk
# body exceeds under the default unroll threshold (the array then went to scratch).
EXTRA_FLAGS = {"attn256.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               "route.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               "selectors.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form",
                                 "-mllvm", "-pragma-unroll-threshold=1000000"]}


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(hipcc: str, source: Path) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line.
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(lambda s: _compile(hipcc, s), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY.relative_to(REPO)} from {len(sources)} sources", flush=True)
    return LIBRARY


if __name__ == "__main__":
    build()
