"""Builds libfuriosa_hip.so (the C ABI of include/furiosa_hip.h) for gfx950 with hipcc.

Usage: python furiosa-opt_amd/build.py [--jobs N]

Every translation unit is compiled in parallel into furiosa-opt_amd/_build/ and linked in place
as furiosa-opt_amd/libfuriosa_hip.so, next to the Python binding that loads it.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "libfuriosa_hip.so"
BUILD = HERE / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("FO_OFFLOAD_ARCH", "gfx950")

SOURCES = [
    "mapping.cpp",
    "abi.cpp",
    "k_storage.hip",
    "k_vector.hip",
    "k_gemm.hip",
    "k_gemm_wheels.hip",
    "k_gemv.hip",
    "k_rowops.hip",
    "k_attention.hip",
    "k_mlp.hip",
]

CFLAGS = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    # packed f32 instructions are not emitted (a known-unreliable form on this pool)
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
    # every multiply and add rounds on its own, as Rust computes them (FMA only where written)
    "-ffp-contract=off",
]


# Per-file device flags. The fused row chain runs with f32 denormals flushed (sign kept), the
# reference's own numeric model (furiosa-opt-std/src/float/bf16.rs:16-40 flushes every subnormal).
EXTRA = {
    "k_rowops.hip": ["-fgpu-flush-denormals-to-zero"],
    # no NaN reaches the attention max (inputs are finite bf16), so fmax needs no quieting
    "k_attention.hip": ["-fno-honor-nans"],
}


def compile_one(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *CFLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def stale(src: str) -> bool:
    """The object is older than its source or any header (incremental builds only)."""
    obj = BUILD / (Path(src).stem + ".o")
    if not obj.exists():
        return True
    deps = [CSRC / src, *CSRC.glob("*.hpp"), HERE.parent / "include" / "furiosa_hip.h", Path(__file__)]
    return any(d.stat().st_mtime > obj.stat().st_mtime for d in deps)


def build(jobs: int = 8, incremental: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    todo = [s for s in SOURCES if stale(s)] if incremental else SOURCES
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(compile_one, todo))
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]
    tmp = OUT.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol (e.g. a kernel stub the host pass failed to emit) fails the link
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    # recompile only translation units older than their sources (build() in __graft_entry__ always
    # compiles everything)
    ap.add_argument("--incremental", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.incremental))
    sys.exit(0)
