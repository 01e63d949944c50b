"""Build libpegaflow_hip.so (gfx950) in-tree with hipcc.

Usage: python -m pegaflow_amd.build [--verbose]
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpegaflow_hip.so")
# Single-block copy latency benchmark (the reference's pinned_copy bench).
BENCH_PINNED_COPY = os.path.join(HERE, "bench_pinned_copy")
# Host-link bandwidth of each copy engine.
BENCH_COPY_ENGINES = os.path.join(HERE, "bench_copy_engines")
ARCH = "gfx950"

SOURCES = [
    "pf_layout.cpp",
    "pf_runtime.cpp",
    "pf_kernels.hip",
    "pf_transfer.cpp",
    "pf_load_state.cpp",
    "pf_engine.cpp",
    "pf_disk.cpp",
    "pf_requests.cpp",
    "pf_hpack.cpp",
    "pf_grpc.cpp",
]

# Packed-FP32 instructions are disabled for all device code (this library
# has no floating-point arithmetic, so the flag costs nothing).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build)")


def build(verbose: bool = False) -> str:
    """Compile every source into LIB; always recompiles."""
    cc = hipcc()
    objs_dir = os.path.join(ROOT, "_build")
    os.makedirs(objs_dir, exist_ok=True)
    objs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(objs_dir, src + ".o")
        cmd = [cc, *HIP_FLAGS, "-c", path, "-o", obj]
        if not src.endswith(".hip"):
            cmd[1:1] = ["-x", "hip"]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib", "-Wl,--no-undefined", "-L/opt/rocm/lib",
           "-lhsa-runtime64", "-lpthread", "-lrt"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_bench(cc, verbose)
    return LIB


def build_bench(cc: str, verbose: bool = False) -> None:
    """The benchmark binaries, linked against the library next to them."""
    for name, out in (("bench_pinned_copy.cpp", BENCH_PINNED_COPY),
                      ("bench_copy_engines.cpp", BENCH_COPY_ENGINES)):
        src = os.path.join(CSRC, name)
        tmp = out + ".tmp"
        cmd = [cc, *HIP_FLAGS, "-x", "hip", src, "-o", tmp, "-L", HERE, "-lpegaflow_hip",
               "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib", "-L/opt/rocm/lib",
               "-lhsa-runtime64"]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {name}:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, out)


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
