"""The engine's host side under sanitizers (CPU only).

tests/native/stress_engine.cpp drives a host-memory engine with a disk tier
from several threads at once (prefix queries that start prefetches into a
pool that evicts constantly, prefix counts, byte-checked slot reads,
statistics, instance churn).  It is built from the library's own sources,
with the sanitizers on the host code only (no device code runs), twice:
ThreadSanitizer, and AddressSanitizer with UndefinedBehaviorSanitizer.
A sanitizer report fails the run through the sanitizer's exit code.
The reference has no sanitizer runs and a known race of its own
(lib.rs:608-612).
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pegaflow_amd", "csrc")
LIB_SOURCES = [os.path.join(CSRC, f) for f in (
    "pf_layout.cpp", "pf_runtime.cpp", "pf_kernels.hip", "pf_transfer.cpp", "pf_load_state.cpp",
    "pf_engine.cpp", "pf_disk.cpp", "pf_requests.cpp", "pf_hpack.cpp", "pf_grpc.cpp")]
NATIVE = os.path.join(ROOT, "tests", "native")
# C++ sources that define device variables.
DEVICE_CPP = {"pf_runtime.cpp"}
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Host-side sanitizers only: each flag is passed to the host compilation.
VARIANTS = {
    "tsan": ("-Xarch_host -fsanitize=thread",
             {"TSAN_OPTIONS": "halt_on_error=1 exitcode=66 second_deadlock_stack=1"}),
    "asan": ("-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
             "-Xarch_host -fno-sanitize-recover=undefined",
             {"ASAN_OPTIONS": "exitcode=67 detect_leaks=1",
              "UBSAN_OPTIONS": "halt_on_error=1 print_stacktrace=1"}),
}


def build(variant: str, main: str = "stress_engine") -> str:
    flags = VARIANTS[variant][0].split()
    out = os.path.join(ROOT, "_build", f"native-{variant}")
    os.makedirs(out, exist_ok=True)
    exe = os.path.join(out, main)
    SOURCES = LIB_SOURCES + [os.path.join(NATIVE, main + ".cpp")]
    deps = SOURCES + [os.path.join(CSRC, f) for f in os.listdir(CSRC)] + [
        os.path.join(ROOT, "include", "pegaflow_hip.h"), os.path.abspath(__file__)]
    newest = max(os.path.getmtime(p) for p in deps)
    if os.path.exists(exe) and os.path.getmtime(exe) > newest:
        return exe
    common = ["-x", "hip", "--offload-arch=gfx950", "-O1", "-g", "-std=c++17",
              "-fno-omit-frame-pointer", "-Xclang", "-target-feature", "-Xclang",
              "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", *flags]

    def compile_one(src):
        obj = os.path.join(out, os.path.basename(src) + ".o")
        # Only the files with device code (the kernels, and the runtime's
        # static scratch array) need their device pass (the link resolves
        # their fat binaries); the others are compiled for the host alone.
        device = src.endswith(".hip") or os.path.basename(src) in DEVICE_CPP
        host_only = [] if device else ["--offload-host-only"]
        subprocess.run([HIPCC, *common, *host_only, "-c", src, "-o", obj], check=True,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        return obj

    with ThreadPoolExecutor(max_workers=4) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    subprocess.run([HIPCC, "--offload-arch=gfx950", *flags, "-o", exe, *objs, "-L/opt/rocm/lib",
                    "-lhsa-runtime64", "-lpthread", "-lrt"],
                   check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return exe


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_engine_stress_under_sanitizer(variant, tmp_path):
    exe = build(variant)
    env = dict(os.environ, **VARIANTS[variant][1])
    r = subprocess.run([exe, str(tmp_path / "pega"), "2.0"], env=env, timeout=300,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-6000:]
    assert "bad 0" in r.stdout


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_tinylfu_sketch_rules():
    """tests/native/lfu_test.cpp under AddressSanitizer+UBSan: the sketch's
    sizing as cache.rs computes it, the count-min property against exact
    counts, halving at the window's end, saturation at 255."""
    exe = build("asan", "lfu_test")
    env = dict(os.environ, **VARIANTS["asan"][1])
    r = subprocess.run([exe], env=env, timeout=120, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-6000:]
    assert r.stdout.strip().endswith("ok")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_block_store_sealing_rules(variant):
    """tests/native/blockstore_test.cpp under AddressSanitizer+UBSan and
    under ThreadSanitizer: whole calls, blocks completed across calls (first
    copies win), sealed blocks not replaced, a key named twice, a slot count
    mismatch, TinyLFU admission, eviction by bytes, and allocations racing a
    monitor thread's evictions."""
    exe = build(variant, "blockstore_test")
    env = dict(os.environ, **VARIANTS[variant][1])
    r = subprocess.run([exe], env=env, timeout=120, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-6000:]
    assert r.stdout.strip().endswith("ok")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_hpack_decoder_rfc7541_examples():
    """tests/native/hpack_test.cpp under AddressSanitizer+UBSan: the native
    gRPC server's HPACK decoder against RFC 7541 Appendix C (integers, three
    requests with and without Huffman coding through one dynamic table) and
    malformed blocks."""
    exe = build("asan", "hpack_test")
    env = dict(os.environ, **VARIANTS["asan"][1])
    r = subprocess.run([exe], env=env, timeout=120, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-6000:]
    assert r.stdout.strip().endswith("ok")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_grpc_server_under_sanitizer(variant):
    """tests/native/grpc_stress.cpp: the native gRPC server with 4 raw HTTP/2
    clients keeping 4 requests in flight each (replies from the connection's
    thread and from the handler on worker threads), PINGs, and a stop with
    the connections open, under each sanitizer."""
    exe = build(variant, "grpc_stress")
    env = dict(os.environ, **VARIANTS[variant][1])
    r = subprocess.run([exe], env=env, timeout=300, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-6000:]
    assert r.stdout.strip().endswith("ok")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_staged_slicing_rules():
    """tests/native/staged_plan_test.cpp under AddressSanitizer+UBSan: the
    staged mode's slices for a Llama-3-8B prefix load and save and a
    tensor-parallel rank's load (sizes worked out by hand), empty, in-place
    and oversized layers, and 3000 random calls against the rules every cut
    keeps (each chunk once in order, slice sizes, contiguous descriptors,
    layers done in order with their last slice)."""
    exe = build("asan", "staged_plan_test")
    env = dict(os.environ, **VARIANTS["asan"][1])
    r = subprocess.run([exe], env=env, timeout=120, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-6000:]
    assert r.stdout.strip().endswith("ok")
