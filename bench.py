#!/usr/bin/env python3
"""KV save/restore benchmark of the MI355X transfer path.

Workload (the reference's Llama-3.1-8B 10K-token prefix): 32 bf16 layers of
[2, 20000, 16, 8, 128] resident in HBM (64 KiB per block per layer), a prefix
of 640 blocks drawn uniformly at random without replacement.  One step is a
full save of the prefix to the pinned host pool (in the reference's split
K/V host layout) followed by a full restore of it into 640 other random
blocks: P = 1,342,177,280 payload bytes cross the host link in each
direction.  By default the save runs in PF_MODE_AUTO (staged: an HBM gather
and copy-engine DMA, the engine's deployed mode) and the restore by the
zero-copy kernel (--save-mode / --load-mode change them).

Printed JSON line (stdout):
  value            save+restore payload GB/s over the timed steps (2P/step)
  restore_*        host -> HBM restore: GB/s, ms per prefix, fraction of the
                   measured host-link peak (best 1 GiB hipMemcpyAsync) and of
                   PCIe Gen5 x16 (63.0 GB/s)
  save_*           HBM -> host save, same figures
  roofline         the timed step's dominant kernel, the zero-copy restore
                   (pinned host -> paged HBM over the host link): P per call /
                   its kernel time (HIP events on the context's stream), vs
                   PCIe Gen5 x16 and vs the measured H2D peak; the save beside
                   it (staged: its link rate by wall clock); traffic from the
                   committed rocprofv3 summary it names (traffic_source)
  device_gather    the HBM-bound gather of the staged mode (paged layers ->
                   packed HBM buffer, all 32 layers in one launch): 2P per
                   launch / its duration, vs 8 TB/s; also the same kernel on
                   a plain contiguous copy of 2P bytes and its fraction
  device_scatter   the staged mode's scatter (packed HBM -> paged layers)
  cpu_baseline     the reference's copy pattern (per-segment save copies,
                   merged-run restore copies) as host memcpy, one thread per
                   physical core of the GPU's NUMA node, on a bounded sample
                   of the same workload, byte-checked
  variants         the same prefix in every transfer mode: the reference's
                   copy pattern (dma_reference), merged-run async copies
                   (dma_batched), the zero-copy kernel and the staged mode
                   (skipped with --quick unless --variants)
  deployed         the engine's default pair (AUTO both ways: staged on the
                   copy engines) against the link's peak, from variants
  other workloads  (skipped with --quick) gpt2_config1, layerwise_qwen3_8b, mla_latent,
                   tp8_rank_llama3_8b, fragmentation_llama3_8b,
                   engine_llama3_8b, two_process_llama3_8b, disk_tier_llama3_8b and
                   pinned_copy_microbench (single-block copy latency)
Everything else goes to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import shutil
import statistics
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
PCIE_GEN5_X16_GBPS = 63.0
GiB = 1 << 30


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--save-mode", default="auto",
                    choices=["dma_reference", "dma_batched", "kernel", "staged", "auto"])
    ap.add_argument("--load-mode", default="kernel",
                    choices=["dma_reference", "dma_batched", "kernel", "staged", "auto"])
    ap.add_argument("--variants", action="store_true",
                    help="also time every transfer mode with --quick (always done without it)")
    ap.add_argument("--sweep", action="store_true",
                    help="also sweep the gather kernel's launch shape")
    ap.add_argument("--threads", type=int, default=0, help="kernel workgroup size (0: default)")
    ap.add_argument("--unroll", type=int, default=0,
                    help="16-byte loads in flight per lane, +256 for non-temporal (0: default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true",
                    help="skip the config 3/4/5 legs (layer-wise, fragmentation, MLA) and "
                         "the disk-tier leg")
    ap.add_argument("--profile", choices=["gather", "scatter", "scatter_sets", "zerocopy"],
                    help="only run the calibration copy and one kernel's launches (PMC passes)")
    ap.add_argument("--profile-gather", action="store_const", const="gather", dest="profile",
                    help="same as --profile gather")
    ap.add_argument("--sweep-scatter", action="store_true",
                    help="also sweep the device scatter's launch shape and chunk order")
    ap.add_argument("--scatter-spread", action="store_true",
                    help="also time the device scatter and gather with the 640 blocks spread "
                         "over all 20,000, a narrower range, or consecutive")
    ap.add_argument("--duplex-study", action="store_true",
                    help="also time each link direction against a plain DMA copy the other way, "
                         "and the two queued kernels' grids in duplex")
    ap.add_argument("--interference-study", action="store_true",
                    help="only run the cross-process interference study (one JSON line)")
    ap.add_argument("--first-layer-study", action="store_true",
                    help="only run the first-layer study: layer-by-layer restores beside a "
                         "GEMM in another process (one JSON line)")
    ap.add_argument("--cu-masks", default="",
                    help="with --first-layer-study: also run the staged variants on contexts "
                         "masked to these compute units per XCD, e.g. '1,2,4'")
    ap.add_argument("--study-engines", default="",
                    help="with --interference-study: staged phases only, once per copy-engine "
                         "pair, e.g. '0x2:0x1,0x8:0x4' (device-to-host mask:host-to-device mask)")
    ap.add_argument("--leg", choices=["gpt2", "layerwise", "mla", "tp8", "fragmentation",
                                      "engine", "two_process", "disk"],
                    help="only run this one workload and print its JSON")
    ap.add_argument("--study-victims", default="",
                    help="with --interference-study: comma-separated victims (default: all)")
    ap.add_argument("--pinned-flags", type=int, default=0,
                    help="PF_PINNED_* flags of the pinned pools (0: mapped, portable)")
    ap.add_argument("--cpu-sample-layers", type=int, default=8)
    ap.add_argument("--staging-mib", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args()


def timed(fn, reps=1):
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def link_peaks(pool, scratch, stream):
    """Best of 10 1-GiB pinned<->device hipMemcpyAsync per direction, and a
    1-GiB device-to-device copy, each timed with HIP events on its stream
    (GB/s, decimal; D2D counts read + write)."""
    from pegaflow_amd import runtime

    dst = runtime.DeviceBuffer(GiB)
    start, end = runtime.Event(), runtime.Event()

    def best(d, s, bytes_counted):
        ms = []
        for _ in range(11):
            start.record(stream)
            runtime.memcpy_async(d, s, GiB, stream)
            end.record(stream)
            end.synchronize()
            ms.append(start.elapsed_ms(end))
        return bytes_counted / (min(ms[1:]) / 1e3) / 1e9

    h2d = best(scratch.ptr, pool.ptr, GiB)
    d2h = best(pool.ptr, scratch.ptr, GiB)
    d2d = best(dst.ptr, scratch.ptr, 2 * GiB)
    dst.close()
    return h2d, d2h, d2d


def duplex(xfer_save, xfer_load, saved, loads, mode, reps=5):
    """Save of one prefix and restore of another issued together on two
    transfer contexts (the engine's save and load workers): aggregate payload
    GB/s with both link directions busy."""
    ts = []
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        xfer_load.load_layers(loads, mode)   # asynchronous
        xfer_save.save_layers(saved, mode)   # returns when saved
        xfer_load.synchronize()
        ts.append(time.perf_counter() - t0)
    return min(ts[1:])


def duplex_threads(xfer_save, xfer_load, saved, loads, mode, reps=5):
    """As duplex, with the restore issued from a second thread, as the
    engine's load thread does (a staged restore on the copy engines returns
    once its copies are done)."""
    import threading

    ts = []
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        th = threading.Thread(target=lambda: (xfer_load.load_layers(loads, mode),
                                              xfer_load.synchronize()))
        th.start()
        xfer_save.save_layers(saved, mode)
        th.join()
        ts.append(time.perf_counter() - t0)
    return min(ts[1:])


def leg_interference(layers, saved, loads, P, reps=3):
    """How much each transfer mode slows a kernel running beside it: a plain
    256 MiB device-to-device copy by the chunk kernel, launched back to back
    from the main thread (its kernel time by HIP events) while a thread saves
    or restores the Llama prefix.  Shader reads and writes of host memory
    (the zero-copy kernel) hold up the memory traffic of every other kernel;
    the staged mode's copies run on the copy engines."""
    import threading

    from pegaflow_amd import _lib
    from pegaflow_amd.runtime import DeviceBuffer
    from pegaflow_amd.transfer import KVCacheRegistration, TransferContext
    from pegaflow_amd import workload as wl

    vb = 256 << 20
    vsrc, vdst = DeviceBuffer(vb), DeviceBuffer(vb)
    xv = TransferContext(0)
    creg = KVCacheRegistration.create(vsrc.ptr, vb, vb // 32768, 32768, 0, 1)
    vplan = wl.save_plan([creg], np.arange(vb // 32768), vdst.ptr)
    xv.set_timing(True)
    xt = TransferContext(0, staging_bytes=256 << 20)

    def victim():
        xv.save_layers(vplan, _lib.MODE_KERNEL)
        return xv.last_kernel_ms()[0]

    for _ in range(3):
        victim()
    solo = statistics.median([victim() for _ in range(20)])
    out = {"victim": "256 MiB device-to-device copy (chunk kernel, 512 threads)",
           "victim_solo_ms": round(solo, 4)}
    ops = {
        "kernel_save": lambda: xt.save_layers(saved, _lib.MODE_KERNEL),
        "staged_save": lambda: xt.save_layers(saved, _lib.MODE_STAGED),
        "kernel_restore": lambda: (xt.load_layers(loads, _lib.MODE_KERNEL), xt.synchronize()),
        "staged_restore": lambda: (xt.load_layers(loads, _lib.MODE_STAGED), xt.synchronize()),
    }
    for name, op in ops.items():
        op()
        t_op, times = [], []

        def worker():
            for _ in range(reps):
                t0 = time.perf_counter()
                op()
                t_op.append(time.perf_counter() - t0)

        th = threading.Thread(target=worker)
        th.start()
        time.sleep(0.002)
        while th.is_alive():
            times.append(victim())
        th.join()
        times = times[1:-1] if len(times) > 3 else times
        med = statistics.median(times)
        out[name] = {"victim_ms": round(med, 4), "slowdown": round(med / solo, 2),
                     "victim_launches": len(times),
                     "transfer_gbps": round(P / statistics.median(t_op) / 1e9, 2)}
        log(f"[bench] interference {name}: {out[name]}")
    xt.close()
    xv.close()
    vsrc.close()
    vdst.close()
    return out


STUDY_PHASES = ["idle", "kernel_save", "staged_save", "kernel_restore", "staged_restore"]


def study_phases(engines: str):
    """The study's phases: every mode, or with engine pairs ('d2h:h2d,...')
    the idle phase and then the staged save and restore on each pair, named
    '<mode>@<d2h>:<h2d>'."""
    if not engines:
        return list(STUDY_PHASES)
    phases = ["idle"]
    for pair in engines.split(","):
        d2h, h2d = (int(v, 0) for v in pair.split(":"))
        phases += [f"staged_save@{d2h:#x}:{h2d:#x}", f"staged_restore@{d2h:#x}:{h2d:#x}"]
    return phases


def _study_transfer(go, done, ready, out, phases):
    """Transfer process of the interference study: each phase saves or
    restores the Llama prefix six times while the victim process measures.
    A phase '<mode>@<d2h>:<h2d>' first moves the staged copies to that pair
    of copy engines."""
    from pegaflow_amd import _lib, runtime
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import PinnedBuffer
    from pegaflow_amd.transfer import TransferContext

    runtime.init(0)
    layers = wl.DeviceLayers(wl.LLAMA3_8B, base_seed=0)
    ids, targets = wl.draw_blocks(wl.LLAMA3_8B.num_blocks, 640, 0)
    P = wl.payload_bytes(layers.regs, 640)
    pool = PinnedBuffer(P)
    x = TransferContext(0, staging_bytes=256 << 20)
    saved = wl.save_plan(layers.regs, ids, pool.ptr)
    loads = wl.load_plan(saved, targets)
    ops = {
        "idle": lambda: time.sleep(0.024),
        "kernel_save": lambda: x.save_layers(saved, _lib.MODE_KERNEL),
        "staged_save": lambda: x.save_layers(saved, _lib.MODE_STAGED),
        "kernel_restore": lambda: (x.load_layers(loads, _lib.MODE_KERNEL), x.synchronize()),
        "staged_restore": lambda: (x.load_layers(loads, _lib.MODE_STAGED), x.synchronize()),
    }
    default_engines = runtime.copy_engines(0)

    def engines_for(name):
        if "@" not in name:
            return default_engines
        return tuple(int(v, 0) for v in name.split("@")[1].split(":"))

    for name in phases:
        runtime.set_copy_engines(0, *engines_for(name))
        ops[name.split("@")[0]]()
    ready.set()
    gbps = {}
    for name in phases:
        runtime.set_copy_engines(0, *engines_for(name))
        go.wait()
        go.clear()
        t = []
        for _ in range(6):
            t0 = time.perf_counter()
            ops[name.split("@")[0]]()
            t.append(time.perf_counter() - t0)
        gbps[name] = round(P / statistics.median(t) / 1e9, 2)
        done.set()
    gbps.pop("idle")
    out.put(gbps)


def _study_victim(go, done, ready, kind, out, phases):
    """Victim process: launches its work back to back through each phase of
    the transfer process and reports the median duration."""
    if kind == "gemm_bf16_8192":
        import torch  # initialized here, in a process that never loads the library

        a = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
        c = torch.empty(8192, 8192, device="cuda", dtype=torch.bfloat16)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

        def victim():
            e0.record()
            torch.mm(a, b, out=c)
            e1.record()
            e1.synchronize()
            return e0.elapsed_time(e1)
    else:
        from pegaflow_amd import _lib, runtime
        from pegaflow_amd import workload as wl
        from pegaflow_amd.runtime import DeviceBuffer, Event, PinnedBuffer, Stream
        from pegaflow_amd.transfer import KVCacheRegistration, TransferContext

        runtime.init(0)
        if kind == "hbm_copy_256MiB":
            vb = 256 << 20
            vsrc, vdst = DeviceBuffer(vb), DeviceBuffer(vb)
            xv = TransferContext(0)
            creg = KVCacheRegistration.create(vsrc.ptr, vb, vb // 32768, 32768, 0, 1)
            vplan = wl.save_plan([creg], np.arange(vb // 32768), vdst.ptr)
            xv.set_timing(True)

            def victim():
                xv.save_layers(vplan, _lib.MODE_KERNEL)
                return xv.last_kernel_ms()[0]
        else:
            h, d = PinnedBuffer(1 << 20), DeviceBuffer(1 << 20)
            st, ev = Stream(), Event()

            def victim():
                t0 = time.perf_counter()
                if kind == "copy_64KiB_h2d":
                    runtime.memcpy_async(d.ptr, h.ptr, 65536, st)
                else:
                    runtime.memcpy_async(h.ptr, d.ptr, 65536, st)
                ev.record(st)
                ev.synchronize()
                return (time.perf_counter() - t0) * 1e3
    for _ in range(5):
        victim()
    ready.wait()
    base = None
    res = {}
    for name in phases:
        times = []
        go.set()
        time.sleep(0.003)
        while not done.is_set():
            times.append(victim())
            time.sleep(0.0005 if kind.startswith("copy") else 0)
        done.clear()
        times = times[1:-1] if len(times) > 3 else times
        med = statistics.median(times)
        base = med if base is None else base
        res[name] = {"median_ms": round(med, 4), "slowdown": round(med / base, 2),
                     "n": len(times)}
    out.put(res)


def interference_study(engines: str = "", victim_list: str = ""):
    """Cross-process interference (the engine server beside a vLLM worker):
    for each victim, a transfer process saves and restores the Llama prefix
    in each mode (or staged on each given copy-engine pair) while a victim
    process runs its work back to back.  Prints one JSON line."""
    import multiprocessing as mp

    ctx = mp.get_context("spawn")
    victims = ["hbm_copy_256MiB", "gemm_bf16_8192", "copy_64KiB_h2d", "copy_64KiB_d2h"]
    if victim_list:
        victims = [v for v in victim_list.split(",") if v]
    if "gemm_bf16_8192" in victims:
        try:
            import torch  # noqa: F401  (the GEMM victim needs it)
        except ImportError:
            victims.remove("gemm_bf16_8192")
    phases = study_phases(engines)
    result = {"metric": "interference of each transfer mode with work in another process",
              "transfer": "llama-3.1-8b 10k-token prefix (32 x [2,20000,16,8,128] bf16, "
                          "640 blocks), six calls per phase",
              "phases": phases,
              "victims": {}}
    for kind in victims:
        log(f"[bench] interference study: victim {kind}")
        go, done, ready = ctx.Event(), ctx.Event(), ctx.Event()
        out, tout = ctx.Queue(), ctx.Queue()
        pt = ctx.Process(target=_study_transfer, args=(go, done, ready, tout, phases))
        pv = ctx.Process(target=_study_victim, args=(go, done, ready, kind, out, phases))
        pt.start()
        pv.start()
        res = out.get(timeout=300)
        res["transfer_gbps"] = tout.get(timeout=60)
        pv.join(60)
        pt.join(60)
        if pt.exitcode != 0 or pv.exitcode != 0:
            raise RuntimeError(f"interference study processes exited {pt.exitcode}, "
                               f"{pv.exitcode}")
        result["victims"][kind] = res
    print(json.dumps(result), flush=True)


def _first_layer_victim(go, stop, ready, count):
    """GEMM process of the first-layer study: bf16 8192^3 products back to
    back, two per synchronization, counted in `count`."""
    import torch  # initialized here, in a process that never loads the library

    a = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    c = torch.empty(8192, 8192, device="cuda", dtype=torch.bfloat16)
    for _ in range(3):
        torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    ready.set()
    go.wait()
    while not stop.is_set():
        torch.mm(a, b, out=c)
        torch.mm(a, b, out=c)
        torch.cuda.synchronize()
        with count.get_lock():
            count.value += 2


def first_layer_study(reps=10, cu_masks=()):
    """Layer-by-layer restores of the Llama prefix beside bf16 8192^3 GEMMs
    that another process runs back to back.  Each restore marks its layers
    in pinned host memory; this process polls layer 0's mark while another
    thread issues the load (a staged load returns once its copies are done).
    Variants, interleaved, `reps` loads each: the staged mode with its first
    layer by the zero-copy kernel or by the copy engines (the default;
    pf_xfer_set_staged_head), the kernel mode, and whole loads of both
    modes; with `cu_masks`, the three staged variants again on contexts
    whose kernels run on k compute units of each XCD, for each k.  Reports
    per variant the first layer's latency from the call, the load's rate,
    and the GEMM's rate during the variant's loads against its rate alone;
    then the same loads on an idle device.  Every load's bytes are checked
    on the device.  One JSON line."""
    import multiprocessing as mp
    import threading

    from pegaflow_amd import _lib, runtime
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import PinnedBuffer
    from pegaflow_amd.transfer import TransferContext, cu_mask_per_xcd

    ctx = mp.get_context("spawn")
    go, stop, ready = ctx.Event(), ctx.Event(), ctx.Event()
    count = ctx.Value("l", 0)
    victim = ctx.Process(target=_first_layer_victim, args=(go, stop, ready, count))
    victim.start()
    runtime.init(0)
    shape = wl.LLAMA3_8B
    layers = wl.DeviceLayers(shape, base_seed=0)
    ids, targets = wl.draw_blocks(shape.num_blocks, 640, 0)
    P = wl.payload_bytes(layers.regs, 640)
    pool = PinnedBuffer(P)
    x_kernel_head = TransferContext(0, staging_bytes=512 << 20)
    x_kernel_head.set_staged_head(_lib.STAGED_HEAD_KERNEL)
    x_engine_head = TransferContext(0, staging_bytes=512 << 20)
    x_engine_head.set_staged_head(_lib.STAGED_HEAD_ENGINE)
    saved = wl.save_plan(layers.regs, ids, pool.ptr)
    loads = wl.load_plan(saved, targets)
    x_kernel_head.save_layers(saved, _lib.MODE_KERNEL)
    words = PinnedBuffer(8 * len(loads))
    wv = words.array.view(np.uint64)
    wv[:] = 0
    serial = [0]

    def marked(x, mode):
        serial[0] += 1
        val = serial[0]
        th = threading.Thread(target=lambda: x.load_layers_marked(
            loads, [(words.ptr, val, True)], mode))
        t0 = time.perf_counter()
        th.start()
        while wv[0] != val:
            time.sleep(0)  # lets the issuing thread take the GIL
        t1 = time.perf_counter()
        th.join()
        x.synchronize()
        t2 = time.perf_counter()
        if any(int(w) != val for w in wv):
            raise RuntimeError("a layer's mark is missing after the load")
        return t1 - t0, t2 - t0

    def whole(x, mode):
        t0 = time.perf_counter()
        x.load_layers(loads, mode)
        x.synchronize()
        return None, time.perf_counter() - t0

    variants = {
        "staged_first_layer_by_kernel": lambda: marked(x_kernel_head, _lib.MODE_STAGED),
        "staged_first_layer_by_copy_engine": lambda: marked(x_engine_head, _lib.MODE_STAGED),
        "kernel": lambda: marked(x_kernel_head, _lib.MODE_KERNEL),
        "staged_whole_load": lambda: whole(x_kernel_head, _lib.MODE_STAGED),
        "kernel_whole_load": lambda: whole(x_kernel_head, _lib.MODE_KERNEL),
    }
    masked = []
    for k in cu_masks:
        xk = TransferContext(0, staging_bytes=512 << 20)
        xk.set_cu_mask(cu_mask_per_xcd(k))
        xk.set_staged_head(_lib.STAGED_HEAD_KERNEL)
        xe = TransferContext(0, staging_bytes=512 << 20)
        xe.set_cu_mask(cu_mask_per_xcd(k))
        xe.set_staged_head(_lib.STAGED_HEAD_ENGINE)
        masked += [xk, xe]
        variants.update({
            f"staged_first_layer_by_kernel_{k}_cus_per_xcd":
                lambda xk=xk: marked(xk, _lib.MODE_STAGED),
            f"staged_first_layer_by_copy_engine_{k}_cus_per_xcd":
                lambda xe=xe: marked(xe, _lib.MODE_STAGED),
            f"staged_whole_load_{k}_cus_per_xcd": lambda xk=xk: whole(xk, _lib.MODE_STAGED),
        })
    for f in variants.values():
        f()
    ready.wait()
    go.set()
    time.sleep(0.3)
    c0, t0 = count.value, time.perf_counter()
    time.sleep(1.5)
    solo_rate = (count.value - c0) / (time.perf_counter() - t0)
    # Every load is checked: the tensors are refilled first (each target
    # block then holds its own words, not the ones the load must bring), and
    # every block of every layer is verified after it, outside the timing.
    runs = {k: {"first": [], "load": [], "gemms": 0, "secs": 0.0} for k in variants}
    bad = checked = 0
    for _ in range(reps):
        for name, f in variants.items():
            r = runs[name]
            layers.refill()
            c0, t0 = count.value, time.perf_counter()
            first, load = f()
            r["secs"] += time.perf_counter() - t0
            r["gemms"] += count.value - c0
            if first is not None:
                r["first"].append(first * 1e3)
            r["load"].append(load)
            bad += wl.verify_restored(layers, ids, targets)
            checked += 1
    stop.set()
    victim.join(60)
    if victim.exitcode != 0:
        raise RuntimeError(f"GEMM process exited {victim.exitcode}")
    beside = {}
    for name, r in runs.items():
        e = {"load_gbps": round(P / statistics.median(r["load"]) / 1e9, 2),
             "gemm_slowdown": round(solo_rate / (r["gemms"] / r["secs"]), 3),
             "gemms": r["gemms"]}
        if r["first"]:
            e.update(first_layer_ms=round(statistics.median(r["first"]), 3),
                     first_layer_ms_min=round(min(r["first"]), 3),
                     first_layer_ms_max=round(max(r["first"]), 3))
        beside[name] = e
    idle = {}
    for name, f in variants.items():
        got = []
        for _ in range(5):
            layers.refill()
            got.append(f())
            bad += wl.verify_restored(layers, ids, targets)
            checked += 1
        e = {"load_gbps": round(P / statistics.median([g[1] for g in got]) / 1e9, 2)}
        if got[0][0] is not None:
            e["first_layer_ms"] = round(statistics.median([g[0] for g in got]) * 1e3, 3)
        idle[name] = e
    print(json.dumps({
        "metric": "first layer of a layer-by-layer restore beside a GEMM in another process",
        "transfer": "llama-3.1-8b 10k-token prefix (32 x [2,20000,16,8,128] bf16, 640 blocks), "
                    "each layer marked in pinned host memory",
        "gemm": "bf16 8192^3 torch.mm back to back, two per synchronization",
        "gemm_alone_ms": round(1e3 / solo_rate, 3),
        "loads_per_variant": reps,
        "cu_masks_per_xcd": list(cu_masks),
        "beside_gemm": beside,
        "idle": idle,
        "loads_checked": checked,
        "bit_exact": bad == 0}), flush=True)
    for x in [x_kernel_head, x_engine_head] + masked:
        x.close()
    words.close()
    pool.close()
    layers.close()


def duplex_study(xfer_load, xfer_save, saved, loads, pool, pool2, dev_buf, P, reps=4):
    """Which direction loses bandwidth when both link directions are busy.
    Each case runs a save and a restore of P bytes at once and reports the
    aggregate payload GB/s and each side's own time (HIP events on its
    stream; for a staged side on the copy engines, from its first kernel to
    the context's stream after the call): the two queued kernels, each
    kernel against a plain DMA copy of P contiguous bytes the other way, the
    two DMA copies, the staged pairs, and the kernels with other
    persistent-grid sizes."""
    from pegaflow_amd import _lib, runtime
    from pegaflow_amd.runtime import Event, Stream

    dma = Stream()
    evs = [Event() for _ in range(4)]

    def kernel_save(s0, s1):
        s0.record(xfer_save.stream)
        xfer_save.save_layers(saved, _lib.MODE_KERNEL)
        s1.record(xfer_save.stream)

    def kernel_restore(s0, s1):
        s0.record(xfer_load.stream)
        xfer_load.load_layers(loads, _lib.MODE_KERNEL)
        s1.record(xfer_load.stream)

    def dma_save(s0, s1):  # device -> pinned host, one contiguous copy
        s0.record(dma)
        runtime.memcpy_async(pool2.ptr, dev_buf.ptr, P, dma)
        s1.record(dma)

    def dma_restore(s0, s1):  # pinned host -> device, one contiguous copy
        s0.record(dma)
        runtime.memcpy_async(dev_buf.ptr, pool.ptr, P, dma)
        s1.record(dma)

    import threading

    def case(restore, save):
        best = None
        for _ in range(reps + 1):
            t0 = time.perf_counter()
            # The restore issued from a second thread, as the engine's load
            # thread issues it (a staged restore on the copy engines returns
            # once its copies are done).
            th = threading.Thread(target=restore, args=(evs[0], evs[1]))
            th.start()
            save(evs[2], evs[3])
            th.join()
            xfer_load.synchronize()
            xfer_save.synchronize()
            dma.synchronize()
            wall = time.perf_counter() - t0
            r = (wall, evs[0].elapsed_ms(evs[1]), evs[2].elapsed_ms(evs[3]))
            best = r if best is None or r[0] < best[0] else best
        wall, r_ms, s_ms = best
        return {"gbps": round(2 * P / wall / 1e9, 2), "restore_gbps": round(P / r_ms / 1e6, 2),
                "save_gbps": round(P / s_ms / 1e6, 2)}

    out = {"kernel_restore+kernel_save": case(kernel_restore, kernel_save),
           "kernel_restore+dma_save": case(kernel_restore, dma_save),
           "dma_restore+kernel_save": case(dma_restore, kernel_save)}
    # The DMA pair needs two streams: the restore on the load context's.
    def dma_restore_ctx(s0, s1):
        s0.record(xfer_load.stream)
        runtime.memcpy_async(dev_buf.ptr, pool.ptr, P, xfer_load.stream)
        s1.record(xfer_load.stream)
    out["dma_restore+dma_save"] = case(dma_restore_ctx, dma_save)

    def staged_save(s0, s1):
        s0.record(xfer_save.stream)
        xfer_save.save_layers(saved, _lib.MODE_STAGED)
        s1.record(xfer_save.stream)

    def staged_restore(s0, s1):
        s0.record(xfer_load.stream)
        xfer_load.load_layers(loads, _lib.MODE_STAGED)
        s1.record(xfer_load.stream)

    out["staged_restore+staged_save"] = case(staged_restore, staged_save)
    out["staged_restore+kernel_save"] = case(staged_restore, kernel_save)
    out["kernel_restore+staged_save"] = case(kernel_restore, staged_save)
    for gs, gr in ((16, 64), (32, 32), (32, 128), (64, 64), (24, 48)):
        xfer_save.set_route_grid(_lib.ROUTE_SAVE_HOST, gs)
        xfer_load.set_route_grid(_lib.ROUTE_LOAD_HOST, gr)
        out[f"kernels_grid_save{gs}_restore{gr}"] = case(kernel_restore, kernel_save)
    xfer_save.set_route_grid(_lib.ROUTE_SAVE_HOST, _lib.SAVE_HOST_DEFAULT_GRID)
    xfer_load.set_route_grid(_lib.ROUTE_LOAD_HOST, _lib.LOAD_HOST_DEFAULT_GRID)
    dma.close()
    for k, v in out.items():
        log(f"[bench] duplex study {k}: {v}")
    return out


class GemmLayer:
    """A bf16 GEMM (fp32 accumulation) sized to about `target_ms` alone,
    queued on one of the library's streams: the per-layer compute of a
    layer-wise restore, in place of a spin kernel, so that the restore
    competes with it for CUs and HBM as a model's layers would.  It runs
    through rocBLAS from /opt/rocm, on the HIP runtime this library is built
    against (torch's wheel carries a HIP runtime of its own, which cannot
    share a process with another).  [8192, K] x [K, 8192], column-major,
    with K calibrated in multiples of 512; operands of N(0, 1) values."""

    OP_N, BF16, F32 = 111, 168, 151  # rocblas_operation_none, rocblas_datatype_*

    def __init__(self, stream, target_ms=2.0):
        from pegaflow_amd.runtime import DeviceBuffer, Event

        vp, i32 = ctypes.c_void_p, ctypes.c_int
        lib = ctypes.CDLL("librocblas.so.5")
        lib.rocblas_create_handle.argtypes = [ctypes.POINTER(vp)]
        lib.rocblas_set_stream.argtypes = [vp, vp]
        lib.rocblas_destroy_handle.argtypes = [vp]
        lib.rocblas_gemm_ex.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp, i32, i32, vp, i32,
                                        i32, vp, vp, i32, i32, vp, i32, i32, i32, i32, i32,
                                        ctypes.c_uint32]
        self.lib, self.stream = lib, stream
        self.handle = vp()
        self._check(lib.rocblas_create_handle(ctypes.byref(self.handle)), "create_handle")
        self._check(lib.rocblas_set_stream(self.handle, stream.handle), "set_stream")
        self.alpha, self.beta = ctypes.c_float(1.0), ctypes.c_float(0.0)
        self.m = 8192
        self.e0, self.e1 = Event(), Event()
        self._DeviceBuffer = DeviceBuffer
        self.a = self.b = self.c = None
        k = 20480
        for _ in range(2):
            self._alloc(k)
            ms = self.time_alone(5)
            k = max(512, int(round(k * target_ms / ms / 512)) * 512)
        self._alloc(k)
        self.alone_ms = self.time_alone(10)

    @staticmethod
    def _check(rc, what):
        if rc != 0:
            raise RuntimeError(f"rocblas_{what} failed with status {rc}")

    def _bf16(self, n, seed):
        """n bf16 values of N(0, 1): the top half of each float32."""
        f = np.random.Generator(np.random.PCG64(seed)).standard_normal(n, dtype=np.float32)
        return (f.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)

    def _alloc(self, k):
        self._free()
        m = self.m
        self.k = k
        self.a, self.b = self._DeviceBuffer(2 * m * k), self._DeviceBuffer(2 * k * m)
        self.c = self._DeviceBuffer(2 * m * m)
        self.a.upload(self._bf16(m * k, 1))
        self.b.upload(self._bf16(k * m, 2))

    def _free(self):
        for buf in (self.a, self.b, self.c):
            if buf is not None:
                buf.close()
        self.a = self.b = self.c = None

    def __call__(self):
        m, k = self.m, self.k
        self._check(self.lib.rocblas_gemm_ex(
            self.handle, self.OP_N, self.OP_N, m, m, k, ctypes.byref(self.alpha),
            self.a.ptr, self.BF16, m, self.b.ptr, self.BF16, k, ctypes.byref(self.beta),
            self.c.ptr, self.BF16, m, self.c.ptr, self.BF16, m, self.F32, 0, 0, 0), "gemm_ex")

    def time_alone(self, reps):
        times = []
        for _ in range(reps + 1):
            self.e0.record(self.stream)
            self()
            self.e1.record(self.stream)
            self.e1.synchronize()
            times.append(self.e0.elapsed_ms(self.e1))
        return statistics.median(times[1:])

    def close(self):
        self.stream.synchronize()
        self._free()
        if self.handle:
            self.lib.rocblas_destroy_handle(self.handle)
        self.handle = None


def leg_layerwise(xfer, seed, gemm=True):
    """Config 3: Qwen3-8B shape (36 x [2,16000,16,8,128] bf16), 313 random
    blocks restored one layer at a time; layer l's completion gates layer l's
    compute on a second stream.  Overlap efficiency = 36 x 2 ms / total, with
    the total from the load's first issue to the last compute kernel's end
    (device events).  The serialized figure gates every compute kernel on the
    whole load, as a caller without per-layer completion must.  The marked
    figure restores all layers in one launch whose kernel writes a device
    word per layer, and gates compute kernel l with a bounded device wait on
    word l.  The engine figure restores the same blocks by hash through
    PegaEngine in its default modes (staged on the copy engines, its first
    layer by the kernel) with a layered LoadState carrying device layer
    words, compute kernel l gated on word l.

    The compute is first a 2 ms spin kernel (one lane, no memory traffic: an
    upper bound on overlap), then (``*_gemm`` keys) a bf16 GEMM calibrated
    to about 2 ms alone, which shares CUs and HBM with the restore: its
    efficiency is the 36 GEMMs' time back to back over the gated total, and
    its slowdown the mean gated GEMM's time over its time back to back (HIP
    events around each GEMM in both)."""
    import hashlib

    from pegaflow_amd import _lib
    from pegaflow_amd import workload as wl
    from pegaflow_amd.engine import PegaEngine
    from pegaflow_amd.load_state import LayerWords, PyLoadState
    from pegaflow_amd.runtime import (DeviceBuffer, Event, PinnedBuffer, Stream, spin,
                                      stream_wait_word)

    shape, n, compute_us = wl.QWEN3_8B, 313, 2000
    layers = wl.DeviceLayers(shape, base_seed=seed)
    ids, targets = wl.draw_blocks(shape.num_blocks, n, seed)
    pool = PinnedBuffer(wl.payload_bytes(layers.regs, n))
    saved = wl.save_plan(layers.regs, ids, pool.ptr)
    xfer.save_layers(saved, _lib.MODE_KERNEL)
    loads = wl.load_plan(saved, targets)
    compute = Stream()
    evs = [Event() for _ in range(shape.layers)]
    g0 = [Event() for _ in range(shape.layers)]
    g1 = [Event() for _ in range(shape.layers)]
    start, done = Event(), Event()

    def spin_work():
        spin(compute, compute_us)

    work = [spin_work]  # the per-layer compute of the runs below
    timed = [False]  # events around each layer's compute (the GEMM runs only)

    def layer_work(l):
        if timed[0]:
            g0[l].record(compute)
        work[0]()
        if timed[0]:
            g1[l].record(compute)

    def work_ms():
        if not timed[0]:
            return 0.0
        return statistics.mean(g0[l].elapsed_ms(g1[l]) for l in range(shape.layers))

    def run(layerwise):
        start.record(xfer.stream)
        compute.wait_event(start)
        xfer.load_layers(loads, _lib.MODE_KERNEL, layer_events=evs)
        for l in range(shape.layers):
            compute.wait_event(evs[l] if layerwise else evs[-1])
            layer_work(l)
        done.record(compute)
        done.synchronize()
        xfer.synchronize()
        per_layer = [start.elapsed_ms(evs[0])] + [evs[l - 1].elapsed_ms(evs[l])
                                                   for l in range(1, shape.layers)]
        return start.elapsed_ms(done), per_layer, work_ms()

    words = DeviceBuffer(8 * shape.layers)
    words.memset(0)
    value = [0]

    def run_marked():
        value[0] += 1
        start.record(xfer.stream)
        compute.wait_event(start)
        xfer.load_layers_marked(loads, [(words.ptr, value[0], False)], _lib.MODE_KERNEL)
        for l in range(shape.layers):
            stream_wait_word(compute, words.ptr + 8 * l, value[0], 10_000_000)
            layer_work(l)
        done.record(compute)
        done.synchronize()
        xfer.synchronize()
        return start.elapsed_ms(done), work_ms()

    def run_compute_only():
        start.record(compute)
        for l in range(shape.layers):
            layer_work(l)
        done.record(compute)
        done.synchronize()
        return start.elapsed_ms(done)

    compute_only = min(run_compute_only() for _ in range(3))
    run(True)
    total, per_layer, _ = min((run(True) for _ in range(3)), key=lambda r: r[0])
    serial, _, _ = min((run(False) for _ in range(2)), key=lambda r: r[0])
    run_marked()
    marked, _ = min(run_marked() for _ in range(3))
    gemm_res = {}
    gl = None
    if gemm:
        gl = GemmLayer(compute)
        work[0] = gl
        timed[0] = True
        gemm_only = min(run_compute_only() for _ in range(3))
        gemm_b2b = work_ms()  # one GEMM's time, back to back with the others
        run(True)
        g_total, g_per_layer, g_ms = min((run(True) for _ in range(3)), key=lambda r: r[0])
        run_marked()
        gm_total, gm_ms = min(run_marked() for _ in range(3))
        gemm_res = {
            "gemm_shape": f"bf16 [{gl.m},{gl.k}] x [{gl.k},{gl.m}] (rocBLAS)",
            "gemm_alone_ms": round(gl.alone_ms, 4),
            "gemm_back_to_back_ms": round(gemm_b2b, 4),
            "gemm_only_total_ms": round(gemm_only, 3),
            "events_gemm": {"total_ms": round(g_total, 3),
                            "efficiency": round(gemm_only / g_total, 4),
                            "gemm_ms_mean": round(g_ms, 4),
                            "gemm_slowdown": round(g_ms / gemm_b2b, 3),
                            "first_layer_ms": round(g_per_layer[0], 4),
                            "per_layer_ms_mean": round(sum(g_per_layer[1:]) /
                                                       (len(g_per_layer) - 1), 4)},
            "marked_gemm": {"total_ms": round(gm_total, 3),
                            "efficiency": round(gemm_only / gm_total, 4),
                            "gemm_ms_mean": round(gm_ms, 4),
                            "gemm_slowdown": round(gm_ms / gemm_b2b, 3)},
        }
        work[0] = spin_work
        timed[0] = False
    bad = wl.verify_restored(layers, ids, targets)
    layers.refill()
    # Through the engine, default modes, gated on device layer words.
    eng = PegaEngine(pool_size=wl.payload_bytes(layers.regs, n) + (256 << 20))
    names = [f"layer.{l}" for l in range(shape.layers)]
    for name, r in zip(names, layers.regs):
        eng.register_context_layer("lw", "qwen3", 0, name, r.data_ptr, r.size_bytes, r.num_blocks,
                                   r.bytes_per_block, r.kv_stride_bytes, r.segments, 0, 1,
                                   shape.layers)
    ids_l, tg_l = [int(i) for i in ids], [int(t) for t in targets]
    hashes = [hashlib.sha256(b"qwen3-%d" % i).digest() for i in ids_l]
    eng.batch_save_kv_blocks("lw", 0, 0, [(nm, ids_l, hashes) for nm in names])
    lw = LayerWords(shape.layers, local=True)
    timed_out = DeviceBuffer(4 * shape.layers)

    def run_engine():
        timed_out.memset(0)
        st = PyLoadState(layer_words=lw)
        start.record(compute)
        eng.batch_load_kv_blocks("lw", 0, 0, st.shm_name(), names, tg_l, hashes)
        for l in range(shape.layers):
            lw.wait_on_device(compute, l, 10_000_000, timed_out.ptr + 4 * l)
            layer_work(l)
        done.record(compute)
        done.synchronize()
        while not st.is_ready():
            time.sleep(0.0001)
        if st.get_state() != 1 or timed_out.download().any():
            raise RuntimeError("engine layer-wise restore failed or a device wait timed out")
        return start.elapsed_ms(done), work_ms()

    run_engine()
    engine_total, _ = min(run_engine() for _ in range(3))
    if gl is not None:
        work[0] = gl
        timed[0] = True
        run_engine()
        ge_total, ge_ms = min(run_engine() for _ in range(3))
        gemm_res["engine_gemm"] = {"total_ms": round(ge_total, 3),
                                   "efficiency": round(gemm_res["gemm_only_total_ms"] / ge_total,
                                                       4),
                                   "gemm_ms_mean": round(ge_ms, 4),
                                   "gemm_slowdown": round(ge_ms / gemm_b2b, 3)}
        work[0] = spin_work
        timed[0] = False
        gl.close()
    bad += wl.verify_restored(layers, ids, targets)
    eng.close()
    lw.close()
    timed_out.close()
    ideal = shape.layers * compute_us / 1e3
    out = {
        "workload": "qwen3-8b 5k-token prefix: 36 x bf16 [2,16000,16,8,128], 313 blocks, "
                    "layer-wise restore gating a 2 ms compute kernel per layer",
        "overlap_efficiency": round(ideal / total, 4),
        "total_ms": round(total, 3),
        "compute_ms": ideal,
        "compute_only_ms": round(compute_only, 3),
        "overlap_efficiency_vs_compute_only": round(compute_only / total, 4),
        "serialized_total_ms": round(serial, 3),
        "serialized_efficiency": round(ideal / serial, 4),
        "marked_total_ms": round(marked, 3),
        "marked_efficiency": round(ideal / marked, 4),
        "engine_total_ms": round(engine_total, 3),
        "engine_efficiency": round(ideal / engine_total, 4),
        "first_layer_ms": round(per_layer[0], 4),
        "per_layer_ms_mean": round(sum(per_layer[1:]) / (len(per_layer) - 1), 4),
        "per_layer_ms_max": round(max(per_layer[1:]), 4),
        "layer_bytes": n * 2 * shape.bytes_per_block,
        **gemm_res,
        "bit_exact": bad == 0,
    }
    compute.close()
    words.close()
    pool.close()
    layers.close()
    return out


def leg_fragmentation(layers, xfer, seed, dma_requests=8):
    """Config 4: 64 requests, prefixes of U[1K,16K] tokens (16-token blocks)
    on the Llama layers, block ids as contiguous runs of geometric length
    with mean 1, 4 or 32, or fully sorted (640).  Each request saves its
    blocks to the pinned pool and then restores those bytes into a second
    draw of the same kind, so saves and restores alternate 50/50 and every
    restore is checkable.  Outside the timed calls, the host regions are
    checked after every save and every block of every layer after each
    mean's batch, tracking which block's words each block holds.  Kernel and
    staged modes run all 64 requests; the DMA modes, about 20x slower, the
    first ``dma_requests``, and every mode is also reported on those same
    first requests."""
    from pegaflow_amd import _lib
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import PinnedBuffer

    shape = layers.shape
    pool = PinnedBuffer(1024 * shape.layers * 2 * shape.bytes_per_block)
    out, bad = {}, 0
    for mean_run in (1, 4, 32, wl.SORTED_MEAN_RUN):
        reqs = wl.fragmentation_requests(shape.num_blocks, mean_run, seed=seed)
        layers.refill()
        src_of = np.arange(shape.num_blocks, dtype=np.int64)
        row, row_first = {}, {}
        for name, mode in _lib.MODE_NAMES.items():
            use = reqs if name in ("kernel", "staged") else reqs[:dma_requests]
            moved = t = moved_first = t_first = 0.0
            for i, (ids, targets) in enumerate(use):
                saved = wl.save_plan(layers.regs, ids, pool.ptr)
                loads = wl.load_plan(saved, targets)
                t0 = time.perf_counter()
                xfer.save_layers(saved, mode)
                t1 = time.perf_counter()
                bad += wl.verify_saved(layers, saved, src_of)
                t2 = time.perf_counter()
                xfer.load_layers(loads, mode)
                xfer.synchronize()
                t3 = time.perf_counter()
                src_of[targets] = src_of[ids]
                nbytes = 2 * wl.payload_bytes(layers.regs, len(ids))
                moved += nbytes
                t += (t1 - t0) + (t3 - t2)
                if i < dma_requests:
                    moved_first += nbytes
                    t_first += (t1 - t0) + (t3 - t2)
            row[name] = round(moved / t / 1e9, 2)
            row_first[name] = round(moved_first / t_first / 1e9, 2)
        bad += wl.verify_blocks(layers, src_of)
        runs = float(np.mean([wl.run_count(ids) for ids, _ in reqs]))
        blocks = float(np.mean([len(ids) for ids, _ in reqs]))
        out[f"mean_run_{mean_run}"] = {
            "gbps": row, f"gbps_first_{dma_requests}_requests": row_first,
            "measured_mean_run": round(blocks / runs, 2)}
        log(f"[bench] fragmentation mean_run={mean_run}: {row}; first {dma_requests}: "
            f"{row_first}")
    pool.close()
    layers.refill()
    return {"workload": "64 requests, prefixes U[1K,16K] tokens on llama-3.1-8b layers, each "
                        "saving its blocks and restoring them into a second draw (saves and "
                        "restores 50/50); GB/s = save + restore payload / their time",
            "by_mean_run": out, "dma_modes_timed_on_requests": dma_requests,
            "bit_exact": bad == 0}


def leg_mla(xfer, seed):
    """Config 5: MLA latent, 61 layers [8192, 64, 576] as bf16 and fp8 bytes
    (one segment per block), 128 random blocks saved then restored into 128
    other blocks; bit-exact per dtype, payload GB/s per direction."""
    from pegaflow_amd import _lib
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import PinnedBuffer

    out = {}
    for shape in (wl.MLA_BF16, wl.MLA_FP8):
        layers = wl.DeviceLayers(shape, base_seed=seed)
        ids, targets = wl.draw_blocks(shape.num_blocks, 128, seed)
        P = wl.payload_bytes(layers.regs, 128)
        pool = PinnedBuffer(P)
        saved = wl.save_plan(layers.regs, ids, pool.ptr)
        loads = wl.load_plan(saved, targets)
        xfer.save_layers(saved, _lib.MODE_KERNEL)
        xfer.load_layers(loads, _lib.MODE_KERNEL)
        xfer.synchronize()
        t_s = timed(lambda: xfer.save_layers(saved, _lib.MODE_KERNEL), 3)
        t_l = timed(lambda: (xfer.load_layers(loads, _lib.MODE_KERNEL), xfer.synchronize()), 3)
        bad = wl.verify_saved(layers, saved) + wl.verify_restored(layers, ids, targets)
        out[shape.name] = {"payload_bytes": P, "save_gbps": round(P / t_s / 1e9, 2),
                           "restore_gbps": round(P / t_l / 1e9, 2),
                           "restore_ms": round(t_l * 1e3, 3), "bit_exact": bad == 0}
        log(f"[bench] {shape.name}: {out[shape.name]}")
        pool.close()
        layers.close()
    return out


def leg_gpt2(xfer, seed):
    """Config 1: GPT-2 shape, 12 fp16 layers [2,512,16,12,64], 64 random
    blocks saved then restored into 64 other blocks (36 MiB each way), in the
    kernel mode and in the reference's call pattern; bit-exact."""
    from pegaflow_amd import _lib
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import PinnedBuffer

    shape = wl.GPT2
    layers = wl.DeviceLayers(shape, base_seed=seed)
    ids, targets = wl.draw_blocks(shape.num_blocks, 64, seed)
    P = wl.payload_bytes(layers.regs, 64)
    pool = PinnedBuffer(P)
    saved = wl.save_plan(layers.regs, ids, pool.ptr)
    loads = wl.load_plan(saved, targets)
    out = {"workload": shape.name + ", 64 random blocks", "payload_bytes": P}
    bad = 0
    for name, mode in (("kernel", _lib.MODE_KERNEL), ("dma_reference", _lib.MODE_DMA_REFERENCE)):
        xfer.save_layers(saved, mode)
        xfer.load_layers(loads, mode)
        xfer.synchronize()
        t_s = timed(lambda: xfer.save_layers(saved, mode), 5)
        t_l = timed(lambda: (xfer.load_layers(loads, mode), xfer.synchronize()), 5)
        bad += wl.verify_saved(layers, saved) + wl.verify_restored(layers, ids, targets)
        out[name] = {"save_gbps": round(P / t_s / 1e9, 2), "restore_gbps": round(P / t_l / 1e9, 2),
                     "save_ms": round(t_s * 1e3, 3), "restore_ms": round(t_l * 1e3, 3)}
    out["bit_exact"] = bad == 0
    log(f"[bench] gpt2: {out}")
    pool.close()
    layers.close()
    return out


def leg_tp_rank(xfer, seed):
    """The Llama prefix as one tensor-parallel rank sees it at TP=8: 32 layers
    [2,20000,16,1,128] (one kv head, 4 KiB segments), 640 random blocks, save
    then restore, in the kernel mode, the staged mode and AUTO (the engine's
    default), in the reference's call pattern (one synchronous copy per
    segment for the save, one async copy per merged run for the restore) and
    merged-run DMA."""
    from pegaflow_amd import _lib
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import PinnedBuffer

    shape, n = wl.LLAMA3_8B_TP8_RANK, 640
    layers = wl.DeviceLayers(shape, base_seed=seed)
    ids, targets = wl.draw_blocks(shape.num_blocks, n, seed)
    P = wl.payload_bytes(layers.regs, n)
    pool = PinnedBuffer(P)
    saved = wl.save_plan(layers.regs, ids, pool.ptr)
    loads = wl.load_plan(saved, targets)
    out = {"workload": "llama-3.1-8b 10k-token prefix on one TP=8 rank: 32 x bf16 "
                       "[2,20000,16,1,128], 640 random blocks, save then restore",
           "payload_bytes": P, "segment_bytes": shape.bytes_per_block}
    bad = 0
    for mode, reps in (("kernel", 5), ("staged", 5), ("auto", 5), ("dma_batched", 1),
                       ("dma_reference", 1)):
        m = _lib.MODE_NAMES[mode]
        t_s = timed(lambda: xfer.save_layers(saved, m), reps)
        t_l = timed(lambda: (xfer.load_layers(loads, m), xfer.synchronize()), reps)
        bad += wl.verify_saved(layers, saved) + wl.verify_restored(layers, ids, targets)
        layers.refill()
        out[mode] = {"save_gbps": round(P / t_s / 1e9, 2), "restore_gbps": round(P / t_l / 1e9, 2),
                     "save_ms": round(t_s * 1e3, 3), "restore_ms": round(t_l * 1e3, 3)}
    out["bit_exact"] = bad == 0
    pool.close()
    layers.close()
    return out


def pinned_copy_microbench(iters=2000):
    """The reference's criterion benchmark of the transfer primitive
    (pegaflow-core/benches/pinned_copy.rs): one block of 2 x 24 KiB copied
    from pinned host memory to the device, contiguous and strided (K/V 27
    blocks apart), as one copy, a copy per segment or a 2D copy, beside the
    same block through the transfer context.  Latency per block (us)."""
    import subprocess

    from pegaflow_amd.build import BENCH_PINNED_COPY

    if not os.path.exists(BENCH_PINNED_COPY):
        raise RuntimeError(f"{BENCH_PINNED_COPY} is not built; run python -m pegaflow_amd.build")
    log("[bench] pinned_copy microbenchmark (single block, 2 x 24 KiB)")
    r = subprocess.run([BENCH_PINNED_COPY, str(iters)], capture_output=True, text=True,
                       timeout=120)
    if r.returncode != 0:
        raise RuntimeError(f"bench_pinned_copy failed ({r.returncode}): {r.stderr.strip()}")
    out = json.loads(r.stdout.strip().splitlines()[-1])
    log(f"[bench] {out}")
    return out


def copy_engine_rates():
    """Host-link GB/s of each of the device's copy engines per direction (one
    1 GiB copy each, best of 3), and the engines the staged mode uses."""
    import subprocess

    from pegaflow_amd.build import BENCH_COPY_ENGINES

    if not os.path.exists(BENCH_COPY_ENGINES):
        raise RuntimeError(f"{BENCH_COPY_ENGINES} is not built; run python -m pegaflow_amd.build")
    log("[bench] copy engines: 1 GiB per engine and direction")
    r = subprocess.run([BENCH_COPY_ENGINES], capture_output=True, text=True, timeout=180)
    if r.returncode != 0:
        raise RuntimeError(f"bench_copy_engines failed ({r.returncode}): {r.stderr.strip()}")
    out = json.loads(r.stdout.strip().splitlines()[-1])
    log(f"[bench] {out}")
    return out


def _start_server(pool_bytes, *extra):
    """pegaflow_amd.rpc.server as a child process on an ephemeral port."""
    import select
    import subprocess

    cmd = [sys.executable, "-u", "-m", "pegaflow_amd.rpc.server", "--addr", "127.0.0.1:0",
           "--pool-size", f"{pool_bytes >> 20}mb", "--log-level", "warning", *extra]
    p = subprocess.Popen(cmd, cwd=os.path.dirname(os.path.abspath(__file__)),
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    t0, seen = time.monotonic(), []
    while time.monotonic() - t0 < 120:
        r, _, _ = select.select([p.stdout], [], [], 1.0)
        if r:
            line = p.stdout.readline()
            if not line:
                break
            seen.append(line)
            if line.startswith("READY "):
                return p, line.split()[1]
        if p.poll() is not None:
            break
    p.kill()
    p.wait(10)
    raise RuntimeError("engine server did not start:\n" + "".join(seen))


def leg_two_process(layers, ids, targets, P, reps=4, server_args=()):
    """The deployment path of the reference: the inference process keeps its
    layer tensors and talks to an engine server in another process, which
    maps the tensors through HIP IPC (registry.rs:144-175).  The inference
    side saves the prefix by hash (service.rs save), then restores it by hash
    into other blocks with a LoadState and polls it, as the connector's
    start_load_kv / get_finished do (worker.py:148-286).  The restore time
    runs from the Load request to the LoadState reading ready; the first
    layer from the request to layer 0 reading done in a layered LoadState.
    Measured over gRPC (the library's native HTTP/2 server)."""
    import hashlib

    from pegaflow_amd import ipc
    from pegaflow_amd import workload as wl
    from pegaflow_amd.load_state import PyLoadState
    from pegaflow_amd.rpc.client import EngineRpcClient

    shape = layers.shape
    names = [f"model.layers.{l}.self_attn" for l in range(len(layers.bufs))]
    handles = [ipc.export_tensor(b.ptr, shape.layer_bytes, 0) for b in layers.bufs]
    ids_l, targets_l = [int(i) for i in ids], [int(t) for t in targets]
    layers.refill()
    p, addr = _start_server((reps + 2) * P + (256 << 20), *server_args)
    out = {"what": "llama prefix saved and restored by hash through the engine server in a "
                   "second process that maps the 32 layer tensors through HIP IPC; restore "
                   "timed from the Load request to the LoadState reading ready, median of the "
                   "warm calls; over gRPC (the library's native HTTP/2 server); engine "
                   "default modes"}
    med = lambda v: statistics.median(v[1:])  # noqa: E731

    def measure(client, tag):
        save_ms, hashes = [], None
        for r in range(reps + 1):
            hashes = [hashlib.sha256(tag + b"%d-" % r + i.to_bytes(8, "little")).digest()
                      for i in ids_l]
            t0 = time.perf_counter()
            ok, msg = client.save("bench", 0, 0, [(n, ids_l, hashes) for n in names])
            save_ms.append((time.perf_counter() - t0) * 1e3)
            assert ok, msg
        load_ms, first_ms, rpc_ms = [], [], []
        for layered in (False, True):
            for r in range(reps + 1):
                st = PyLoadState(num_layers=len(names)) if layered else PyLoadState()
                t0 = time.perf_counter()
                ok, msg = client.load("bench", 0, 0, st.shm_name(), names, targets_l, hashes)
                assert ok, msg
                rpc_ms.append((time.perf_counter() - t0) * 1e3)
                t_first = None
                while not st.is_ready():
                    if layered and t_first is None and st.layers_done() >= 1:
                        t_first = time.perf_counter()
                    if time.perf_counter() - t0 > 60:
                        raise RuntimeError("two-process restore did not complete in 60 s")
                t1 = time.perf_counter()
                assert st.get_state() == 1
                (first_ms if layered else load_ms).append(
                    ((t_first or t1) - t0) * 1e3 if layered else (t1 - t0) * 1e3)
        bad = wl.verify_restored(layers, ids, targets)
        layers.refill()
        return {"save_ms": round(med(save_ms), 2), "save_gbps": round(P / med(save_ms) / 1e6, 2),
                "restore_ms": round(med(load_ms), 2),
                "restore_gbps": round(P / med(load_ms) / 1e6, 2),
                "first_layer_ms": round(med(first_ms), 3),
                "load_request_return_ms": round(statistics.median(rpc_ms), 3),
                "bit_exact": bad == 0}

    try:
        with EngineRpcClient(f"http://{addr}", connect_timeout_s=30) as client:
            t0 = time.perf_counter()
            for name, handle in zip(names, handles):
                ok, msg = client.register_context("bench", "llama3-8b", 0, 1, 0, len(names), name,
                                                  handle, shape.num_blocks,
                                                  shape.bytes_per_block, shape.kv_stride_bytes,
                                                  shape.segments)
                assert ok, msg
            out["register_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
            out.update(measure(client, b"rpc"))
            ok, msg = client.unregister_context("bench")
            assert ok, msg
            client.shutdown()
        p.wait(60)
    finally:
        if p.poll() is None:
            p.kill()
            p.wait(10)
    return out


def fs_type(path):
    """Filesystem type of the mount that holds path (from /proc/mounts)."""
    path, best, kind = os.path.realpath(path), "", "unknown"
    try:
        with open("/proc/mounts") as f:
            for line in f:
                parts = line.split()
                mnt = parts[1]
                if (path == mnt or path.startswith(mnt.rstrip("/") + "/")) and len(mnt) > len(best):
                    best, kind = mnt, parts[2]
    except OSError:
        pass
    return kind


def leg_engine(layers, ids, targets, P, reps=4):
    """The same prefix saved and restored through PegaEngine (by hash, with
    block-store bookkeeping and a LoadState) instead of the bare transfer
    context: what a vLLM connector sees."""
    import hashlib

    from pegaflow_amd import workload as wl
    from pegaflow_amd.engine import PegaEngine
    from pegaflow_amd.load_state import PyLoadState

    shape = layers.shape
    names = [f"layer.{l}" for l in range(len(layers.bufs))]
    ids_l, targets_l = [int(i) for i in ids], [int(t) for t in targets]
    e = PegaEngine(pool_size=(reps + 1) * P + (256 << 20))
    for name, buf in zip(names, layers.bufs):
        e.register_context_layer("bench", "llama3-8b", 0, name, buf.ptr, shape.layer_bytes,
                                 shape.num_blocks, shape.bytes_per_block, shape.kv_stride_bytes,
                                 shape.segments, 0, 1, len(names))
    layers.refill()
    from pegaflow_amd import _lib

    save_s, ksave_s = [], []
    hashes = None
    # The engine's default modes (saves and loads staged on the copy
    # engines), then saves by the kernel for comparison.
    for r in range(2 * (reps + 1)):  # every save uses new hashes: nothing is deduplicated
        if r == reps + 1:
            e.set_transfer_modes(_lib.MODE_KERNEL, _lib.MODE_AUTO)
        hashes = [hashlib.sha256(b"engine%d-" % r + int(i).to_bytes(8, "little")).digest()
                  for i in ids_l]
        t0 = time.perf_counter()
        e.batch_save_kv_blocks("bench", 0, 0, [(n, ids_l, hashes) for n in names])
        (save_s if r <= reps else ksave_s).append(time.perf_counter() - t0)
    bad = 0

    def restore(layered):
        """One load of the prefix by hash: (seconds to ready, to layer 0 done)."""
        st = PyLoadState(num_layers=len(names)) if layered else PyLoadState()
        t0 = time.perf_counter()
        e.batch_load_kv_blocks("bench", 0, 0, st.shm_name(), names, targets_l, hashes)
        t_first = None
        while not st.is_ready():
            if layered and t_first is None and st.layers_done() >= 1:
                t_first = time.perf_counter()
            if time.perf_counter() - t0 > 60:
                raise RuntimeError("engine restore did not complete within 60 s")
        t1 = time.perf_counter()
        if st.get_state() != 1:
            raise RuntimeError("engine restore failed")
        return t1 - t0, (t_first or t1) - t0

    loads = {}
    for mode in ("auto", "kernel"):
        e.set_transfer_modes(_lib.MODE_AUTO, _lib.MODE_NAMES[mode])
        for layered in (False, True):
            runs = [restore(layered) for _ in range(reps + 1)]
            loads[(mode, layered)] = runs
            bad += wl.verify_restored(layers, ids, targets)
            layers.refill()
    e.set_transfer_modes()
    # Duplex: a save of a new batch and a restore of the last one at once,
    # from two threads (the reference's save and load workers).
    import threading

    duplex_s = []
    for r in range(reps + 1):
        new = [hashlib.sha256(b"duplex%d-" % r + int(i).to_bytes(8, "little")).digest()
               for i in ids_l]
        go = threading.Barrier(3)
        ends, errs = {}, []

        def saver():
            try:
                go.wait()
                e.batch_save_kv_blocks("bench", 0, 0, [(n, ids_l, new) for n in names])
                ends["save"] = time.perf_counter()
            except BaseException as err:  # reported below
                errs.append(err)

        def loader():
            try:
                go.wait()
                restore(False)
                ends["load"] = time.perf_counter()
            except BaseException as err:  # reported below
                errs.append(err)

        ts = [threading.Thread(target=saver), threading.Thread(target=loader)]
        for t in ts:
            t.start()
        go.wait()
        t0 = time.perf_counter()
        for t in ts:
            t.join(120)
        if errs:
            raise errs[0]
        duplex_s.append(max(ends.values()) - t0)
        bad += wl.verify_restored(layers, ids, targets)
        layers.refill()
        hashes = new  # the next round restores what this one saved
    restore(False)  # the last duplex save, restored and checked
    bad += wl.verify_restored(layers, ids, targets)
    layers.refill()
    # Small restores (the first 1 and 16 blocks of the prefix, all 32
    # layers): latency from the call to the LoadState reading ready.
    # The same through the reference's copy pattern (one async copy per
    # merged run) for comparison.
    small = {}
    for mode, n in (("kernel", 1), ("kernel", 16), ("dma_reference", 1), ("dma_reference", 16)):
        e.set_transfer_modes(_lib.MODE_KERNEL, _lib.MODE_NAMES[mode])
        lat = []
        for r in range(21):
            st = PyLoadState()
            t0 = time.perf_counter()
            e.batch_load_kv_blocks("bench", 0, 0, st.shm_name(), names, targets_l[:n], hashes[:n])
            while not st.is_ready():
                if time.perf_counter() - t0 > 10:
                    raise RuntimeError("small engine restore did not complete within 10 s")
            lat.append(time.perf_counter() - t0)
            bad += st.get_state() != 1
        small[f"{mode}_{n}_blocks_us"] = round(statistics.median(lat[1:]) * 1e6, 1)
    e.set_transfer_modes()
    bad += wl.verify_restored(layers, ids[:16], targets[:16])
    layers.refill()
    stats = e.stats()
    e.close()
    med = lambda v: statistics.median(v[1:])  # noqa: E731
    gbps = lambda runs: round(P / med([t for t, _ in runs]) / 1e9, 3)  # noqa: E731
    return {
        "small_restore_latency": small,
        "what": "the llama prefix through PegaEngine: save by hash (new hashes each time), load "
                "by hash with a plain LoadState (as the reference's connector) and with a "
                "layered one (per-layer completion; first layer from the call to layer 0 "
                "reading done), median of the warm calls; the engine's default modes (auto: "
                "saves and loads staged on the copy engines), kernel saves and loads for "
                "comparison, and a save and a restore at once from two threads (duplex)",
        "save_mode": "auto (staged)",
        "load_mode": "auto (staged)",
        "save_gbps": round(P / statistics.median(save_s[1:]) / 1e9, 3),
        "kernel_save_gbps": round(P / statistics.median(ksave_s[1:]) / 1e9, 3),
        "restore_gbps": gbps(loads[("auto", False)]),
        "restore_layered_gbps": gbps(loads[("auto", True)]),
        "first_layer_ms": round(med([f for _, f in loads[("auto", True)]]) * 1e3, 3),
        "kernel_restore_gbps": gbps(loads[("kernel", False)]),
        "kernel_first_layer_ms": round(med([f for _, f in loads[("kernel", True)]]) * 1e3, 3),
        "duplex_gbps": round(2 * P / med(duplex_s) / 1e9, 3),
        "first_save_gbps": round(P / save_s[0] / 1e9, 3),
        "save_ms": [round(t * 1e3, 2) for t in save_s],
        "kernel_save_ms": [round(t * 1e3, 2) for t in ksave_s],
        "restore_ms": [round(t * 1e3, 2) for t, _ in loads[("auto", False)]],
        "kernel_restore_ms": [round(t * 1e3, 2) for t, _ in loads[("kernel", False)]],
        "duplex_ms": [round(t * 1e3, 2) for t in duplex_s],
        "sealed_blocks": stats["sealed_blocks"],
        "bit_exact": bad == 0,
    }


def leg_disk(layers, ids, targets, P):
    """Disk tier (seal_offload.rs) on the Llama prefix: the engine saves the
    prefix into its pinned pool and writes it to packed files (fsync'd, then
    dropped from the page cache); a fresh engine on the same directory reads
    it back into its pool on a prefix query and loads it into HBM."""
    import hashlib
    import tempfile

    from pegaflow_amd import workload as wl
    from pegaflow_amd.engine import PegaEngine
    from pegaflow_amd.load_state import PyLoadState

    shape = layers.shape
    base = os.environ.get("PEGAFLOW_DISK_DIR") or tempfile.gettempdir()
    st_fs = os.statvfs(base)
    free = st_fs.f_bavail * st_fs.f_frsize
    if free < 2 * P:
        return {"skipped": f"{free / 1e9:.1f} GB free under {base}, need {2 * P / 1e9:.1f}"}
    root = tempfile.mkdtemp(prefix="pega_disk_", dir=base)
    names = [f"layer.{l}" for l in range(len(layers.bufs))]
    hashes = [hashlib.sha256(b"prefix" + int(i).to_bytes(8, "little")).digest() for i in ids]
    ids_l, targets_l = [int(i) for i in ids], [int(t) for t in targets]
    io_threads = 8

    def engine():
        e = PegaEngine(pool_size=P + (256 << 20))
        e.enable_disk(root, quota_bytes=4 * P, io_threads=io_threads)
        for name, buf in zip(names, layers.bufs):
            e.register_context_layer("bench", "llama3-8b", 0, name, buf.ptr, shape.layer_bytes,
                                     shape.num_blocks, shape.bytes_per_block,
                                     shape.kv_stride_bytes, shape.segments, 0, 1, len(names))
        return e

    try:
        layers.refill()
        e1 = engine()
        t0 = time.perf_counter()
        e1.batch_save_kv_blocks("bench", 0, 0, [(n, ids_l, hashes) for n in names])
        t1 = time.perf_counter()
        e1.flush_disk()
        t2 = time.perf_counter()
        s1 = e1.disk_stats()
        e1.close()
        e2 = engine()
        t3 = time.perf_counter()
        q1 = e2.count_prefix_hit_blocks_with_prefetch("bench", hashes)
        e2.wait_prefetch()
        t4 = time.perf_counter()
        q2 = e2.count_prefix_hit_blocks_with_prefetch("bench", hashes)
        st = PyLoadState(num_layers=len(names))
        t5 = time.perf_counter()
        e2.batch_load_kv_blocks("bench", 0, 0, st.shm_name(), names, targets_l, hashes)
        while not st.is_ready():
            if time.perf_counter() - t5 > 60:
                raise RuntimeError("disk-tier restore did not complete within 60 s")
            time.sleep(0.0002)
        t6 = time.perf_counter()
        state = st.get_state()
        s2 = e2.disk_stats()
        e2.close()
        bad = wl.verify_restored(layers, ids, targets)
    finally:
        shutil.rmtree(root, ignore_errors=True)
    return {
        "what": "llama prefix saved through the engine, written to packed files, read back "
                "cold by a fresh engine on a prefix query, restored into HBM",
        "filesystem": fs_type(base),
        "engine_save_gbps": round(P / (t1 - t0) / 1e9, 3),
        "write_gbps": round(P / (t2 - t1) / 1e9, 3),
        "files": s1["files"], "file_bytes": s1["bytes"],
        "cold_read_gbps": round(P / (t4 - t3) / 1e9, 3),
        "io_threads": io_threads,
        "first_query": q1["prefetch_state"],
        "restore_gbps": round(P / (t6 - t5) / 1e9, 3),
        "disk_to_hbm_ms": round((t6 - t3) * 1e3, 3),
        "bit_exact": bad == 0 and state == 1 and q2["hit_blocks"] == len(ids_l)
                     and s2["prefetched_blocks"] == len(ids_l),
    }


def profile_kernels(kind, seed):
    """For rocprofv3 --pmc passes.  Every mode first runs the copy kernel 3
    times as a plain contiguous 1 GiB device copy (known bytes: 1 GiB read,
    1 GiB written: the counters' calibration), then 3 launches of:
      gather:   the Llama prefix paged -> packed HBM buffer (2P algorithmic
                bytes per launch);
      scatter:  the packed HBM buffer -> 640 other blocks of the paged
                tensors (2P);
      scatter_sets: two sets of the 32 layer tensors (42 GB each), A and B:
                gathers from A, A, B, B, then scatters into A, B, A, B in
                round-robin order (512 threads, 1 load per lane) and
                A, B, A, B in XCD-major order (2 loads per lane), then one
                more into A, which is checked;
      zerocopy: the prefix saved to pinned host memory, then restored from
                it (P over the host link per call; each call is two
                launches, its first eighth of layers, then the rest).
    Kernels are told apart by grid size (printed)."""
    from pegaflow_amd import _lib, runtime
    from pegaflow_amd import workload as wl
    from pegaflow_amd.runtime import DeviceBuffer, PinnedBuffer
    from pegaflow_amd.transfer import KVCacheRegistration, TransferContext

    runtime.init(0)
    xfer = TransferContext(0)
    src, dst = DeviceBuffer(GiB), DeviceBuffer(GiB)
    src.fill_random(seed + 99)
    chunk = 32768
    reg = KVCacheRegistration.create(src.ptr, GiB, GiB // chunk, chunk, 0, 1)
    plain = wl.save_plan([reg], np.arange(GiB // chunk), dst.ptr)
    for _ in range(3):
        xfer.save_layers(plain, _lib.MODE_KERNEL)
    src.close()
    dst.close()
    layers = wl.DeviceLayers(wl.LLAMA3_8B, base_seed=seed)
    ids, targets = wl.draw_blocks(wl.LLAMA3_8B.num_blocks, 640, seed)
    P = wl.payload_bytes(layers.regs, 640)
    info = {"plain_copy_bytes_read": GiB, "plain_copy_bytes_written": GiB,
            "plain_workgroups": (GiB // chunk) * 4, "kind": kind}
    if kind in ("gather", "scatter"):
        gbuf = DeviceBuffer(P)
        gather = wl.save_plan(layers.regs, ids, gbuf.ptr)
        xfer.save_layers(gather, _lib.MODE_KERNEL)
        plan = gather if kind == "gather" else wl.load_plan(gather, targets)
        for _ in range(3):
            if kind == "gather":
                xfer.save_layers(plan, _lib.MODE_KERNEL)
            else:
                xfer.load_layers(plan, _lib.MODE_KERNEL)
                xfer.synchronize()
        ok = (wl.verify_saved(layers, gather) == 0 if kind == "gather"
              else wl.verify_restored(layers, ids, targets) == 0)
        info.update({f"{kind}_algorithmic_bytes": 2 * P,
                     f"{kind}_workgroups": 40960 * (4 if kind == "gather" else 2),
                     "bit_exact": ok})
        gbuf.close()
    elif kind == "scatter_sets":
        other = wl.DeviceLayers(wl.LLAMA3_8B, base_seed=seed + 1)
        gbuf = DeviceBuffer(P)
        gather = wl.save_plan(layers.regs, ids, gbuf.ptr)
        xfer.save_layers(gather, _lib.MODE_KERNEL)
        gather_b = wl.save_plan(other.regs, ids, gbuf.ptr)
        for plan in (gather, gather, gather_b, gather_b):
            xfer.save_layers(plan, _lib.MODE_KERNEL)
        xfer.save_layers(gather, _lib.MODE_KERNEL)  # the packed buffer holds set A's blocks
        # Set B receives set A's packed bytes: its targets are not checked.
        into = [wl.load_plan(gather, targets), wl.load_plan(gather_b, targets)]
        nt = _lib.KERNEL_NONTEMPORAL
        for shape in ((512, 1 | nt), (512, 2 | nt | _lib.KERNEL_XCD_MAJOR)):
            xfer.set_kernel_shape_dir(_lib.ROUTE_LOAD_DEVICE, *shape)
            for r in range(4):
                xfer.load_layers(into[r % 2], _lib.MODE_KERNEL)
                xfer.synchronize()
        xfer.load_layers(into[0], _lib.MODE_KERNEL)
        xfer.synchronize()
        info.update({"scatter_algorithmic_bytes": 2 * P,
                     "order": "gather A, A, B, B, A; scatter round-robin A, B, A, B; "
                              "XCD-major A, B, A, B; A",
                     "bit_exact": wl.verify_restored(layers, ids, targets) == 0})
        gbuf.close()
        other.close()
    else:
        pool = PinnedBuffer(P)
        saved = wl.save_plan(layers.regs, ids, pool.ptr)
        loads = wl.load_plan(saved, targets)
        for _ in range(3):
            xfer.save_layers(saved, _lib.MODE_KERNEL)
        for _ in range(3):
            xfer.load_layers(loads, _lib.MODE_KERNEL)
            xfer.synchronize()
        info.update({"zerocopy_link_bytes_per_call": P,
                     "bit_exact": wl.verify_saved(layers, saved) == 0 and
                     wl.verify_restored(layers, ids, targets) == 0})
        pool.close()
    print(json.dumps(info), flush=True)
    layers.close()
    xfer.close()


def read_traffic(name, key="traffic_bytes_per_launch"):
    """Memory traffic in bytes from a committed rocprofv3 --pmc summary under
    profiles/ (its "<key> = N" line), with the file's name, or (None, None)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith(key + " ") or line.startswith(key + "="):
                    return int(line.split("=")[1].strip()), "profiles/" + name
    except OSError:
        pass
    return None, None


def _cpulist(text):
    """CPU ids of a sysfs cpulist ("0-7,16-23")."""
    out = set()
    for part in text.strip().split(","):
        if part:
            a, _, b = part.partition("-")
            out.update(range(int(a), int(b or a) + 1))
    return out


def _read(path, default=""):
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return default


def host_cores_near_gpu(device=0):
    """The GPU's NUMA node (from its PCI address) and one CPU per physical
    core of that node that this process may run on (its affinity mask), as
    the CPU baseline's threads.  Falls back to the whole affinity mask when
    the node is unknown or shares no CPU with it."""
    from pegaflow_amd import runtime

    try:
        bdf = runtime.pci_bus_id(device)
    except Exception:  # noqa: BLE001 - no device here: no node to be near
        bdf = "unknown"
    node = int(_read(f"/sys/bus/pci/devices/{bdf}/numa_node", "-1") or -1)
    allowed = os.sched_getaffinity(0)
    node_cpus = _cpulist(_read(f"/sys/devices/system/node/node{node}/cpulist")) if node >= 0 \
        else set()
    cpus = sorted(node_cpus & allowed) or sorted(allowed)
    cores = {}
    for c in cpus:
        topo = f"/sys/devices/system/cpu/cpu{c}/topology"
        cores.setdefault((_read(f"{topo}/physical_package_id"), _read(f"{topo}/core_id", str(c))),
                         c)
    return {"pci_bus_id": bdf, "numa_node": node, "node_cpus": len(node_cpus),
            "allowed_cpus": len(allowed), "cores": sorted(cores.values())}


def cpu_model() -> str:
    """The CPU's model name as lscpu reports it (its BIOS name too when the
    two differ), else /proc/cpuinfo's."""
    import subprocess

    names = []
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in text.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "BIOS Model name") and val.strip() not in names:
                names.append(val.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    if not names:
        for line in _read("/proc/cpuinfo").splitlines():
            if line.startswith("model name"):
                names.append(line.split(":", 1)[1].strip())
                break
    return " / ".join(names) or "unknown"


def cpu_baseline(shape, ids, targets, n_layers, seed, device=0):
    """The reference's CPU-side copy pattern, timed with host memcpy: save =
    one copy per segment (gpu_worker.rs:344-360), restore = one copy per merged
    run (transfer.rs:116-198), over host-resident copies of n_layers layers,
    on one thread per physical core of the GPU's NUMA node and on one thread.
    The threaded result is compared byte for byte with the single-thread
    result and checked in closed form (pool regions = source segments in
    save order, target blocks = source blocks, source words = the fill)."""
    import oracle
    from pegaflow_amd.workload import layer_seed

    near = host_cores_near_gpu(device)
    threads = max(1, len(near["cores"]))
    n, nb = len(ids), shape.num_blocks
    bpb, kv = shape.bytes_per_block, shape.kv_stride_bytes
    tensors = []
    for l in range(n_layers):
        t = np.empty(shape.layer_bytes, np.uint8)
        oracle.fill_random(t, layer_seed(seed, l))
        tensors.append(t)
    pool = np.zeros(n_layers * n * 2 * bpb, np.uint8)
    ss, sd, sz, ls, ld, lz = [], [], [], [], [], []
    for l, t in enumerate(tensors):
        reg = oracle.layout(t.ctypes.data, shape.layer_bytes, nb, bpb, kv, shape.segments)
        base = pool.ctypes.data + l * n * 2 * bpb
        k, v, _ = oracle.save_host_layout(reg, n, base, base + n * bpb)
        a, b, c = oracle.save_copies(reg, t.ctypes.data, ids, k, v)
        ss.append(a), sd.append(b), sz.append(c)
        a, b, c = oracle.load_copies(reg, t.ctypes.data, targets, k, v)
        ls.append(a), ld.append(b), lz.append(c)
    save = [np.concatenate(x) for x in (ss, sd, sz)]
    load = [np.concatenate(x) for x in (ls, ld, lz)]
    payload = n_layers * n * 2 * bpb

    # Passes are repeated for at least `seconds` (and 5 passes); the median
    # pass is reported.
    def run(t, seconds):
        ts, tl = [], []
        start = time.perf_counter()
        while len(ts) < 5 or (time.perf_counter() - start < seconds and len(ts) < 5000):
            t0 = time.perf_counter()
            oracle.run_copies(*save, nthreads=t)
            t1 = time.perf_counter()
            oracle.run_copies(*load, nthreads=t)
            t2 = time.perf_counter()
            ts.append(t1 - t0)
            tl.append(t2 - t1)
        return statistics.median(ts), statistics.median(tl), len(ts), time.perf_counter() - start

    def targets_of(t):
        return t.reshape(2, nb, bpb)[:, targets]

    run(threads, 0)  # warm
    s_mt, l_mt, reps_mt, secs_mt = run(threads, 6.0)
    pool_mt = pool.copy()
    tgt_mt = [targets_of(t) for t in tensors]
    pool[:] = 0
    for t in tensors:
        t.reshape(2, nb, bpb)[:, targets] = 0
    s_1, l_1, reps_1, secs_1 = run(1, 4.0)
    bad = int(np.count_nonzero(pool != pool_mt))
    bad += sum(int(np.count_nonzero(targets_of(t) != m)) for t, m in zip(tensors, tgt_mt))
    for l, t in enumerate(tensors):
        segs = t.reshape(2, nb, bpb)
        region = pool[l * n * 2 * bpb:(l + 1) * n * 2 * bpb].reshape(2, n, bpb)
        src = segs[:, ids]
        bad += int(np.count_nonzero(region != src)) + int(np.count_nonzero(segs[:, targets] != src))
        for j in ids[:4]:
            for sg in range(2):
                off = sg * kv + int(j) * bpb
                want = oracle.random_words(bpb // 8, layer_seed(seed, l), off // 8)
                bad += int(np.count_nonzero(t[off:off + bpb].view(np.uint64) != want))
    return {
        "value": round(2 * payload / (s_mt + l_mt) / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n_layers} of {shape.layers} layers of the same workload "
                   f"({n} blocks, save then restore, {2 * payload / 1e6:.0f} MB moved per "
                   f"pass), host memory; median pass of {reps_mt} over {secs_mt:.1f} s on "
                   f"{threads} threads, of {reps_1} over {secs_1:.1f} s on one"),
        "save_gbps": round(payload / s_mt / 1e9, 3),
        "restore_gbps": round(payload / l_mt / 1e9, 3),
        "single_thread_gbps": round(2 * payload / (s_1 + l_1) / 1e9, 3),
        "save_copies": int(len(save[0])),
        "restore_copies": int(len(load[0])),
        "bit_exact": bad == 0,
        "threads": ("one per physical core of the GPU's NUMA node in this process's CPU set"
                    if near["node_cpus"] else "one per physical core in this process's CPU set"),
        "numa": {k: v for k, v in near.items() if k != "cores"},
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
    }


def scatter_spread(xfer, layers, gather_buf, ids, targets, seed, reps=6):
    """The device scatter (packed HBM -> the blocks of 32 layers) and the
    device gather (the blocks -> packed HBM) of 640 blocks, with the blocks
    drawn ever closer together: uniformly from all 20,000 (the workload),
    the same sorted, from the first 2,000, the first 640 in a random order,
    and the first 640 in order.  Every case moves the same 2P bytes in the
    same 40,960 chunks of 32 KiB with the same launch; only where the random
    side's chunks lie in memory changes.  Median kernel time of `reps`
    launches each (HIP events on the context's stream)."""
    from pegaflow_amd import _lib
    from pegaflow_amd import workload as wl

    n = len(ids)
    rng = np.random.Generator(np.random.PCG64(seed + 7))
    cases = {
        "all_20000_random": np.asarray(targets),
        "all_20000_sorted": np.sort(np.asarray(targets)),
        "first_2000_random": rng.choice(2000, n, replace=False),
        "first_640_permuted": rng.permutation(n),
        "first_640_in_order": np.arange(n),
    }
    P2 = 2 * wl.payload_bytes(layers.regs, n)
    gather_ids = wl.save_plan(layers.regs, ids, gather_buf.ptr)
    xfer.set_timing(True)
    out = {}
    for name, blocks in cases.items():
        row = {}
        for kind in ("scatter", "gather"):
            plan = (wl.load_plan(gather_ids, blocks) if kind == "scatter"
                    else wl.save_plan(layers.regs, blocks, gather_buf.ptr))

            def go():
                if kind == "scatter":
                    xfer.load_layers(plan, _lib.MODE_KERNEL)
                    xfer.synchronize()
                else:
                    xfer.save_layers(plan, _lib.MODE_KERNEL)
                return xfer.last_kernel_ms()[0]

            go()
            ms = statistics.median(go() for _ in range(reps))
            row[kind] = {"ms": round(ms, 4), "gbps": round(P2 / ms / 1e6, 1),
                         "frac": round(P2 / ms / 1e6 / HBM_PEAK_GBPS, 4)}
        out[name] = row
        log(f"[bench] scatter spread {name}: {row}")
    layers.refill()
    return out


def run_leg(args):
    """One workload on its own (--leg): its JSON object on stdout."""
    from pegaflow_amd import runtime
    from pegaflow_amd.transfer import TransferContext
    from pegaflow_amd import workload as wl

    runtime.init(0)
    xfer = TransferContext(0, staging_bytes=args.staging_mib << 20)
    simple = {"gpt2": leg_gpt2, "layerwise": leg_layerwise, "mla": leg_mla, "tp8": leg_tp_rank}
    if args.leg in simple:
        out = simple[args.leg](xfer, args.seed)
    else:
        shape = wl.LLAMA3_8B
        layers = wl.DeviceLayers(shape, base_seed=args.seed)
        ids, targets = wl.draw_blocks(shape.num_blocks, 640, args.seed)
        P = wl.payload_bytes(layers.regs, 640)
        if args.leg == "fragmentation":
            out = leg_fragmentation(layers, xfer, args.seed)
        elif args.leg == "engine":
            out = leg_engine(layers, ids, targets, P)
        elif args.leg == "two_process":
            out = leg_two_process(layers, ids, targets, P)
        else:
            out = leg_disk(layers, ids, targets, P)
        layers.close()
    xfer.close()
    print(json.dumps({args.leg: out}), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the KV transfer path has no cross-GPU step "
              "(each rank moves its own layers over its own host link); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if args.profile:
        profile_kernels(args.profile, args.seed)
        return
    if args.interference_study:
        interference_study(args.study_engines, args.study_victims)
        return
    if args.first_layer_study:
        first_layer_study(cu_masks=[int(k) for k in args.cu_masks.split(",") if k])
        return
    if args.leg:
        run_leg(args)
        return

    # The single-block latency benchmark runs as its own process, before this
    # one touches the GPU.
    micro = None if args.quick else pinned_copy_microbench()
    engines = None if args.quick else copy_engine_rates()

    from pegaflow_amd import _lib, runtime
    from pegaflow_amd.runtime import DeviceBuffer, PinnedBuffer
    from pegaflow_amd.transfer import KVCacheRegistration, TransferContext
    from pegaflow_amd import workload as wl

    shape = wl.LLAMA3_8B
    n_blocks = 640
    runtime.init(0)
    log(f"[bench] allocating {shape.layers} x {shape.layer_bytes / 1e9:.2f} GB layer tensors")
    layers = wl.DeviceLayers(shape, base_seed=args.seed)
    ids, targets = wl.draw_blocks(shape.num_blocks, n_blocks, args.seed)
    P = wl.payload_bytes(layers.regs, n_blocks)
    assert P == 1_342_177_280
    pool = PinnedBuffer(P, args.pinned_flags)
    gather_buf = DeviceBuffer(P)
    xfer = TransferContext(0, staging_bytes=args.staging_mib << 20)
    modes = _lib.MODE_NAMES
    saved = wl.save_plan(layers.regs, ids, pool.ptr)
    loads = wl.load_plan(saved, targets)

    log("[bench] host-link and HBM copy peaks")
    h2d_peak, d2h_peak, d2d_gbps = link_peaks(pool, gather_buf, xfer.stream)
    log(f"[bench] h2d {h2d_peak:.1f} GB/s, d2h {d2h_peak:.1f} GB/s, d2d {d2d_gbps:.0f} GB/s")

    # Device gather: the same save batch into a packed HBM buffer.
    gather = wl.save_plan(layers.regs, ids, gather_buf.ptr)
    xfer.set_timing(True)
    sweep = {}
    default_shape = (512, 1 | _lib.KERNEL_NONTEMPORAL)
    nt_names = {0: "", _lib.KERNEL_NT_LOADS: "_ntl", _lib.KERNEL_NT_STORES: "_nts",
                _lib.KERNEL_NONTEMPORAL: "_nt"}

    def shape_sweep(label, plan, run, reps, bytes_moved, shapes):
        for threads, unroll in shapes:
            xfer.set_kernel_shape(threads, unroll)
            run(plan)
            ms = []
            for _ in range(reps):
                run(plan)
                ms.append(xfer.last_kernel_ms()[0])
            key = (f"{label}_t{threads}_u{unroll & 0xff}{nt_names[unroll & 0x300]}"
                   f"{'_xcd' if unroll & _lib.KERNEL_XCD_MAJOR else ''}")
            sweep[key] = round(bytes_moved / (min(ms) / 1e3) / 1e9, 1)
            log(f"[bench] sweep {key}: {min(ms):.4f} ms = {sweep[key]} GB/s")
        xfer.reset_kernel_shape()

    if args.sweep:
        save_k = lambda plan: xfer.save_layers(plan, _lib.MODE_KERNEL)  # noqa: E731
        load_k = lambda plan: (xfer.load_layers(plan, _lib.MODE_KERNEL),  # noqa: E731
                               xfer.synchronize())
        shape_sweep("gather", gather, save_k, 5, 2 * P,
                    [(t, u | nt) for t in (256, 512, 768, 1024) for u in (1, 2, 4)
                     for nt in (0, _lib.KERNEL_NT_LOADS, _lib.KERNEL_NT_STORES,
                                _lib.KERNEL_NONTEMPORAL)])
        xcd_shapes = [(t, u | _lib.KERNEL_NONTEMPORAL | x) for t in (256, 512, 1024)
                      for u in (1, 2) for x in (0, _lib.KERNEL_XCD_MAJOR)]
        shape_sweep("gatherx", gather, save_k, 5, 2 * P, xcd_shapes)
        scatter_plan = wl.load_plan(gather, targets)
        shape_sweep("scatter", scatter_plan, load_k, 5, 2 * P, xcd_shapes)
        # The same kernel as a plain contiguous copy of the packed buffer.
        creg = KVCacheRegistration.create(gather_buf.ptr, P, P // 32768, 32768, 0, 1)
        plain_dst = DeviceBuffer(P)
        plain = wl.save_plan([creg], np.arange(P // 32768), plain_dst.ptr)
        shape_sweep("plaincopy", plain, save_k, 5, 2 * P, xcd_shapes)
        plain_dst.close()
        layers.refill()
        for grid in (1024, 2048, 4096):
            xfer.set_max_grid(grid)
            shape_sweep(f"gather_grid{grid}", gather, save_k, 5, 2 * P, [default_shape])
        xfer.set_max_grid(0)
        link_shapes = [(t, u | nt) for t in (256, 512, 1024) for u in (2, 4, 8)
                       for nt in (0, _lib.KERNEL_NONTEMPORAL)]
        shape_sweep("zerocopy_restore", loads, load_k, 2, P, link_shapes)
        shape_sweep("zerocopy_save", saved, save_k, 2, P, link_shapes)
    if args.threads or args.unroll:
        xfer.set_kernel_shape(args.threads, args.unroll)
    xfer.save_layers(gather, _lib.MODE_KERNEL)
    g_ms, g_launch = [], 0
    for _ in range(10):
        xfer.save_layers(gather, _lib.MODE_KERNEL)
        ms, g_launch = xfer.last_kernel_ms()
        g_ms.append(ms)
    gather_ms = sum(g_ms) / len(g_ms)
    gather_gbps = 2 * P / (gather_ms / 1e3) / 1e9
    log(f"[bench] device gather {gather_ms:.3f} ms/launch ({g_launch} launch) = "
        f"{gather_gbps:.0f} GB/s")
    # The same kernel and launch shape as a plain contiguous copy of the
    # packed buffer (2P bytes moved, 32 KiB chunks in address order): the
    # copy ceiling the gather's random chunk order is held against.
    creg = KVCacheRegistration.create(gather_buf.ptr, P, P // 32768, 32768, 0, 1)
    plain_dst = DeviceBuffer(P)
    plain = wl.save_plan([creg], np.arange(P // 32768), plain_dst.ptr)
    xfer.save_layers(plain, _lib.MODE_KERNEL)
    p_ms = []
    for _ in range(5):
        xfer.save_layers(plain, _lib.MODE_KERNEL)
        p_ms.append(xfer.last_kernel_ms()[0])
    plain_dst.close()
    plain_gbps = 2 * P / (sum(p_ms) / len(p_ms) / 1e3) / 1e9
    log(f"[bench] plain contiguous copy, same kernel: {plain_gbps:.0f} GB/s")
    # Device scatter: the packed HBM buffer back into the target blocks.
    scatter = wl.load_plan(gather, targets)
    # The context times its two candidate scatter shapes on its first large
    # scatters and keeps the faster; the timed launches follow the choice.
    for _ in range(6):
        xfer.load_layers(scatter, _lib.MODE_KERNEL)
        xfer.synchronize()
    s_threads, s_unroll, s_decided = xfer.route_shape(_lib.ROUTE_LOAD_DEVICE)
    s_ms = []
    for _ in range(10):
        xfer.load_layers(scatter, _lib.MODE_KERNEL)
        ms, _ = xfer.last_kernel_ms()
        s_ms.append(ms)
    scatter_ms = sum(s_ms) / len(s_ms)
    scatter_gbps = 2 * P / (scatter_ms / 1e3) / 1e9
    if args.sweep_scatter:
        load_k = lambda plan: (xfer.load_layers(plan, _lib.MODE_KERNEL),  # noqa: E731
                               xfer.synchronize())
        scatter_shapes = [(t, u | nt | x) for t in (256, 512, 1024) for u in (1, 2, 4)
                          for nt in (0, _lib.KERNEL_NT_LOADS, _lib.KERNEL_NT_STORES,
                                     _lib.KERNEL_NONTEMPORAL)
                          for x in (0, _lib.KERNEL_XCD_MAJOR)]
        shape_sweep("scatter", scatter, load_k, 5, 2 * P, scatter_shapes)
        # The same chunks with each layer's blocks in destination order.
        dst_sorted = []
        for lt in scatter:
            b = lt.blocks[np.argsort(lt.blocks["block_idx"], kind="stable")]
            dst_sorted.append(type(lt)(lt.registration, b))
        shape_sweep("scatter_dstsorted", dst_sorted, load_k, 5, 2 * P, scatter_shapes)
        layers.refill()

    spread = scatter_spread(xfer, layers, gather_buf, ids, targets, args.seed) \
        if args.scatter_spread else None

    variants = {}
    if args.variants or not args.quick:
        for name, m in modes.items():
            # The reference's pattern waits for each of its 40,960 save copies:
            # bound by the completion latency of each, which varies from run to
            # run (9-48 us a copy), so it gets the best of two.
            reps = 2 if name == "dma_reference" else 3
            t_s = timed(lambda: xfer.save_layers(saved, m), reps)
            t_l = timed(lambda: (xfer.load_layers(loads, m), xfer.synchronize()), reps)
            variants[name] = {"save_gbps": round(P / t_s / 1e9, 2),
                              "restore_gbps": round(P / t_l / 1e9, 2),
                              "save_ms": round(t_s * 1e3, 3), "restore_ms": round(t_l * 1e3, 3)}
            log(f"[bench] variant {name}: {variants[name]}")

    save_mode, load_mode = modes[args.save_mode], modes[args.load_mode]
    log(f"[bench] steps: save={args.save_mode} restore={args.load_mode} "
        f"warmup={args.warmup} steps={args.steps}")
    xfer.set_timing(True)
    t_save, t_load, k_save, k_load = [], [], [], []
    for i in range(args.warmup):
        xfer.save_layers(saved, save_mode)
        xfer.load_layers(loads, load_mode)
        xfer.synchronize()
    runtime.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        a = time.perf_counter()
        xfer.save_layers(saved, save_mode)
        k_save.append(xfer.last_kernel_ms()[0])
        b = time.perf_counter()
        xfer.load_layers(loads, load_mode)
        xfer.synchronize()
        k_load.append(xfer.last_kernel_ms()[0])
        c = time.perf_counter()
        t_save.append(b - a)
        t_load.append(c - b)
    runtime.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed / args.steps * 1e3
    value = 2 * P * args.steps / elapsed / 1e9
    save_s, load_s = statistics.median(t_save), statistics.median(t_load)

    bad_host = wl.verify_saved(layers, saved)
    bad_dev = wl.verify_restored(layers, ids, targets)
    log(f"[bench] verify: host mismatches {bad_host}, device mismatches {bad_dev}")

    # Full duplex: a second prefix saved (into a second pool) while the first
    # is restored, on two contexts as the engine's save and load workers do.
    pool2 = PinnedBuffer(P, args.pinned_flags)
    xfer2 = TransferContext(0, staging_bytes=(args.staging_mib << 20) if args.duplex_study else 0)
    saved2 = wl.save_plan(layers.regs, ids, pool2.ptr)
    # The two zero-copy kernels at once from one thread (the staged pair
    # below needs the restore on its own thread: a staged load returns once
    # its copies are done).
    t_dup = duplex(xfer2, xfer, saved2, loads, _lib.MODE_KERNEL)
    bad_dup = wl.verify_saved(layers, saved2) + wl.verify_restored(layers, ids, targets)
    log(f"[bench] duplex save+restore {t_dup * 1e3:.3f} ms = {2 * P / t_dup / 1e9:.1f} GB/s, "
        f"mismatches {bad_dup}")
    # The staged pair on the copy engines (one engine each way), the restore
    # from a second thread as the engine's load thread issues it.
    xfer_s = TransferContext(0, staging_bytes=args.staging_mib << 20)
    t_dup_staged = duplex_threads(xfer_s, xfer, saved2, loads, _lib.MODE_STAGED)
    xfer_s.close()
    bad_dup += wl.verify_saved(layers, saved2) + wl.verify_restored(layers, ids, targets)
    log(f"[bench] duplex staged save+restore {t_dup_staged * 1e3:.3f} ms = "
        f"{2 * P / t_dup_staged / 1e9:.1f} GB/s, mismatches {bad_dup}")
    bad_host += bad_dup
    log("[bench] interference: a device copy kernel beside each transfer mode")
    interference = leg_interference(layers, saved, loads, P)
    if args.duplex_study:
        extra_duplex = duplex_study(xfer, xfer2, saved2, loads, pool, pool2, gather_buf, P)
    xfer2.close()
    pool2.close()

    extra = {}
    if not args.quick:
        log("[bench] config 1: gpt2 shape")
        extra["gpt2_config1"] = leg_gpt2(xfer, args.seed)
        log("[bench] config 3: layer-wise restore (qwen3-8b)")
        extra["layerwise_qwen3_8b"] = leg_layerwise(xfer, args.seed)
        log(f"[bench] {extra['layerwise_qwen3_8b']}")
        log("[bench] config 5: MLA latent bf16 / fp8")
        extra["mla_latent"] = leg_mla(xfer, args.seed)
        log("[bench] one TP=8 rank of the llama prefix (4 KiB segments)")
        extra["tp8_rank_llama3_8b"] = leg_tp_rank(xfer, args.seed)
        log(f"[bench] {extra['tp8_rank_llama3_8b']}")
        log("[bench] config 4: fragmentation sweep")
        extra["fragmentation_llama3_8b"] = leg_fragmentation(layers, xfer, args.seed)
        log("[bench] engine: save and restore by hash")
        extra["engine_llama3_8b"] = leg_engine(layers, ids, targets, P)
        log(f"[bench] {extra['engine_llama3_8b']}")
        log("[bench] two processes: gRPC engine server mapping the layers by HIP IPC")
        extra["two_process_llama3_8b"] = leg_two_process(layers, ids, targets, P)
        log(f"[bench] {extra['two_process_llama3_8b']}")
        log("[bench] disk tier: offload, cold prefetch, restore")
        extra["disk_tier_llama3_8b"] = leg_disk(layers, ids, targets, P)
        log(f"[bench] {extra['disk_tier_llama3_8b']}")

    k_save_ms, k_load_ms = statistics.median(k_save), statistics.median(k_load)
    # The step's dominant kernel: a side whose host-link bytes a kernel moves
    # (the zero-copy kernel) spends about its whole call in that kernel; a
    # staged side's kernels are its HBM gather or scatter, a few percent of
    # the call, and its link bytes are copy-engine DMA.
    zc_file = "copy_chunks_llama3_8b_zerocopy_traffic.txt"
    sides = {
        "save": {"kernel_ms": k_save_ms, "wall_s": save_s, "peak": d2h_peak,
                 "zero_copy": k_save_ms > 0.5 * save_s * 1e3,
                 "traffic": read_traffic(zc_file, "save_traffic_bytes_per_call"),
                 "kernel": "copy_chunks_queue_kernel<2,nt-loads> 512 threads x 32 persistent "
                           "workgroups (zero-copy save: 40,960 chunks of 32 KiB, paged HBM -> "
                           "pinned host, 2 launches per call)"},
        "restore": {"kernel_ms": k_load_ms, "wall_s": load_s, "peak": h2d_peak,
                    "zero_copy": k_load_ms > 0.5 * load_s * 1e3,
                    "traffic": read_traffic(zc_file, "restore_traffic_bytes_per_call"),
                    "kernel": "copy_chunks_queue_kernel<2,nt,nt> 512 threads x 64 persistent "
                              "workgroups (zero-copy restore: 40,960 chunks of 32 KiB, pinned "
                              "host -> paged HBM, 2 launches per call)"},
    }

    def side_entry(name):
        sd = sides[name]
        if sd["zero_copy"]:
            gbps = P / (sd["kernel_ms"] / 1e3) / 1e9
            return {"kernel": sd["kernel"], "achieved": round(gbps, 2),
                    "frac": round(gbps / PCIE_GEN5_X16_GBPS, 4),
                    "measured_peak": round(sd["peak"], 2),
                    "frac_of_measured_peak": round(gbps / sd["peak"], 4),
                    "ms_per_call": round(sd["kernel_ms"], 4),
                    "traffic": sd["traffic"][0], "traffic_source": sd["traffic"][1]}
        gbps = P / sd["wall_s"] / 1e9
        return {"mode": "staged: HBM gather/scatter kernels on the device, the host-link "
                        "bytes by copy-engine DMA (wall clock)",
                "link_gbps": round(gbps, 2), "frac": round(gbps / PCIE_GEN5_X16_GBPS, 4),
                "measured_peak": round(sd["peak"], 2),
                "frac_of_measured_peak": round(gbps / sd["peak"], 4),
                "hbm_kernel_ms_per_call": round(sd["kernel_ms"], 4)}

    zc_sides = [n for n in ("save", "restore") if sides[n]["zero_copy"]]
    dominant = max(zc_sides, key=lambda n: sides[n]["kernel_ms"]) if zc_sides else None
    gather_traffic, gather_traffic_src = read_traffic("copy_chunks_llama3_8b_prefix_traffic.txt")
    scatter_traffic, scatter_traffic_src = read_traffic(
        "copy_chunks_llama3_8b_scatter_traffic.txt")

    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] cpu baseline: {args.cpu_sample_layers} layers")
        cpu = cpu_baseline(shape, ids, targets, args.cpu_sample_layers, args.seed)
        log(f"[bench] cpu baseline {cpu}")

    out = {
        "metric": "KV save/load GB/s + ms per 10K-tok Llama-3-8B prefix (frac of PCIe/HBM peak)",
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded splitmix64 random bits in bf16-shaped KV tensors)",
        "config": {
            "workload": "llama-3.1-8b 10k-token prefix: 32 x bf16 [2,20000,16,8,128], "
                        "640 random blocks, save then restore into 640 other blocks",
            "payload_bytes_per_direction": P,
            "save_mode": args.save_mode,
            "restore_mode": args.load_mode,
            "parallelism": "single gpu",
        },
        "restore_gbps": round(P / load_s / 1e9, 3),
        "restore_ms_per_prefix": round(load_s * 1e3, 3),
        "restore_frac_of_measured_h2d_peak": round(P / load_s / 1e9 / h2d_peak, 4),
        "restore_frac_of_pcie_gen5": round(P / load_s / 1e9 / PCIE_GEN5_X16_GBPS, 4),
        "save_gbps": round(P / save_s / 1e9, 3),
        "save_ms_per_prefix": round(save_s * 1e3, 3),
        "save_frac_of_measured_d2h_peak": round(P / save_s / 1e9 / d2h_peak, 4),
        "save_frac_of_pcie_gen5": round(P / save_s / 1e9 / PCIE_GEN5_X16_GBPS, 4),
        "restore_kernel_ms": round(k_load_ms, 3),
        "save_kernel_ms": round(k_save_ms, 3),
        "host_link_peak_gbps": {"h2d": round(h2d_peak, 2), "d2h": round(d2h_peak, 2),
                                "pcie_gen5_x16": PCIE_GEN5_X16_GBPS},
        # The step's dominant kernel (the zero-copy side with the longer
        # kernel time): achieved = P per call / the call's kernel time (HIP
        # events on the context's stream around each launch, summed over the
        # call's two launches); the other side as a sub-entry.
        "roofline": ({"bound": "pcie", "peak": PCIE_GEN5_X16_GBPS, "unit": "GB/s",
                      "bytes_per_call": P, "side": dominant, **side_entry(dominant),
                      ("restore" if dominant == "save" else "save"):
                          side_entry("restore" if dominant == "save" else "save")}
                     if dominant else None),
        # The HBM-bound kernels of the staged mode, timed outside the steps.
        "device_gather": {
            "bound": "hbm",
            "achieved": round(gather_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gather_gbps / HBM_PEAK_GBPS, 4),
            "traffic": gather_traffic,
            "traffic_source": gather_traffic_src,
            "kernel": "copy_chunks_v16_kernel<1,nt,nt> 512 threads (device gather: 40960 "
                      "chunks of 32 KiB, 1 launch)",
            "bytes_per_launch": 2 * P,
            "ms_per_launch": round(gather_ms, 4),
            "plain_copy_gbps": round(plain_gbps, 1),
            "frac_of_plain_copy": round(gather_gbps / plain_gbps, 4),
        },
        "device_scatter": {"bound": "hbm", "achieved": round(scatter_gbps, 1),
                           "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                           "frac": round(scatter_gbps / HBM_PEAK_GBPS, 4),
                           "traffic": scatter_traffic, "traffic_source": scatter_traffic_src,
                           "kernel": f"copy_chunks_v16_kernel<{s_unroll & 0xff},nt,nt> "
                                     f"{s_threads} threads, "
                                     f"{'XCD-major' if s_unroll & _lib.KERNEL_XCD_MAJOR else 'round-robin'}"
                                     " tile order, chosen by the context from two timed "
                                     f"candidates (decided: {s_decided}) (device scatter: "
                                     "packed HBM -> 640 blocks)",
                           "bytes_per_launch": 2 * P, "ms_per_launch": round(scatter_ms, 4)},
        "d2d_memcpy_gbps": round(d2d_gbps, 1),
        "interference": interference,
        **({"copy_engines": engines} if engines else {}),
        "duplex_staged": {"gbps": round(2 * P / t_dup_staged / 1e9, 3),
                          "ms_per_save_plus_restore": round(t_dup_staged * 1e3, 3),
                          "what": "as duplex, both staged on the copy engines, the restore "
                                  "issued from a second thread"},
        "duplex": {"gbps": round(2 * P / t_dup / 1e9, 3), "ms_per_save_plus_restore":
                   round(t_dup * 1e3, 3),
                   "what": "a prefix saved while another is restored, both by the zero-copy "
                           "kernel (two transfer contexts, one thread)",
                   **({"study": extra_duplex} if args.duplex_study else {})},
        "bit_exact": bad_host == 0 and bad_dev == 0,
        "cpu_baseline": cpu,
    }
    if out["roofline"] is None:  # no zero-copy side: the staged mode's HBM kernel
        out["roofline"] = dict(out["device_scatter"], side="device scatter (staged restore)")
    out.update(extra)
    if micro is not None:
        out["pinned_copy_microbench"] = micro
    if variants:
        out["variants"] = variants
    if variants.get("auto"):
        # The pair the engine deploys: PF_MODE_AUTO both ways, which these
        # long host runs resolve to the staged mode (HBM gather/scatter plus
        # copy-engine DMA over the link); its link bytes are DMA, so its
        # roofline is the link's, from the variants' wall-clock timing.
        a = variants["auto"]
        out["deployed"] = {
            "save_mode": "auto (staged)", "restore_mode": "auto (staged)",
            "bound": "pcie", "unit": "GB/s", "peak": PCIE_GEN5_X16_GBPS,
            "save_gbps": a["save_gbps"], "restore_gbps": a["restore_gbps"],
            "save_frac": round(a["save_gbps"] / PCIE_GEN5_X16_GBPS, 4),
            "restore_frac": round(a["restore_gbps"] / PCIE_GEN5_X16_GBPS, 4),
            "save_frac_of_measured_d2h_peak": round(a["save_gbps"] / d2h_peak, 4),
            "restore_frac_of_measured_h2d_peak": round(a["restore_gbps"] / h2d_peak, 4),
        }
    if sweep:
        out["gather_sweep_gbps"] = sweep
    if spread:
        out["scatter_spread"] = spread
    print(json.dumps(out), flush=True)
    xfer.close()
    pool.close()
    gather_buf.close()
    layers.close()
    if not out["bit_exact"]:
        sys.exit(1)


if __name__ == "__main__":
    main()
