"""Fragmentation sweep on the GPU: block ids drawn as contiguous runs of
geometric length (mean 1, 4, 32, and 640 = fully sorted), each request
saving its blocks to the pinned pool and restoring them into a second draw
of the same kind, requests one after another on the same layer tensors, in
every transfer mode.

  * Small Llama-like shapes: the host pool after every save and the layer
    tensors after every restore equal the oracle's, run on a CPU copy of the
    same tensors; the DMA modes issue exactly the oracle's number of merged
    copies (transfer.rs:134-177).
  * Full Llama-3.1-8B shape (32 x [2,20000,16,8,128] bf16): every host chunk
    after every save, and every block of every layer after the batch, hold
    the splitmix64 words of the block they came from, tracked through the
    restores (closed form, checked on the device).
"""

import sys

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd import workload as wl
from pegaflow_amd.runtime import DeviceBuffer, PinnedBuffer
from pegaflow_amd.transfer import (KVCacheRegistration, LayerTransfer, TransferContext,
                                   block_array)

pytestmark = pytest.mark.gpu

# AUTO picks the kernel or the staged mode per call from the host side's
# run lengths, so it meets both choices across the run lengths below.
MODES = {"dma_reference": _lib.MODE_DMA_REFERENCE, "dma_batched": _lib.MODE_DMA_BATCHED,
         "kernel": _lib.MODE_KERNEL, "staged": _lib.MODE_STAGED, "auto": _lib.MODE_AUTO}
MEANS = (1, 4, 32, 640)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx(gpu):
    c = TransferContext(0, staging_bytes=64 << 20)
    yield c
    c.close()


@pytest.mark.parametrize("mode", list(MODES))
def test_fragmentation_small_vs_oracle(ctx, mode):
    """4 split layers of [2, 2048 blocks, 512 B segments]; per mean run
    length, 3 requests of 20-300 blocks: save, check the pool, restore into
    the request's second draw, check the tensors and the copy count."""
    m = MODES[mode]
    n_layers, nb, bpb = 4, 2048, 512
    kv = nb * bpb
    size = 2 * kv
    devs, refs, regs, oregs = [], [], [], []
    for l in range(n_layers):
        d = DeviceBuffer(size)
        d.fill_random(oracle.layer_seed(41, l))
        devs.append(d)
        refs.append(d.download())
        regs.append(KVCacheRegistration.create(d.ptr, size, nb, bpb, kv, 2))
    oregs = [oracle.layout(r.ctypes.data, size, nb, bpb, kv, 2) for r in refs]
    host = PinnedBuffer(n_layers * 300 * 2 * bpb)
    ohost = np.zeros(host.nbytes, np.uint8)
    rng = np.random.Generator(np.random.PCG64(17))
    for mean in MEANS:
        for r in range(3):
            n = int(rng.integers(20, 301))
            mm = float("inf") if mean >= wl.SORTED_MEAN_RUN else mean
            ids = wl.draw_runs(rng, nb, n, mm)
            mask = np.zeros(nb, bool)
            mask[ids] = True
            targets = wl.draw_runs(rng, nb, n, mm, exclude=mask)
            say(f"[gpu] fragmentation small mode={mode} mean={mean} req={r} n={n} "
                f"runs={wl.run_count(ids)}/{wl.run_count(targets)}")
            saved, osaved = [], []
            for l in range(n_layers):
                base, obase = host.ptr + l * n * 2 * bpb, ohost.ctypes.data + l * n * 2 * bpb
                k, v, _ = oracle.save_host_layout(oregs[l], n, base, base + n * bpb)
                ok_, ov, _ = oracle.save_host_layout(oregs[l], n, obase, obase + n * bpb)
                saved.append(LayerTransfer(regs[l], block_array(ids, k, v)))
                osaved.append((ok_, ov))
            host.array[:] = 0
            ohost[:] = 0
            ctx.save_layers(saved, m)
            if mode == "dma_reference":
                assert ctx.last_stats()[1] == n_layers * 2 * n  # one copy per segment
            for l in range(n_layers):
                oracle.process_save(oregs[l], refs[l], ids, *osaved[l])
            assert np.array_equal(host.array, ohost), "host pool differs from the oracle"
            loads = []
            for lt in saved:
                b = lt.blocks.copy()
                b["block_idx"] = targets
                loads.append(LayerTransfer(lt.registration, b))
            ctx.load_layers(loads, m)
            ctx.synchronize()
            copies = ctx.last_stats()[1]
            runs = sum(oracle.process_load(oregs[l], refs[l], targets, *osaved[l])
                       for l in range(n_layers))
            if mode.startswith("dma"):
                assert copies == runs, (copies, runs)
            for l in range(n_layers):
                assert np.array_equal(devs[l].download(), refs[l]), f"layer {l} differs"
    host.close()
    for d in devs:
        d.close()


@pytest.fixture(scope="module")
def llama(gpu):
    layers = wl.DeviceLayers(wl.LLAMA3_8B, base_seed=4)
    yield layers
    layers.close()


@pytest.mark.parametrize("mode", list(MODES))
def test_fragmentation_llama_full_size(ctx, llama, mode):
    """Config 4 at its real shape: per mean run length, 2 requests of
    U[1K,16K] tokens, each saved then restored into its second draw, in one
    mode; host chunks checked after every save, all 20,000 blocks of all 32
    layers after the batch."""
    m = MODES[mode]
    shape = llama.shape
    llama.refill()  # every block holds its own words again
    src_of = np.arange(shape.num_blocks, dtype=np.int64)
    pool = PinnedBuffer(1024 * shape.layers * 2 * shape.bytes_per_block)
    for mean in MEANS:
        for i, (ids, targets) in enumerate(wl.fragmentation_requests(
                shape.num_blocks, mean, seed=MEANS.index(mean) + 10 * list(MODES).index(mode),
                n_requests=2)):
            say(f"[gpu] fragmentation llama mode={mode} mean={mean} req={i} n={len(ids)} "
                f"runs={wl.run_count(ids)}/{wl.run_count(targets)}")
            saved = wl.save_plan(llama.regs, ids, pool.ptr)
            ctx.save_layers(saved, m)
            assert wl.verify_saved(llama, saved, src_of) == 0
            ctx.load_layers(wl.load_plan(saved, targets), m)
            ctx.synchronize()
            src_of[targets] = src_of[ids]
    pool.close()
    assert wl.verify_blocks(llama, src_of) == 0
