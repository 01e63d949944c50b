"""GPU tests of the exported transfer.rs primitives, the calls a maintainer
swaps in for transfer.rs itself: copy_gpu_to_cpu, copy_cpu_to_gpu_async,
batch_copy_segments_to_gpu (its copies and its batch count) and
copy_block_gpu_to_cpu (contiguous, split and strided layouts), each checked
byte for byte against the oracle run on a CPU copy of the same tensor."""

import sys

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.runtime import DeviceBuffer, PinnedBuffer, Stream
from pegaflow_amd.transfer import (KVCacheRegistration, batch_copy_segments_to_gpu,
                                   copy_block_gpu_to_cpu, copy_cpu_to_gpu_async,
                                   copy_gpu_to_cpu, segment_offset)

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _tensor(size, seed):
    dev = DeviceBuffer(size)
    dev.fill_random(seed)
    return dev, dev.download()


def test_copy_gpu_to_cpu_and_back(gpu):
    """Synchronous D2H at several offsets and sizes (transfer.rs:56-76), then
    asynchronous H2D on a stream (transfer.rs:80-113) from pageable and from
    pinned memory; a too-small buffer is refused and copies nothing."""
    say("[gpu] copy_gpu_to_cpu / copy_cpu_to_gpu_async")
    dev, ref = _tensor(1 << 20, 11)
    for off, size in [(0, 1 << 20), (8, 24), (4096, 32768), (1000, 3), ((1 << 20) - 16, 16)]:
        out = np.zeros(size, np.uint8)
        copy_gpu_to_cpu(dev.ptr, off, out, size)
        assert np.array_equal(out, ref[off: off + size]), (off, size)
    s = Stream()
    pinned = PinnedBuffer(1 << 16)
    for src_kind in ("pageable", "pinned"):
        for off, size in [(0, 65536), (24, 40), (123456, 4096)]:
            data = np.random.Generator(np.random.PCG64(off + size)).integers(
                0, 256, size, dtype=np.uint8)
            if src_kind == "pinned":
                pinned.array[:size] = data
                src = pinned.array[:size]
            else:
                src = data.copy()
            copy_cpu_to_gpu_async(dev.ptr, off, src, size, s)
            s.synchronize()
            ref[off: off + size] = data
            assert np.array_equal(dev.download(), ref), (src_kind, off, size)
    with pytest.raises(_lib.PegaFlowError, match="CPU buffer too small: 8 bytes, need 9 bytes"):
        copy_cpu_to_gpu_async(dev.ptr, 0, np.ones(8, np.uint8), 9, s)
    s.synchronize()
    assert np.array_equal(dev.download(), ref)
    pinned.close()
    s.close()
    dev.close()


LAYOUTS = {
    # name: (num_blocks, bytes_per_block, segments, kv_stride, size)
    "split": (96, 4096, 2, 96 * 4096, 2 * 96 * 4096),
    "split_padded": (96, 1024, 2, 100 * 1024, 100 * 1024 + 96 * 1024),
    "single": (64, 73728, 1, 0, 64 * 73728),
    "contig2": (50, 2048, 2, 2048, 51 * 2048),
    "strided": (40, 512, 2, 256, 39 * 512 + 256 + 512),
}


@pytest.mark.parametrize("name", list(LAYOUTS))
def test_copy_block_gpu_to_cpu_vs_oracle(gpu, name):
    """Every block of the layout: contiguous layouts copy block_size_bytes
    from segment 0's offset, the others each segment s to dst + s*bpb
    (transfer.rs:201-239)."""
    nb, bpb, segs, kv, size = LAYOUTS[name]
    say(f"[gpu] copy_block_gpu_to_cpu {name}")
    dev, ref = _tensor(size, 23)
    reg = KVCacheRegistration.create(dev.ptr, size, nb, bpb, kv, segs)
    oreg = oracle.layout(0, size, nb, bpb, kv, segs)
    contiguous = oracle.is_contiguous(oreg)
    for b in range(nb):
        dst = np.zeros(bpb * segs, np.uint8)
        if contiguous:
            o = oracle.segment_offset(oreg, b, 0)
            if o + bpb * segs > size:
                with pytest.raises(_lib.PegaFlowError, match=f"Block {b} exceeds registered"):
                    copy_block_gpu_to_cpu(reg, b, dst)
                continue
            expect = ref[o: o + bpb * segs]
        else:
            expect = np.concatenate([ref[oracle.segment_offset(oreg, b, s):][:bpb]
                                     for s in range(segs)])
        copy_block_gpu_to_cpu(reg, b, dst)
        assert np.array_equal(dst, expect), (name, b)
    with pytest.raises(_lib.PegaFlowError, match="exceeds registered memory"):
        copy_block_gpu_to_cpu(reg, nb + 100, np.zeros(bpb * segs, np.uint8))
    dev.close()


@pytest.mark.parametrize("host_kind", ["pinned", "pageable"])
@pytest.mark.parametrize("seed", range(3))
def test_batch_copy_segments_to_gpu_vs_oracle(gpu, host_kind, seed):
    """The load of one split layer as process_load_task issues it
    (gpu_worker.rs:226-256): the K list then the V list, each through
    batch_copy_segments_to_gpu.  The bytes equal the oracle's process_load
    and each list's batch count equals the oracle's merged runs.  Targets mix
    sorted stretches (long runs) with random blocks; the host regions are the
    save layout of lib.rs:636-705."""
    rng = np.random.Generator(np.random.PCG64(seed))
    nb, bpb = 512, 2048
    kv = nb * bpb
    size = 2 * kv
    dev, ref = _tensor(size, 31 + seed)
    reg = KVCacheRegistration.create(dev.ptr, size, nb, bpb, kv, 2)
    oreg = oracle.layout(ref.ctypes.data, size, nb, bpb, kv, 2)
    n = 200
    start = int(rng.integers(0, nb - 100))
    targets = np.concatenate([np.arange(start, start + 60),
                              rng.choice(np.setdiff1d(np.arange(nb),
                                                      np.arange(start, start + 60)),
                                         n - 60, replace=False)])
    host_bytes = rng.integers(0, 256, 2 * n * bpb, dtype=np.uint8)
    if host_kind == "pinned":
        pool = PinnedBuffer(2 * n * bpb)
        pool.array[:] = host_bytes
        base = pool.ptr
    else:
        pool = None
        keep = host_bytes.copy()
        base = keep.ctypes.data
    k_src = base + np.arange(n, dtype=np.uint64) * bpb
    v_src = base + n * bpb + np.arange(n, dtype=np.uint64) * bpb
    # The oracle reads its own copy of the host regions.
    ohost = host_bytes.copy()
    ok_ = ohost.ctypes.data + np.arange(n, dtype=np.uint64) * bpb
    ov = ohost.ctypes.data + n * bpb + np.arange(n, dtype=np.uint64) * bpb
    s = Stream()
    say(f"[gpu] batch_copy_segments_to_gpu {host_kind} seed={seed}")
    got_batches = []
    for seg, src in ((0, k_src), (1, v_src)):
        offs = [segment_offset(reg, int(b), seg) for b in targets]
        got_batches.append(batch_copy_segments_to_gpu(offs, src, bpb, reg, s))
    s.synchronize()
    oracle.process_load(oreg, ref, targets, ok_, ov)
    assert np.array_equal(dev.download(), ref)
    expect = []
    for seg, src in ((0, ok_), (1, ov)):
        offs = [oracle.segment_offset(oreg, int(b), seg) for b in targets]
        expect.append(len(oracle.merge_runs(offs, src, bpb)))
    assert got_batches == expect
    assert 1 < expect[0] < n  # the sorted stretch merged, the random part did not
    s.close()
    if pool is not None:
        pool.close()
    dev.close()
