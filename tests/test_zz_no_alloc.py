"""pf_load_layers_noalloc, the load entry point that allocates nothing,
against pf_load_layers (PF_MODE_KERNEL) on the same inputs: two twin sets of
layer tensors filled with the same words, one restored through each entry
point, compared byte for byte on the device.

  * Two calls in a row on one stream with no wait between them, the second
    smaller and overlapping the first's targets: the second call's
    descriptors and tile queue reuse the static scratch while the first may
    still run.
  * Device-memory sources (fixed-map launches), unaligned host regions (the
    byte kernel), an overlapping layout (in-order copies), repeated targets
    (the last copy wins), and the current device's null stream; these small
    cases are also checked against the oracle.
  * The scratch's limit: exactly PF_NOALLOC_MAX_CHUNKS chunks pass, one more
    is refused before anything is issued.
  * Graph capture: on a stream that is capturing, the call is refused with
    PF_ERR_UNSUPPORTED before anything is issued (the shared scratch cannot
    hold a captured call's descriptors), and the stream works afterwards.
"""

import ctypes
import sys

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.runtime import DeviceBuffer, PinnedBuffer, Stream, compare
from pegaflow_amd.transfer import (KVCacheRegistration, LayerTransfer, TransferContext,
                                   block_array, load_layers_noalloc)

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Twins:
    """Two identical sets of split KV-first layer tensors."""

    def __init__(self, n_layers, nb, bpb, seed, kv=None, size=None):
        self.nb, self.bpb = nb, bpb
        self.kv = nb * bpb if kv is None else kv
        self.size = self.kv + nb * bpb if size is None else size
        self.seeds = [oracle.layer_seed(seed, l) for l in range(n_layers)]
        self.x, self.y = [], []
        for s in self.seeds:
            for side in (self.x, self.y):
                b = DeviceBuffer(self.size)
                b.fill_random(s)
                side.append(b)

    def regs(self, side):
        return [KVCacheRegistration.create(b.ptr, self.size, self.nb, self.bpb, self.kv, 2)
                for b in side]

    def mismatches(self):
        return sum(compare(a.ptr, b.ptr, self.size) for a, b in zip(self.x, self.y))

    def close(self):
        for b in self.x + self.y:
            b.close()


def _loads(regs, targets, k_base, v_base, bpb):
    n = len(targets)
    k = k_base + np.arange(n, dtype=np.uint64) * bpb
    v = v_base + np.arange(n, dtype=np.uint64) * bpb
    return [LayerTransfer(r, block_array(targets, k + l * 2 * n * bpb, v + l * 2 * n * bpb))
            for l, r in enumerate(regs)]


@pytest.fixture(scope="module")
def ctx(gpu):
    c = TransferContext(0)
    yield c
    c.close()


def test_two_calls_in_a_row_second_smaller(ctx):
    """8 Llama-shape layers [2, 2000, 16, 8, 128] from pinned memory: 640
    targets (10,240 chunks, queued launch), then at once 100 other targets,
    half of them among the first call's."""
    n_layers, nb, bpb = 8, 2000, 32768
    t = Twins(n_layers, nb, bpb, seed=5)
    rng = np.random.Generator(np.random.PCG64(5))
    n1, n2 = 640, 100
    pool = PinnedBuffer(n_layers * 2 * (n1 + n2) * bpb)
    oracle.fill_random(pool.array, 77)
    t1 = rng.choice(nb, n1, replace=False)
    t2 = np.concatenate([t1[:50], rng.choice(np.setdiff1d(np.arange(nb), t1), 50,
                                             replace=False)])
    base2 = pool.ptr + n_layers * 2 * n1 * bpb
    stream = Stream()
    for rnd in range(2):  # the same scratch serves the next pair of calls
        say(f"[gpu] noalloc two calls in a row, round {rnd}")
        for side in (t.x, t.y):
            for b, s in zip(side, t.seeds):
                b.fill_random(s + rnd)
        load_layers_noalloc(_loads(t.regs(t.x), t1, pool.ptr, pool.ptr + n1 * bpb, bpb), stream)
        load_layers_noalloc(_loads(t.regs(t.x), t2, base2, base2 + n2 * bpb, bpb), stream)
        stream.synchronize()
        ctx.load_layers(_loads(t.regs(t.y), t1, pool.ptr, pool.ptr + n1 * bpb, bpb))
        ctx.load_layers(_loads(t.regs(t.y), t2, base2, base2 + n2 * bpb, bpb))
        ctx.synchronize()
        assert t.mismatches() == 0
    stream.close()
    pool.close()
    t.close()


def _small_case(ctx, stream, nb, bpb, kv, size, targets, src_kind, host_offset, seed):
    """One layer restored through both entry points and on the oracle."""
    t = Twins(1, nb, bpb, seed, kv=kv, size=size)
    n = len(targets)
    if src_kind == "device":
        src = DeviceBuffer(2 * n * bpb + 4096)
        data = np.random.Generator(np.random.PCG64(seed)).integers(
            0, 256, 2 * n * bpb, dtype=np.uint8)
        src.upload(np.concatenate([np.zeros(host_offset, np.uint8), data]))
    else:
        src = PinnedBuffer(2 * n * bpb + 4096)
        data = np.random.Generator(np.random.PCG64(seed)).integers(
            0, 256, 2 * n * bpb, dtype=np.uint8)
        src.array[host_offset: host_offset + 2 * n * bpb] = data
    base = src.ptr + host_offset
    load_layers_noalloc(_loads(t.regs(t.x), targets, base, base + n * bpb, bpb), stream)
    if stream is None:
        from pegaflow_amd import runtime
        runtime.synchronize()
    else:
        stream.synchronize()
    ctx.load_layers(_loads(t.regs(t.y), targets, base, base + n * bpb, bpb))
    ctx.synchronize()
    assert t.mismatches() == 0
    # The oracle on a CPU copy of the original layer.
    ref = np.zeros(size, np.uint8)
    oracle.fill_random(ref, t.seeds[0])
    host = data.copy()
    oreg = oracle.layout(ref.ctypes.data, size, nb, bpb, kv, 2)
    k = host.ctypes.data + np.arange(n, dtype=np.uint64) * bpb
    v = host.ctypes.data + n * bpb + np.arange(n, dtype=np.uint64) * bpb
    oracle.process_load(oreg, ref, targets, k, v)
    assert np.array_equal(t.x[0].download(), ref)
    src.close()
    t.close()


@pytest.mark.parametrize("src_kind", ["pinned", "device"])
def test_small_cases_vs_load_layers_and_oracle(ctx, src_kind):
    stream = Stream()
    say(f"[gpu] noalloc small cases src={src_kind}")
    nb, bpb = 64, 4096
    # Split layout, repeated targets (the last copy wins).
    _small_case(ctx, stream, nb, bpb, nb * bpb, 2 * nb * bpb, [3, 9, 3, 60, 9, 0], src_kind,
                0, 1)
    # Host regions 8 bytes off 16-byte alignment: the byte kernel.
    _small_case(ctx, stream, nb, bpb, nb * bpb, 2 * nb * bpb, [5, 6, 7, 40], src_kind, 8, 2)
    # Overlapping split layout (kv_stride < num_blocks * bpb): in-order copies.
    _small_case(ctx, stream, 16, 256, 1024, 1024 + 16 * 256, [2, 5, 3, 2], src_kind, 0, 3)
    # The current device's null stream.
    _small_case(ctx, None, nb, bpb, nb * bpb, 2 * nb * bpb, [1, 2, 62], src_kind, 0, 4)
    stream.close()


def test_scratch_limit(ctx):
    """32 layers x 1024 blocks x 2 segments = 65,536 chunks fill the scratch
    exactly; 1025 blocks are refused before anything is issued."""
    say("[gpu] noalloc scratch limit")
    n_layers, nb, bpb = 32, 1100, 256
    t = Twins(n_layers, nb, bpb, seed=9)
    pool = PinnedBuffer(n_layers * 2 * 1025 * bpb)
    oracle.fill_random(pool.array, 99)
    stream = Stream()
    targets = np.arange(1024)[::-1]
    assert n_layers * 2 * len(targets) == _lib.NOALLOC_MAX_CHUNKS
    load_layers_noalloc(_loads(t.regs(t.x), targets, pool.ptr, pool.ptr + 1024 * bpb, bpb),
                        stream)
    stream.synchronize()
    ctx.load_layers(_loads(t.regs(t.y), targets, pool.ptr, pool.ptr + 1024 * bpb, bpb))
    ctx.synchronize()
    assert t.mismatches() == 0
    with pytest.raises(_lib.PegaFlowError, match="65600 chunks exceed the 65536-chunk scratch"):
        load_layers_noalloc(_loads(t.regs(t.x), np.arange(1025), pool.ptr,
                                   pool.ptr + 1025 * bpb, bpb), stream)
    stream.synchronize()
    assert t.mismatches() == 0  # nothing was issued
    stream.close()
    pool.close()
    t.close()


def _hip():
    """The HIP runtime the library itself is linked against."""
    h = ctypes.CDLL("libamdhip64.so.7")
    h.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    h.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    h.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    return h


def test_graph_capture_is_refused(ctx):
    """A call on a capturing stream fails with PF_ERR_UNSUPPORTED and leaves
    nothing in the graph; the same call after the capture ends restores the
    same bytes as pf_load_layers."""
    say("[gpu] noalloc under graph capture")
    nb, bpb = 64, 4096
    t = Twins(1, nb, bpb, seed=11)
    targets = np.array([4, 17, 33, 2], dtype=np.int64)
    n = len(targets)
    pool = PinnedBuffer(2 * n * bpb)
    oracle.fill_random(pool.array, 123)
    stream = Stream()
    hip = _hip()
    relaxed = 2  # hipStreamCaptureModeRelaxed
    assert hip.hipStreamBeginCapture(stream.handle, relaxed) == 0
    graph = ctypes.c_void_p()
    try:
        with pytest.raises(_lib.PegaFlowError, match="capturing a graph") as ei:
            load_layers_noalloc(_loads(t.regs(t.x), targets, pool.ptr, pool.ptr + n * bpb, bpb),
                                stream)
        assert ei.value.code == _lib.PF_ERR_UNSUPPORTED
    finally:
        assert hip.hipStreamEndCapture(stream.handle, ctypes.byref(graph)) == 0
        if graph.value:
            hip.hipGraphDestroy(graph)
    stream.synchronize()
    assert t.mismatches() == 0  # nothing was issued
    load_layers_noalloc(_loads(t.regs(t.x), targets, pool.ptr, pool.ptr + n * bpb, bpb), stream)
    stream.synchronize()
    ctx.load_layers(_loads(t.regs(t.y), targets, pool.ptr, pool.ptr + n * bpb, bpb))
    ctx.synchronize()
    assert t.mismatches() == 0
    stream.close()
    pool.close()
    t.close()
