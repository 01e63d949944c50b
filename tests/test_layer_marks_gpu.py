"""GPU tests of layer marks: per-layer completion written by the load itself.

A marked load (pf_load_layers_marked) sets word l of every signal target to
the call's value once layer l's bytes are in place.  These tests check, on
device 0 through the C ABI:
  * bytes: identical to the oracle in every transfer mode, for layer lists
    that mix aligned, unaligned (8-byte host offset), empty and in-order
    (overlapping layout) layers;
  * marks: every word of every target (host and device memory) holds the
    value after the call, and repeated calls with larger values re-mark every
    layer (the kernel's tile counters return to zero after each launch);
  * ordering: a consumer stream that waits on layer l's device word and then
    copies layer l always copies the restored bytes;
  * the bounded wait ends on its time limit when the word is never set.
"""

import sys

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.runtime import (DeviceBuffer, PinnedBuffer, Stream, memcpy_async,
                                  stream_wait_word, host_wait_word, verify_random_chunks)
from pegaflow_amd.transfer import (KVCacheRegistration, LayerTransfer, TransferContext,
                                   block_array)

pytestmark = pytest.mark.gpu

MODES = {"dma_reference": _lib.MODE_DMA_REFERENCE, "dma_batched": _lib.MODE_DMA_BATCHED,
         "kernel": _lib.MODE_KERNEL, "staged": _lib.MODE_STAGED}
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx(gpu):
    c = TransferContext(0, staging_bytes=16 * MiB)
    yield c
    c.close()


class Case:
    """One layer of a mixed marked load, with its oracle copy."""

    def __init__(self, nb, bpb, segs, kv, size, save_ids, load_ids, seed, host_offset=0):
        self.dev = DeviceBuffer(size)
        self.dev.fill_random(seed)
        self.ref = self.dev.download()
        self.reg = KVCacheRegistration.create(self.dev.ptr, size, nb, bpb, kv, segs)
        self.oreg = oracle.layout(self.ref.ctypes.data, size, nb, bpb, kv, segs)
        m = max(len(save_ids), 1)
        self.host = PinnedBuffer(2 * m * bpb * segs + 4096)
        base = self.host.ptr + host_offset
        self.k, self.v, self.split = oracle.save_host_layout(self.oreg, len(save_ids), base,
                                                             base + len(save_ids) * bpb)
        self.save_ids, self.load_ids = save_ids, load_ids
        self.ohost = np.zeros(self.host.nbytes, np.uint8)
        obase = self.ohost.ctypes.data + host_offset
        self.ok_, self.ov, _ = oracle.save_host_layout(self.oreg, len(save_ids), obase,
                                                       obase + len(save_ids) * bpb)

    def save(self, ctx, mode):
        self.host.array[:] = 0
        ctx.save_layers([LayerTransfer(self.reg, block_array(self.save_ids, self.k,
                                                             self.v if self.split else None))],
                        mode)
        oracle.process_save(self.oreg, self.ref, self.save_ids, self.ok_,
                            self.ov if self.split else None)
        assert np.array_equal(self.host.array, self.ohost)

    def load_transfer(self):
        return LayerTransfer(self.reg, block_array(self.load_ids, self.k,
                                                   self.v if self.split else None))

    def check_load(self):
        oracle.process_load(self.oreg, self.ref, self.load_ids, self.ok_,
                            self.ov if self.split else None)
        assert np.array_equal(self.dev.download(), self.ref)

    def close(self):
        self.dev.close()
        self.host.close()


def _mixed_cases(seed):
    nb, bpb = 40, 256
    kv = nb * bpb
    return [
        Case(nb, bpb, 2, kv, 2 * kv, [3, 9, 27, 1], [0, 5, 39, 12], seed),
        Case(nb, bpb, 2, kv, 2 * kv, [4, 5], [6, 7], seed + 1, host_offset=8),  # unaligned
        Case(nb, bpb, 2, kv, 2 * kv, [], [], seed + 2),  # empty layer
        Case(nb, bpb, 2, kv, 2 * kv, list(range(nb))[::-1], list(range(nb)), seed + 3),
        Case(10, 64, 2, 160, 160 + 640, [1, 2, 3], [4, 3, 2], seed + 4),  # overlapping: in order
        Case(nb, 4608, 1, 0, nb * 4608, [9, 1, 30], [2, 3, 4], seed + 5),  # blocks-first
        Case(nb, bpb, 2, kv, 2 * kv, [11, 12, 13], [13, 12, 11], seed + 6),
    ]


@pytest.mark.parametrize("mode", list(MODES))
def test_marked_load_mixed_layers_vs_oracle(ctx, mode):
    say(f"[gpu] marked load, mixed layers, mode={mode}")
    cases = _mixed_cases(40)
    L = len(cases)
    host_words = PinnedBuffer(8 * L)
    dev_words = DeviceBuffer(8 * L)
    dev_words.memset(0)
    host_words.array[:] = 0
    try:
        for value in (5, 6):  # a second call re-marks every layer
            for c in cases:
                c.dev.upload(c.ref)  # start from the oracle's current bytes
                c.save(ctx, MODES[mode])
            ctx.load_layers_marked([c.load_transfer() for c in cases],
                                   [(host_words.ptr, value, True), (dev_words.ptr, value, False)],
                                   MODES[mode])
            ctx.synchronize()
            hw = host_words.array.view(np.uint64)
            dw = dev_words.download().view(np.uint64)
            assert hw.tolist() == [value] * L, f"host marks {hw.tolist()}"
            assert dw.tolist() == [value] * L, f"device marks {dw.tolist()}"
            for c in cases:
                c.check_load()
    finally:
        for c in cases:
            c.close()
        host_words.close()
        dev_words.close()


def test_pipelined_marked_load_vs_oracle(ctx):
    """A marked load large enough to be issued in two parts (16 layers,
    about 30K chunks from pinned memory): the second part's marks use the
    call-wide layer index, so every word of both targets holds the value,
    twice in a row (the tile counters return to zero), with an empty layer
    and an in-order (overlapping) layer in the second part; bytes against
    the oracle.  Three copy launches: layers 0-1, 2-11, 13-15 (layer 12 is
    copied in order by DMA); issued whole it would be two.  The first part
    (2 x 32 MiB) is still running when the second part's descriptors are
    uploaded, so they must not overlap the first part's mark tables."""
    say("[gpu] pipelined marked load vs oracle")
    rng = np.random.Generator(np.random.PCG64(77))
    nb, bpb, m = 1100, 256, 1024
    cases = []
    for l in range(16):
        if l < 2:  # the first part: 32 MiB per layer, still copying while the rest is issued
            cases.append(Case(600, 32768, 2, 600 * 32768, 2 * 600 * 32768,
                              rng.choice(600, 512, replace=False).tolist(),
                              rng.choice(600, 512, replace=True).tolist(), 500 + l))
        elif l == 12:
            cases.append(Case(10, bpb, 2, 1280, 1280 + 2560, [1, 2, 3], [4, 3, 2], 500 + l))
        elif l == 9:
            cases.append(Case(nb, bpb, 2, nb * bpb, 2 * nb * bpb, [], [], 500 + l))
        else:
            cases.append(Case(nb, bpb, 2, nb * bpb, 2 * nb * bpb,
                              rng.choice(nb, m, replace=False).tolist(),
                              rng.choice(nb, m, replace=True).tolist(), 500 + l))
    L = len(cases)
    host_words = PinnedBuffer(8 * L)
    dev_words = DeviceBuffer(8 * L)
    dev_words.memset(0)
    host_words.array[:] = 0
    try:
        for c in cases:
            c.save(ctx, _lib.MODE_KERNEL)
        for value in (5, 6):
            ctx.load_layers_marked([c.load_transfer() for c in cases],
                                   [(host_words.ptr, value, True), (dev_words.ptr, value, False)],
                                   _lib.MODE_KERNEL)
            ctx.synchronize()
            assert ctx.last_stats()[0] == 3, f"copy launches {ctx.last_stats()[0]}"
            hw = host_words.array.view(np.uint64)
            dw = dev_words.download().view(np.uint64)
            assert hw.tolist() == [value] * L, f"host marks {hw.tolist()}"
            assert dw.tolist() == [value] * L, f"device marks {dw.tolist()}"
            for c in cases:
                c.check_load()
    finally:
        for c in cases:
            c.close()
        host_words.close()
        dev_words.close()


def test_marked_load_rejects_bad_targets(ctx):
    say("[gpu] marked load argument checks")
    c = Case(16, 512, 2, 16 * 512, 2 * 16 * 512, [1], [2], 3)
    words = PinnedBuffer(64)
    try:
        lt = [c.load_transfer()]
        for bad in ([(words.ptr, 0, True)],                 # value 0
                    [(words.ptr + 4, 1, True)],             # misaligned
                    [(12345678 * 4096, 1, False)],          # not an allocation
                    [(words.ptr, 1, True)] * 5,             # too many targets
                    []):                                    # none
            with pytest.raises(_lib.PegaFlowError):
                ctx.load_layers_marked(lt, bad, _lib.MODE_KERNEL)
        # Too short for the layer count: 2 layers need 16 bytes from the end.
        with pytest.raises(_lib.PegaFlowError):
            ctx.load_layers_marked(lt * 2, [(words.ptr + 56, 1, True)], _lib.MODE_KERNEL)
    finally:
        c.close()
        words.close()


def test_device_wait_orders_consumer_per_layer(ctx):
    """Qwen3-8B layer shape (bf16 [2, N, 16, 8, 128]), 12 layers of 2048
    blocks, 313 random blocks restored from pinned memory in one marked
    launch.  A consumer stream waits on each layer's device word and then
    snapshots that layer; every snapshot must hold the restored bytes, which
    it could not if a wait ended before that layer's copy had landed (the
    snapshots are queued within microseconds, the layers take ~0.4 ms each)."""
    say("[gpu] device-side per-layer wait, 12 layers x 313 blocks")
    n_layers, nb, bpb, n = 12, 2048, 32768, 313
    kv = nb * bpb
    size = 2 * kv
    rng = np.random.Generator(np.random.PCG64(5))
    ids = rng.choice(nb, n, replace=False)
    targets = rng.choice(np.setdiff1d(np.arange(nb), ids), n, replace=False)
    seeds = [oracle.layer_seed(17, l) for l in range(n_layers)]
    bufs = [DeviceBuffer(size) for _ in range(n_layers)]
    snaps = [DeviceBuffer(size) for _ in range(n_layers)]
    host = PinnedBuffer(n_layers * n * 2 * bpb)
    host_words = PinnedBuffer(8 * n_layers)
    dev_words = DeviceBuffer(8 * n_layers)
    flag = DeviceBuffer(4 * n_layers)
    consumer = Stream()
    try:
        regs, saved = [], []
        for l, b in enumerate(bufs):
            b.fill_random(seeds[l])
            reg = KVCacheRegistration.create(b.ptr, size, nb, bpb, kv, 2)
            base = host.ptr + l * n * 2 * bpb
            regs.append(reg)
            saved.append(LayerTransfer(reg, block_array(ids.tolist(),
                                                        base + np.arange(n) * bpb,
                                                        base + n * bpb + np.arange(n) * bpb)))
        ctx.save_layers(saved, _lib.MODE_KERNEL)
        loads = []
        for reg, lt in zip(regs, saved):
            blk = lt.blocks.copy()
            blk["block_idx"] = targets
            loads.append(LayerTransfer(reg, blk))
        for value in (1, 2):
            for l, b in enumerate(bufs):
                b.fill_random(seeds[l])
            if value == 1:
                dev_words.memset(0)
            flag.memset(0)
            ctx.load_layers_marked(loads, [(host_words.ptr, value, True),
                                           (dev_words.ptr, value, False)], _lib.MODE_KERNEL)
            for l in range(n_layers):
                stream_wait_word(consumer, dev_words.ptr + 8 * l, value, 10_000_000,
                                 flag.ptr + 4 * l)
                memcpy_async(snaps[l].ptr, bufs[l].ptr, size, consumer)
            for l in range(n_layers):
                assert host_wait_word(host_words.ptr + 8 * l, value, 10_000_000)
            consumer.synchronize()
            ctx.synchronize()
            assert not flag.download().any(), "a device wait timed out"
            # Every snapshot: restored targets hold their source block, others unchanged.
            blocks = np.arange(nb, dtype=np.uint64)
            src = blocks.copy()
            src[targets] = ids
            for l in range(n_layers):
                addrs = np.concatenate([snaps[l].ptr + blocks * bpb,
                                        snaps[l].ptr + kv + blocks * bpb])
                offs = np.concatenate([src * bpb // 8, (kv + src * bpb) // 8])
                assert verify_random_chunks(addrs, offs, bpb, seeds[l]) == 0, f"layer {l}"
    finally:
        consumer.close()
        for b in bufs + snaps:
            b.close()
        host.close()
        host_words.close()
        dev_words.close()
        flag.close()


def test_bounded_wait_times_out(gpu):
    """A word the host never sets: the wait kernel ends on its time limit,
    flags the timeout, and later work on the stream runs."""
    say("[gpu] bounded device wait time-out (2 ms)")
    word = DeviceBuffer(8)
    flag = DeviceBuffer(4)
    out = DeviceBuffer(64)
    src = DeviceBuffer(64)
    s = Stream()
    try:
        word.memset(0)
        flag.memset(0)
        out.memset(0)
        src.fill_random(3)
        stream_wait_word(s, word.ptr, 1, 2000, flag.ptr)
        memcpy_async(out.ptr, src.ptr, 64, s)
        s.synchronize()
        assert flag.download().view(np.uint32)[0] == 1
        assert np.array_equal(out.download(), src.download())
        # A word already at the value: no wait and no flag.
        flag.memset(0)
        word.upload(np.array([7], np.uint64).view(np.uint8))
        stream_wait_word(s, word.ptr, 7, 2000, flag.ptr)
        s.synchronize()
        assert flag.download().view(np.uint32)[0] == 0
    finally:
        s.close()
        for b in (word, flag, out, src):
            b.close()
