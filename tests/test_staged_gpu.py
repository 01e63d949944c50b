"""GPU parity of the staged mode's slicing, and of PF_MODE_AUTO's choice.

The staged mode cuts a call's chunks, in layer order, into slices that may
span layers and alternate between the context's two streams.  These tests
shrink the slices to a few chunks so that slices cross layer boundaries,
chunk-size changes, empty layers and layers copied in place in list order,
and compare every byte with the oracle (each layer's save and load restated
on the host, in the reference's order).
"""

import sys

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.runtime import DeviceBuffer, Event, PinnedBuffer, copy_engines
from pegaflow_amd.transfer import KVCacheRegistration, LayerTransfer, TransferContext, block_array

pytestmark = pytest.mark.gpu
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Layer:
    """One layer tensor with its oracle copy; host regions at given offsets
    of a pinned buffer shared by the call's layers (and the same offsets of a
    numpy buffer for the oracle)."""

    def __init__(self, nb, bpb, segs, kv, size, seed):
        self.dev = DeviceBuffer(size)
        self.dev.fill_random(seed)
        self.ref = self.dev.download()
        self.reg = KVCacheRegistration.create(self.dev.ptr, size, nb, bpb, kv, segs)
        self.oreg = oracle.layout(self.ref.ctypes.data, size, nb, bpb, kv, segs)
        self.bpb = bpb

    def place(self, ids, host, ohost, off):
        """The reference's host layout for `ids` at byte `off` of both buffers."""
        n = len(ids)
        self.k, self.v, self.split = oracle.save_host_layout(
            self.oreg, n, host.ptr + off, host.ptr + off + n * self.bpb)
        self.ok_, self.ov, _ = oracle.save_host_layout(
            self.oreg, n, ohost.ctypes.data + off, ohost.ctypes.data + off + n * self.bpb)
        self.save_ids = list(ids)

    def transfer(self, ids):
        return LayerTransfer(self.reg, block_array(ids, self.k, self.v if self.split else None))

    def oracle_save(self):
        oracle.process_save(self.oreg, self.ref, self.save_ids, self.ok_,
                            self.ov if self.split else None)

    def oracle_load(self, ids):
        oracle.process_load(self.oreg, self.ref, ids, self.ok_, self.ov if self.split else None)

    def close(self):
        self.dev.close()


def _mixed_layers(seed):
    """Split layers of two segment sizes, an empty one, an overlapping layout
    (its loads are copied in place, in list order), a blocks-first layer and
    an unaligned one; with their save and load ids."""
    nb, bpb = 40, 256
    kv = nb * bpb
    specs = [
        ((nb, bpb, 2, kv, 2 * kv), [3, 9, 27, 1, 30, 31, 32], [0, 5, 39, 12, 13, 14, 15]),
        ((nb, bpb, 2, kv, 2 * kv), list(range(nb))[::-1], list(range(nb))),
        ((nb, bpb, 2, kv, 2 * kv), [], []),
        ((nb, 512, 2, nb * 512, 2 * nb * 512), [4, 5, 6, 7, 8], [9, 9, 1, 2, 9]),
        ((10, 64, 2, 160, 160 + 640), [1, 2, 3], [4, 3, 2]),
        ((nb, 4608, 1, 0, nb * 4608), [9, 1, 30, 2], [2, 3, 4, 5]),
        ((30, 24, 2, 30 * 24 + 8, 30 * 24 * 2 + 8), [4, 5, 6], [20, 0, 29]),
        ((nb, bpb, 2, kv, 2 * kv), [11, 12, 13], [13, 12, 11]),
    ]
    layers = [Layer(*shape, seed + i) for i, (shape, _, _) in enumerate(specs)]
    return layers, [s for _, s, _ in specs], [l for _, _, l in specs]


class PageableBuffer:
    """Ordinary (pageable) host memory with PinnedBuffer's fields: staged
    copies to and from it go through HIP, not the copy engines."""

    def __init__(self, nbytes):
        self.array = np.zeros(nbytes, np.uint8)
        self.ptr = self.array.ctypes.data
        self.nbytes = nbytes

    def close(self):
        self.array = None


def _place_all(layers, save_ids, gap=0, pinned=True):
    """Host regions of all layers one after another, `gap` bytes apart (a gap
    that is not a multiple of 16 leaves later regions unaligned)."""
    regions = [2 * max(len(ids), 1) * L.bpb for L, ids in zip(layers, save_ids)]
    size = sum(regions) + gap * len(regions)
    host = PinnedBuffer(size) if pinned else PageableBuffer(size)
    ohost = np.zeros(size, np.uint8)
    off = 0
    for L, ids, r in zip(layers, save_ids, regions):
        L.place(ids, host, ohost, off)
        off += r + gap
    return host, ohost


@pytest.mark.parametrize("slices,pinned,grid", [((3000, 5000), True, 0), ((1, 1), True, 0),
                                                ((65536, 2048), True, 0),
                                                ((3000, 5000), False, 0),
                                                ((3000, 5000), False, 3),
                                                ((1, 1), False, 2)])
def test_staged_slices_across_layers_vs_oracle(gpu, slices, pinned, grid):
    """One staged save, then one staged load with per-layer events, of eight
    mixed layers, with slices of a few chunks (or one chunk each): host
    regions and every layer tensor equal the oracle's; the layer events
    complete in layer order.  A second load of the same call with layer marks
    sets every layer's word.  Pinned host regions take the copy engines;
    pageable ones HIP's copies over the context's two streams.  grid > 0
    runs the device routes' kernels queued, on both streams at once."""
    say(f"[gpu] staged slices across layers, slice caps {slices}, pinned={pinned}, "
        f"device-route grid {grid}")
    ctx = TransferContext(0, staging_bytes=64 * 1024)
    ctx.set_staged_slices(*slices)
    if grid:
        ctx.set_route_grid(_lib.ROUTE_SAVE_DEVICE, grid)
        ctx.set_route_grid(_lib.ROUTE_LOAD_DEVICE, grid)
    layers, save_ids, load_ids = _mixed_layers(70)
    host, ohost = _place_all(layers, save_ids, gap=8, pinned=pinned)
    words = PinnedBuffer(8 * len(layers))
    try:
        host.array[:] = 0
        ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)], _lib.MODE_STAGED)
        for L in layers:
            L.oracle_save()
        assert np.array_equal(host.array, ohost), "host regions differ from the oracle"
        evs = [Event() for _ in layers]
        ctx.load_layers([L.transfer(ids) for L, ids in zip(layers, load_ids)], _lib.MODE_STAGED,
                        layer_events=evs)
        ctx.synchronize()
        for i in range(1, len(evs)):
            assert evs[i - 1].elapsed_ms(evs[i]) >= 0.0, f"layer {i} completed before {i - 1}"
        for L, ids in zip(layers, load_ids):
            L.oracle_load(ids)
            assert np.array_equal(L.dev.download(), L.ref), "layer differs from the oracle"
        # The same load again, marked: its bytes are unchanged (the oracle
        # already holds them) and every word is set.
        words.array[:] = 0
        ctx.load_layers_marked([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                               [(words.ptr, 7, True)], _lib.MODE_STAGED)
        ctx.synchronize()
        assert words.array.view(np.uint64).tolist() == [7] * len(layers)
        for L in layers:
            assert np.array_equal(L.dev.download(), L.ref)
    finally:
        for L in layers:
            L.close()
        host.close()
        words.close()
        ctx.close()


def test_staged_two_lanes_queued_vs_oracle(gpu):
    """Four split layers [2, 512, 16, 8, 128] from pageable memory, 200 random
    blocks each, staged in 1 MiB slices over the context's two streams with
    both device routes queued on 16 workgroups: each stream's kernels pull
    tiles from a queue of their own while the other stream's run, and every
    byte of the save and of the load equals the oracle's."""
    say("[gpu] staged save/load over two lanes, queued device routes")
    nb, bpb = 512, 32768
    rng = np.random.Generator(np.random.PCG64(31))
    layers = [Layer(nb, bpb, 2, nb * bpb, 2 * nb * bpb, 300 + i) for i in range(4)]
    save_ids = [rng.choice(nb, 200, replace=False).tolist() for _ in layers]
    load_ids = [rng.choice(nb, 200, replace=False).tolist() for _ in layers]
    host, ohost = _place_all(layers, save_ids, pinned=False)
    ctx = TransferContext(0, staging_bytes=4 * MiB)
    ctx.set_staged_slices(MiB, MiB)
    ctx.set_route_grid(_lib.ROUTE_SAVE_DEVICE, 16)
    ctx.set_route_grid(_lib.ROUTE_LOAD_DEVICE, 16)
    try:
        for rnd in range(2):
            ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)],
                            _lib.MODE_STAGED)
            for L in layers:
                L.oracle_save()
            assert np.array_equal(host.array, ohost), f"round {rnd}: host regions differ"
            ctx.load_layers([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                            _lib.MODE_STAGED)
            ctx.synchronize()
            for L, ids in zip(layers, load_ids):
                L.oracle_load(ids)
                assert np.array_equal(L.dev.download(), L.ref), f"round {rnd}: layer differs"
            launches, copies = ctx.last_stats()
            assert launches > 2 and copies > 2
    finally:
        for L in layers:
            L.close()
        host.close()
        ctx.close()


@pytest.mark.parametrize("head,staging,load_slice", [
    ("kernel", 64 * 1024, 0), ("engine", 64 * 1024, 0),
    ("kernel", 4 * MiB, 128 * 1024), ("engine", 4 * MiB, 128 * 1024)])
def test_staged_pipelined_load_vs_oracle(gpu, head, staging, load_slice):
    """A staged save and load large enough to be pipelined (9 layers, 19,606
    chunks).  The save slices its first layer onto the copy engine and plans
    the rest under that copy; the load copies its first layer (when the
    caller waits layer by layer: by the zero-copy kernel, or sliced onto the
    copy engine with the context's head route set so; else sliced onto the
    copy engine) before the other layers are planned.  With 64 KiB of
    staging the copies go through two 32 KiB slots; with 4 MiB and 128 KiB
    load slices, a load waited for layer by layer keeps 8 slots of 128 KiB.  After the first layer come an empty layer, a layer copied
    in place in list order, and a layer whose host region is ordinary
    (pageable) memory, copied through HIP run by run; slices start small and
    grow.  Bytes against the oracle for the save (pinned and pageable host
    regions), a load with per-layer events (in layer order), a marked load
    (every layer's mark set) and a plain one."""
    say(f"[gpu] staged pipelined load, mixed later layers, first layer by {head}, "
        f"staging {staging}, load slices {load_slice or 'default'}")
    ctx = TransferContext(0, staging_bytes=staging)
    ctx.set_staged_slices(0, load_slice)
    with pytest.raises(_lib.PegaFlowError, match="unknown staged head route 2"):
        ctx.set_staged_head(2)
    ctx.set_staged_head(_lib.STAGED_HEAD_KERNEL if head == "kernel" else _lib.STAGED_HEAD_ENGINE)
    nb, bpb = 2048, 256
    kv = nb * bpb
    rng = np.random.Generator(np.random.PCG64(31))
    specs = []  # (layer shape, save ids, load ids, host region pageable)
    for i in range(9):
        if i == 3:
            specs.append(((nb, bpb, 2, kv, 2 * kv), [], [], False))
        elif i == 5:
            specs.append(((10, 64, 2, 160, 160 + 640), [1, 2, 3], [4, 3, 2], False))
        else:
            specs.append(((nb, bpb, 2, kv, 2 * kv), rng.permutation(nb)[:1400].tolist(),
                          rng.permutation(nb)[:1400].tolist(), i == 7))
    layers = [Layer(*shape, 200 + i) for i, (shape, _, _, _) in enumerate(specs)]
    regions = [2 * max(len(save), 1) * L.bpb for L, (_, save, _, _) in zip(layers, specs)]
    pinned = PinnedBuffer(sum(regions))
    opinned = np.zeros(pinned.nbytes, np.uint8)
    pageable = PageableBuffer(regions[7])
    opage = np.zeros(pageable.nbytes, np.uint8)
    words = PinnedBuffer(8 * len(layers))
    off = 0
    for L, (_, save, _, paged), r in zip(layers, specs, regions):
        if paged:
            L.place(save, pageable, opage, 0)
        else:
            L.place(save, pinned, opinned, off)
            off += r
    loads = lambda: [L.transfer(ids) for L, (_, _, ids, _) in zip(layers, specs)]  # noqa: E731
    try:
        pinned.array[:] = 0
        ctx.save_layers([L.transfer(save) for L, (_, save, _, _) in zip(layers, specs)],
                        _lib.MODE_STAGED)
        for L in layers:
            L.oracle_save()
        assert np.array_equal(pinned.array, opinned), "pinned host regions differ"
        assert np.array_equal(pageable.array, opage), "pageable host region differs"
        evs = [Event() for _ in layers]
        ctx.load_layers(loads(), _lib.MODE_STAGED, layer_events=evs)
        ctx.synchronize()
        for i in range(1, len(evs)):
            assert evs[i - 1].elapsed_ms(evs[i]) >= 0.0, f"layer {i} completed before {i - 1}"
        for i, (L, (_, _, ids, _)) in enumerate(zip(layers, specs)):
            L.oracle_load(ids)
            assert np.array_equal(L.dev.download(), L.ref), f"layer {i} differs from the oracle"
        words.array[:] = 0
        ctx.load_layers_marked(loads(), [(words.ptr, 9, True)], _lib.MODE_STAGED)
        ctx.synchronize()
        assert words.array.view(np.uint64).tolist() == [9] * len(layers)
        for L in layers:
            assert np.array_equal(L.dev.download(), L.ref)
        # A load completed as a whole (no events, no marks) is staged for
        # every layer, the first included: into refilled tensors.
        for i, L in enumerate(layers):
            L.dev.fill_random(300 + i)
            L.ref[:] = L.dev.download()  # in place: the oracle's layout points here
        ctx.load_layers(loads(), _lib.MODE_STAGED)
        ctx.synchronize()
        for i, (L, (_, _, ids, _)) in enumerate(zip(layers, specs)):
            L.oracle_load(ids)
            assert np.array_equal(L.dev.download(), L.ref), f"plain load: layer {i} differs"
    finally:
        for L in layers:
            L.close()
        pinned.close()
        pageable.close()
        words.close()
        ctx.close()


def test_staged_head_route_from_setting_and_environment(gpu, monkeypatch):
    """The first layer's route of a layer-by-layer staged load: the default
    context copies it through the copy engines, a context set to the kernel
    and one created under PEGAFLOW_STAGED_HEAD=kernel copy it by the
    zero-copy kernel (fewer DMA copies for the same load, the same count for
    both); PEGAFLOW_STAGED_HEAD=engine gives the default's count.  Every
    context's load is checked against the oracle."""
    say("[gpu] staged head route: default, set, environment")
    nb, bpb = 2048, 256
    kv = nb * bpb
    rng = np.random.Generator(np.random.PCG64(57))
    specs = [(rng.permutation(nb)[:1000].tolist(), rng.permutation(nb)[:1000].tolist())
             for _ in range(9)]  # 18,000 chunks: pipelined
    layers = [Layer(nb, bpb, 2, kv, 2 * kv, 500 + i) for i in range(9)]
    host, ohost = _place_all(layers, [save for save, _ in specs])
    words = PinnedBuffer(8 * len(layers))
    ctxs = []
    try:
        plain = TransferContext(0, staging_bytes=4 * MiB)
        ctxs.append(plain)
        plain.save_layers([L.transfer(save) for L, (save, _) in zip(layers, specs)],
                          _lib.MODE_KERNEL)
        for L in layers:
            L.oracle_save()
        assert np.array_equal(host.array, ohost)
        set_kernel = TransferContext(0, staging_bytes=4 * MiB)
        ctxs.append(set_kernel)
        set_kernel.set_staged_head(_lib.STAGED_HEAD_KERNEL)
        monkeypatch.setenv("PEGAFLOW_STAGED_HEAD", "kernel")
        ctxs.append(TransferContext(0, staging_bytes=4 * MiB))
        monkeypatch.setenv("PEGAFLOW_STAGED_HEAD", "engine")
        ctxs.append(TransferContext(0, staging_bytes=4 * MiB))
        monkeypatch.delenv("PEGAFLOW_STAGED_HEAD")
        dma = []
        for k, ctx in enumerate(ctxs):
            words.array[:] = 0
            ctx.load_layers_marked([L.transfer(load) for L, (_, load) in zip(layers, specs)],
                                   [(words.ptr, k + 1, True)], _lib.MODE_STAGED)
            ctx.synchronize()
            dma.append(ctx.last_stats()[1])
            assert words.array.view(np.uint64).tolist() == [k + 1] * len(layers)
            for i, (L, (_, load)) in enumerate(zip(layers, specs)):
                if k == 0:
                    L.oracle_load(load)
                assert np.array_equal(L.dev.download(), L.ref), f"context {k}: layer {i}"
        say(f"[gpu] DMA copies: default {dma[0]}, set to the kernel {dma[1]}, environment "
            f"kernel {dma[2]}, environment engine {dma[3]}")
        assert dma[0] > dma[1] == dma[2] and dma[3] == dma[0], dma
    finally:
        for c in ctxs:
            c.close()
        for L in layers:
            L.close()
        host.close()
        words.close()


def test_staged_save_overlapping_hosts_keeps_list_order(gpu):
    """Host destinations that overlap across layers (layer 1's region starts
    inside layer 0's V region): the staged save copies in list order, as the
    reference does, so the later copy's bytes are kept.  The third layer
    names one block twice (two host chunks with the same bytes)."""
    say("[gpu] staged save, overlapping host destinations")
    ctx = TransferContext(0, staging_bytes=64 * 1024)
    ctx.set_staged_slices(1024, 1024)
    nb, bpb = 32, 256
    kv = nb * bpb
    layers = [Layer(nb, bpb, 2, kv, 2 * kv, 90 + i) for i in range(3)]
    ids = [[1, 2, 3, 4], [5, 6, 7, 8], [9, 9, 10, 11]]
    size = 16 * bpb * 3
    host = PinnedBuffer(size)
    ohost = np.zeros(size, np.uint8)
    layers[0].place(ids[0], host, ohost, 0)
    layers[1].place(ids[1], host, ohost, 6 * bpb)          # inside layer 0's V region
    layers[2].place(ids[2], host, ohost, 20 * bpb)
    try:
        host.array[:] = 0
        ctx.save_layers([L.transfer(i) for L, i in zip(layers, ids)], _lib.MODE_STAGED)
        for L in layers:
            L.oracle_save()
        assert np.array_equal(host.array, ohost)
    finally:
        for L in layers:
            L.close()
        host.close()
        ctx.close()


def test_auto_mode_follows_host_runs(gpu):
    """PF_MODE_AUTO runs staged (DMA copies over the link) when the host side
    lies in long contiguous runs, as a save batch's regions do, and runs the
    zero-copy kernels when the host chunks are scattered; bytes are exact
    either way."""
    say("[gpu] auto mode follows host runs")
    ctx = TransferContext(0, staging_bytes=64 * MiB)
    nb, bpb, n, n_layers = 256, 32768, 64, 4
    kv = nb * bpb
    layers = [Layer(nb, bpb, 2, kv, 2 * kv, 120 + i) for i in range(n_layers)]
    rng = np.random.Generator(np.random.PCG64(12))
    ids = rng.choice(nb, n, replace=False).tolist()
    targets = rng.choice(np.setdiff1d(np.arange(nb), ids), n, replace=False).tolist()
    hosts = []
    try:
        for scattered in (False, True):
            host = PinnedBuffer(n_layers * 2 * n * bpb)
            hosts.append(host)
            ohost = np.zeros(host.nbytes, np.uint8)
            for i, L in enumerate(layers):
                L.place(ids, host, ohost, i * 2 * n * bpb)
            if scattered:  # each layer's K and V chunks in a shuffled order
                for L in layers:
                    perm = rng.permutation(n)
                    L.k, L.ok_ = L.k[perm], L.ok_[perm]
                    L.v, L.ov = L.v[perm], L.ov[perm]
            host.array[:] = 0
            ctx.save_layers([L.transfer(ids) for L in layers], _lib.MODE_AUTO)
            _, dma = ctx.last_stats()
            assert (dma == 0) == scattered, f"save: {dma} DMA copies (scattered={scattered})"
            for L in layers:
                L.oracle_save()
            assert np.array_equal(host.array, ohost)
            ctx.load_layers([L.transfer(targets) for L in layers], _lib.MODE_AUTO)
            ctx.synchronize()
            _, dma = ctx.last_stats()
            assert (dma == 0) == scattered, f"load: {dma} DMA copies (scattered={scattered})"
            for L in layers:
                L.oracle_load(targets)
                assert np.array_equal(L.dev.download(), L.ref)
        # Without staging, AUTO is the kernel mode (the same load again: the
        # targets already hold these bytes).
        plain = TransferContext(0)
        plain.load_layers([L.transfer(targets) for L in layers], _lib.MODE_AUTO)
        plain.synchronize()
        assert plain.last_stats()[1] == 0
        plain.close()
        for L in layers:
            assert np.array_equal(L.dev.download(), L.ref)
    finally:
        for L in layers:
            L.close()
        for h in hosts:
            h.close()
        ctx.close()


def test_copy_engines_known(gpu):
    """The staged mode's copies use one or two copy engines per direction,
    different engines for the two directions (so a save and a load can run
    at once)."""
    d2h, h2d = copy_engines(0)
    say(f"[gpu] copy engines: d2h {d2h:#x}, h2d {h2d:#x}")
    assert d2h and h2d, "no copy engines known for device 0"
    assert bin(d2h).count("1") <= 2 and bin(h2d).count("1") <= 2
    assert d2h & h2d == 0
    # Not the engines hipMemcpyAsync uses on MI355X (engine 0 host to device,
    # engine 1 device to host), and among the fast engines 0-3.
    assert (d2h | h2d) & 0x3 == 0 and (d2h | h2d) & ~0xF == 0


def test_set_copy_engines(gpu):
    """pf_set_copy_engines moves the staged copies to other engines (a staged
    save and load over them stay bit-exact against the oracle); masks of
    more than two engines, or of engines the runtime does not offer, are
    refused; 0 keeps a direction's choice."""
    from pegaflow_amd.runtime import set_copy_engines

    say("[gpu] set copy engines")
    d2h, h2d = copy_engines(0)
    try:
        set_copy_engines(0, 0x1, 0x2)
        assert copy_engines(0) == (0x1, 0x2)
        set_copy_engines(0, 0, 0x8)
        assert copy_engines(0) == (0x1, 0x8)
        with pytest.raises(_lib.PegaFlowError, match="one or two engine bits"):
            set_copy_engines(0, 0x7, 0)
        with pytest.raises(_lib.PegaFlowError, match="available"):
            set_copy_engines(0, 1 << 30, 0)
        layers, save_ids, load_ids = _mixed_layers(90)
        host, ohost = _place_all(layers, save_ids)
        ctx = TransferContext(0, staging_bytes=4 * MiB)
        try:
            ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)],
                            _lib.MODE_STAGED)
            for L in layers:
                L.oracle_save()
            assert np.array_equal(host.array, ohost)
            ctx.load_layers([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                            _lib.MODE_STAGED)
            ctx.synchronize()
            for L, ids in zip(layers, load_ids):
                L.oracle_load(ids)
                assert np.array_equal(L.dev.download(), L.ref)
        finally:
            for L in layers:
                L.close()
            host.close()
            ctx.close()
    finally:
        set_copy_engines(0, d2h, h2d)
    assert copy_engines(0) == (d2h, h2d)


@pytest.mark.parametrize("per_xcd", [1, 4])
def test_cu_masked_context_vs_oracle(gpu, per_xcd):
    """A context whose streams run on `per_xcd` compute units of each XCD:
    kernel and staged saves, and loads with per-layer events and with marks,
    of the mixed layers and of four [2, 512, 16, 8, 128] layers with 200
    random blocks each, equal the oracle byte for byte.  Unmasking the
    context afterwards keeps it working."""
    from pegaflow_amd.transfer import cu_mask_per_xcd

    say(f"[gpu] CU-masked context, {per_xcd} CUs per XCD")
    mask = cu_mask_per_xcd(per_xcd)
    assert sum(bin(w).count("1") for w in mask) == 8 * per_xcd
    ctx = TransferContext(0, staging_bytes=4 * MiB)
    ctx.set_cu_mask(mask)
    mixed, mixed_save, mixed_load = _mixed_layers(110)
    nb, bpb = 512, 32768
    rng = np.random.Generator(np.random.PCG64(per_xcd))
    big = [Layer(nb, bpb, 2, nb * bpb, 2 * nb * bpb, 120 + i) for i in range(4)]
    layers = mixed + big
    save_ids = mixed_save + [rng.choice(nb, 200, replace=False).tolist() for _ in big]
    load_ids = mixed_load + [rng.choice(nb, 200, replace=False).tolist() for _ in big]
    host, ohost = _place_all(layers, save_ids)
    words = PinnedBuffer(8 * len(layers))
    try:
        for rnd, mode in enumerate((_lib.MODE_KERNEL, _lib.MODE_STAGED)):
            if rnd == 1 and per_xcd == 4:
                ctx.set_cu_mask(None)  # the staged round on unmasked streams
            host.array[:] = 0
            ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)], mode)
            ctx.synchronize()
            for L in layers:
                L.oracle_save()
            assert np.array_equal(host.array, ohost), f"mode {mode}: host regions differ"
            evs = [Event() for _ in layers]
            ctx.load_layers([L.transfer(ids) for L, ids in zip(layers, load_ids)], mode,
                            layer_events=evs)
            ctx.synchronize()
            for i, (L, ids) in enumerate(zip(layers, load_ids)):
                L.oracle_load(ids)
                assert np.array_equal(L.dev.download(), L.ref), f"mode {mode}: layer {i} differs"
            words.array[:] = 0
            ctx.load_layers_marked([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                                   [(words.ptr, 5 + rnd, True)], mode)
            ctx.synchronize()
            assert words.array.view(np.uint64).tolist() == [5 + rnd] * len(layers)
            for L in layers:
                assert np.array_equal(L.dev.download(), L.ref)
    finally:
        for L in layers:
            L.close()
        host.close()
        words.close()
        ctx.close()


def test_cu_mask_refusals(gpu, monkeypatch):
    """Masks that would leave an XCD without a compute unit are refused
    before any stream is replaced (the context keeps working); so are 0 CUs
    per XCD and more than the device has.  PEGAFLOW_CUS_PER_XCD masks new
    contexts, and a bad value fails their creation."""
    from pegaflow_amd.transfer import cu_mask_per_xcd

    say("[gpu] CU mask refusals")
    ctx = TransferContext(0, staging_bytes=MiB)
    try:
        with pytest.raises(_lib.PegaFlowError, match="leaves XCD 1 without a compute unit"):
            ctx.set_cu_mask([1, 0, 0, 0, 0, 0, 0, 0])
        with pytest.raises(_lib.PegaFlowError, match="leaves XCD 0 without a compute unit"):
            ctx.set_cu_mask([0xFEFEFEFE] * 8)
        with pytest.raises(_lib.PegaFlowError, match="CUs per XCD"):
            cu_mask_per_xcd(0)
        with pytest.raises(_lib.PegaFlowError, match="CUs per XCD"):
            cu_mask_per_xcd(10_000)
        with pytest.raises(_lib.PegaFlowError, match="fewer than"):
            cu_mask_per_xcd(8, words=1)
        layers, save_ids, load_ids = _mixed_layers(130)
        host, ohost = _place_all(layers, save_ids)
        try:
            ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)],
                            _lib.MODE_KERNEL)
            ctx.synchronize()
            for L in layers:
                L.oracle_save()
            assert np.array_equal(host.array, ohost)
            monkeypatch.setenv("PEGAFLOW_CUS_PER_XCD", "2")
            masked = TransferContext(0, staging_bytes=MiB)
            try:
                masked.load_layers([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                                   _lib.MODE_STAGED)
                masked.synchronize()
                for L, ids in zip(layers, load_ids):
                    L.oracle_load(ids)
                    assert np.array_equal(L.dev.download(), L.ref)
            finally:
                masked.close()
            monkeypatch.setenv("PEGAFLOW_CUS_PER_XCD", "0")
            with pytest.raises(_lib.PegaFlowError, match="CUs per XCD"):
                TransferContext(0, staging_bytes=MiB)
        finally:
            for L in layers:
                L.close()
            host.close()
    finally:
        ctx.close()


def test_marked_slices_mixed_routes_vs_oracle(gpu):
    """A marked staged load whose slices take both marking routes: 16 small
    layers (one slice holds more of them than a scatter can mark itself, so
    they and the large layer whose first piece shares that slice are marked
    by a marking kernel), then large layers spanning several 64 KiB slices
    (each marked by the scatters of its slices, its tile count adding up over
    them; some of those slices also finish the previous layer).  Every
    layer's word is set and every byte equals the oracle; a second load (new
    value, into refilled tensors) marks every layer again: no count is left
    over from the first."""
    say("[gpu] marked staged load: scatter-marked and kernel-marked layers")
    # 256-byte segments throughout, so chunk size never closes a slice:
    # slices of 64 KiB (256 chunks).  Layers 0 and 1 alone (slices growing),
    # layers 2-15 (1 KiB each) with the first 200 chunks of layer 16 in one
    # slice of 15 pieces, then layer 16's 1 MiB over 15 more slices, the
    # last shared with layer 17's start, and likewise for 17 and 18.
    nb, big_nb = 96, 2100
    small = [(nb, 256, 2, nb * 256, 2 * nb * 256) for _ in range(16)]
    big = [(big_nb, 256, 2, big_nb * 256, 2 * big_nb * 256) for _ in range(3)]
    layers = [Layer(*shape, 900 + i) for i, shape in enumerate(small + big)]
    rng = np.random.Generator(np.random.PCG64(91))
    save_ids = [([5, 9] if i < 16 else rng.permutation(big_nb)[:2048].tolist())
                for i in range(len(layers))]
    load_ids = [([1, 2] if i < 16 else rng.permutation(big_nb)[:2048].tolist())
                for i in range(len(layers))]
    host, ohost = _place_all(layers, save_ids)
    ctx = TransferContext(0, staging_bytes=4 * MiB)
    ctx.set_staged_slices(0, 64 * 1024)
    words = PinnedBuffer(8 * len(layers))
    try:
        host.array[:] = 0  # gaps and empty layers' regions are never written
        ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)], _lib.MODE_STAGED)
        ctx.synchronize()
        for L in layers:
            L.oracle_save()
        assert np.array_equal(host.array, ohost), "host regions differ from the oracle"
        for value in (21, 22):
            for i, (L, ids) in enumerate(zip(layers, load_ids)):
                L.dev.fill_random(value * 100 + i)
                L.ref[:] = L.dev.download()  # in place: the oracle's layout points here
                L.oracle_load(ids)
            words.array[:] = 0
            ctx.load_layers_marked([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                                   [(words.ptr, value, True)], _lib.MODE_STAGED)
            ctx.synchronize()
            assert words.array.view(np.uint64).tolist() == [value] * len(layers)
            for i, L in enumerate(layers):
                assert np.array_equal(L.dev.download(), L.ref), f"load {value}: layer {i}"
    finally:
        for L in layers:
            L.close()
        host.close()
        words.close()
        ctx.close()


def _fuzz_layers(rng, seed):
    """1-20 layers of random kinds: split K/V of 16-byte aligned segments (the
    common case), blocks-first single segments, padded K/V gaps, overlapping
    K/V (copied in place, in list order) and unaligned segments; random save
    and load ids (some layers empty)."""
    specs = []
    for _ in range(int(rng.integers(1, 21))):
        nb = int(rng.integers(4, 64))
        kind = rng.choice(["split", "split", "split", "single", "padded", "overlap", "unaligned"])
        if kind == "unaligned":
            bpb = int(rng.choice([24, 40, 72]))
        else:
            bpb = int(rng.choice([64, 256, 1024, 4096, 8192]))
        if kind == "single":
            shape = (nb, bpb, 1, 0, nb * bpb)
        elif kind == "padded":
            kv = nb * bpb + 16 * int(rng.integers(1, 9))
            shape = (nb, bpb, 2, kv, kv + nb * bpb)
        elif kind == "overlap":
            kv = (nb * bpb) // 2
            shape = (nb, bpb, 2, kv, kv + nb * bpb)
        else:
            shape = (nb, bpb, 2, nb * bpb, 2 * nb * bpb)
        m = 0 if rng.random() < 0.1 else int(rng.integers(1, nb + 1))
        save = rng.choice(nb, m, replace=False).tolist()
        load = rng.choice(nb, m, replace=False).tolist()
        specs.append((shape, save, load))
    layers = [Layer(*shape, seed * 100 + i) for i, (shape, _, _) in enumerate(specs)]
    return layers, [s for _, s, _ in specs], [l for _, _, l in specs]


@pytest.mark.parametrize("mode", ["staged", "kernel", "auto"])
@pytest.mark.parametrize("seed", range(8))
def test_staged_marked_fuzz_vs_oracle(gpu, seed, mode):
    """Seeded random calls with per-layer marks: random layers (see
    _fuzz_layers) with random load slice caps from one chunk to 256 KiB.  In
    the staged mode slices hold many layers, parts of layers, or a chunk
    each, and their scatters mark layers themselves, across slices, or leave
    them to the marking kernel; the kernel mode marks from inside its
    launches; AUTO picks either per call.  After a save in the same mode,
    two marked loads (into refilled tensors) must set every layer's word and
    leave every byte as the oracle does."""
    rng = np.random.Generator(np.random.PCG64(4000 + seed))
    layers, save_ids, load_ids = _fuzz_layers(rng, seed)
    cap = int(rng.choice([1, 512, 4096, 16 * 1024, 64 * 1024, 256 * 1024]))
    say(f"[gpu] marked fuzz seed={seed} mode={mode}: {len(layers)} layers, load slice cap {cap}")
    m = _lib.MODE_NAMES[mode]
    host, ohost = _place_all(layers, save_ids, gap=16 * int(rng.integers(0, 3)))
    ctx = TransferContext(0, staging_bytes=4 * MiB)
    ctx.set_staged_slices(0, cap)
    words = PinnedBuffer(8 * len(layers))
    try:
        host.array[:] = 0  # gaps and empty layers' regions are never written
        ctx.save_layers([L.transfer(ids) for L, ids in zip(layers, save_ids)], m)
        ctx.synchronize()
        for L in layers:
            L.oracle_save()
        assert np.array_equal(host.array, ohost), "host regions differ from the oracle"
        for value in (31, 32):
            for i, (L, ids) in enumerate(zip(layers, load_ids)):
                L.dev.fill_random(seed * 1000 + value * 50 + i)
                L.ref[:] = L.dev.download()  # in place: the oracle's layout points here
                L.oracle_load(ids)
            words.array[:] = 0
            ctx.load_layers_marked([L.transfer(ids) for L, ids in zip(layers, load_ids)],
                                   [(words.ptr, value, True)], m)
            ctx.synchronize()
            assert words.array.view(np.uint64).tolist() == [value] * len(layers)
            for i, L in enumerate(layers):
                assert np.array_equal(L.dev.download(), L.ref), f"load {value}: layer {i}"
    finally:
        for L in layers:
            L.close()
        host.close()
        words.close()
        ctx.close()
