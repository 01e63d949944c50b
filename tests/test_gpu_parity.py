"""GPU parity of the HIP transfer path against the oracle and golden data.

Every test runs the product path (libpegaflow_hip.so through its C ABI) on
device 0 and compares bytes:
  * small shapes: against the CPU oracle on the same seeded inputs, and
    against the committed golden fixtures;
  * full workload shapes (Llama-3.1-8B prefix, its TP=8 rank, MLA
    latent): through size-independent closed forms — each host chunk
    and every block of every layer tensor must hold exactly the
    splitmix64 words of the block it came from (a permutation identity plus
    "untouched blocks unchanged"), checked on the device.
All four transfer modes must give identical bytes.
"""

import hashlib
import json
import os
import sys

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.runtime import (DeviceBuffer, Event, PinnedBuffer, Stream, memcpy_async, spin,
                                  verify_random_chunks)
from pegaflow_amd.transfer import (KVCacheRegistration, LayerTransfer, TransferContext,
                                   block_array)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODES = {"dma_reference": _lib.MODE_DMA_REFERENCE, "dma_batched": _lib.MODE_DMA_BATCHED,
         "kernel": _lib.MODE_KERNEL, "staged": _lib.MODE_STAGED}
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx(gpu):
    c = TransferContext(0, staging_bytes=64 * MiB)
    yield c
    c.close()


class Layers:
    """Device layer tensors of one shape, filled with seeded random words."""

    def __init__(self, n_layers, num_blocks, bpb, segments, base_seed, pad_blocks=0):
        self.nb, self.bpb, self.segments = num_blocks, bpb, segments
        self.kv = (num_blocks + pad_blocks) * bpb if segments == 2 else 0
        self.size = (self.kv + num_blocks * bpb) if segments == 2 else num_blocks * bpb
        self.seeds = [oracle.layer_seed(base_seed, l) for l in range(n_layers)]
        self.bufs = []
        for l in range(n_layers):
            b = DeviceBuffer(self.size)
            b.fill_random(self.seeds[l])
            self.bufs.append(b)
        self.regs = [KVCacheRegistration.create(b.ptr, self.size, num_blocks, bpb, self.kv,
                                                segments) for b in self.bufs]

    def close(self):
        for b in self.bufs:
            b.close()
        self.bufs = []


def save_transfers(layers: Layers, ids, host: PinnedBuffer, region_stride=None):
    """Reference host layout (lib.rs:636-747): per layer a K region then a V
    region (split), or one region of whole blocks; returns per-layer bases."""
    n = len(ids)
    bs = layers.bpb * layers.segments
    per_layer = n * bs if region_stride is None else region_stride
    out, bases = [], []
    for l, reg in enumerate(layers.regs):
        base = host.ptr + l * per_layer
        k, v, split = oracle.save_host_layout(oracle.layout(0, reg.size_bytes, reg.num_blocks,
                                                            reg.bytes_per_block,
                                                            reg.kv_stride_bytes, reg.segments),
                                              n, base, base + n * layers.bpb)
        out.append(LayerTransfer(reg, block_array(ids, k, v if split else None)))
        bases.append(base)
    return out, bases


def load_transfers(layers: Layers, targets, saved):
    out = []
    for reg, lt in zip(layers.regs, saved):
        b = lt.blocks.copy()
        b["block_idx"] = np.asarray(targets, np.int64)
        out.append(LayerTransfer(reg, b))
    return out


def closed_form_host_check(layers: Layers, ids, saved):
    """Host chunk j of layer l holds the words of block ids[j] (per segment)."""
    bad = 0
    for l, lt in enumerate(saved):
        addrs, offs = [], []
        for j, b in enumerate(ids):
            if layers.segments == 2 and layers.kv > layers.bpb:
                addrs += [int(lt.blocks["k_host"][j]), int(lt.blocks["v_host"][j])]
                offs += [b * layers.bpb // 8, (layers.kv + b * layers.bpb) // 8]
            else:
                addrs.append(int(lt.blocks["k_host"][j]))
                offs.append(b * layers.bpb * layers.segments // 8)
        chunk = layers.bpb if layers.segments == 2 else layers.bpb * layers.segments
        bad += verify_random_chunks(addrs, offs, chunk, layers.seeds[l])
    return bad


def closed_form_tensor_check(layers: Layers, src_of: dict):
    """Every block b of every layer holds the words of block src_of.get(b, b)."""
    bad = 0
    nb, bpb = layers.nb, layers.bpb
    blocks = np.arange(nb, dtype=np.uint64)
    src = blocks.copy()
    for b, s in src_of.items():
        src[b] = s
    for l, buf in enumerate(layers.bufs):
        if layers.segments == 2:
            addrs = np.concatenate([buf.ptr + blocks * bpb, buf.ptr + layers.kv + blocks * bpb])
            offs = np.concatenate([src * bpb // 8, (layers.kv + src * bpb) // 8])
        else:
            addrs = buf.ptr + blocks * bpb
            offs = src * bpb // 8
        bad += verify_random_chunks(addrs, offs, bpb, layers.seeds[l])
    return bad


# ---------------------------------------------------------------------------
def test_fill_kernel_matches_oracle_words(gpu):
    buf = DeviceBuffer(1 << 16)
    buf.fill_random(987654321, word_offset=5)
    got = buf.download().view(np.uint64)
    assert np.array_equal(got, oracle.random_words(len(got), 987654321, 5))
    assert verify_random_chunks([buf.ptr], [5], 1 << 16, 987654321) == 0
    assert verify_random_chunks([buf.ptr + 8], [5], 64, 987654321) == 8  # shifted: all differ
    buf.close()


@pytest.mark.parametrize("fixture", ["tiny_kvfirst", "tiny_blocks"])
@pytest.mark.parametrize("mode", list(MODES))
def test_golden_tiny(ctx, fixture, mode):
    say(f"[gpu] golden {fixture} mode={mode}")
    f = np.load(os.path.join(GOLDEN, fixture + ".npz"))
    nb, bpb, kv, segs = (int(f[k]) for k in ("num_blocks", "bytes_per_block",
                                             "kv_stride_bytes", "segments"))
    size = int(f["size_bytes"])
    kept = [int(b) for b in f["save_ids"] if b >= 0]
    targets = [int(b) for b in f["load_ids"] if b >= 0]
    host = PinnedBuffer(1 << 16)
    for layer in range(2):
        dev = DeviceBuffer(size)
        dev.upload(f[f"input_{layer}"])
        reg = KVCacheRegistration.create(dev.ptr, size, nb, bpb, kv, segs)
        k, v, split = oracle.save_host_layout(
            oracle.layout(0, size, nb, bpb, kv, segs), len(kept), host.ptr,
            host.ptr + len(kept) * bpb)
        lt = LayerTransfer(reg, block_array(kept, k, v if split else None))
        host.array[:] = 0
        ctx.save_layers([lt], MODES[mode])
        m = len(kept)
        if split:
            assert np.array_equal(host.array[: m * bpb], f[f"host_k_{layer}"])
            assert np.array_equal(host.array[m * bpb: 2 * m * bpb], f[f"host_v_{layer}"])
        else:
            assert np.array_equal(host.array[: m * bpb * segs], f[f"host_{layer}"])
        lt2 = LayerTransfer(reg, block_array(targets, k, v if split else None))
        ctx.load_layers([lt2], MODES[mode])
        ctx.synchronize()
        assert np.array_equal(dev.download(), f[f"restored_{layer}"])
        dev.close()
    host.close()


@pytest.mark.parametrize("mode", list(MODES))
def test_gpt2_config1_golden(ctx, mode):
    """Config 1: GPT-2 shape, 12 fp16 layers [2,512,16,12,64]; 64 random
    blocks saved, loaded into 64 other random blocks; digests must match."""
    with open(os.path.join(GOLDEN, "gpt2_config1.json")) as fh:
        g = json.load(fh)
    say(f"[gpu] gpt2 config1 mode={mode}")
    layers = Layers(g["layers"], g["num_blocks"], g["bytes_per_block"], 2, g["base_seed"])
    assert layers.size == g["size_bytes"]
    n = len(g["save_ids"])
    host = PinnedBuffer(g["layers"] * 2 * n * g["bytes_per_block"])
    saved, bases = save_transfers(layers, g["save_ids"], host)
    ctx.save_layers(saved, MODES[mode])
    seg = n * g["bytes_per_block"]
    for l, base in enumerate(bases):
        off = base - host.ptr
        assert hashlib.sha256(host.array[off: off + seg].tobytes()).hexdigest() == \
            g["host_k_sha256"][l]
        assert hashlib.sha256(host.array[off + seg: off + 2 * seg].tobytes()).hexdigest() == \
            g["host_v_sha256"][l]
    ctx.load_layers(load_transfers(layers, g["load_ids"], saved), MODES[mode])
    ctx.synchronize()
    for l, buf in enumerate(layers.bufs):
        assert hashlib.sha256(buf.download().tobytes()).hexdigest() == g["restored_sha256"][l]
    layers.close()
    host.close()


def _oracle_roundtrip_case(ctx, mode, nb, bpb, segs, kv, size, save_ids, load_ids,
                           host_offset=0, seed=3, load_error=None):
    """Runs save(save_ids) then load(load_ids) on device and on the oracle.
    With ``load_error`` (a message pattern) the load must fail with it on
    both, leaving the device bytes as they were."""
    dev = DeviceBuffer(size)
    dev.fill_random(seed)
    ref = dev.download()
    reg = KVCacheRegistration.create(dev.ptr, size, nb, bpb, kv, segs)
    oreg = oracle.layout(ref.ctypes.data, size, nb, bpb, kv, segs)
    m = len(save_ids)
    bs = bpb * segs
    host = PinnedBuffer(2 * m * bs + 4096)
    base = host.ptr + host_offset
    k, v, split = oracle.save_host_layout(oreg, m, base, base + m * bpb)
    host.array[:] = 0
    ctx.save_layers([LayerTransfer(reg, block_array(save_ids, k, v if split else None))], mode)
    got_host = host.array.copy()
    # Oracle on the CPU copy, with host buffers at the same relative offsets.
    ohost = np.zeros_like(got_host)
    obase = ohost.ctypes.data + host_offset
    ok_, ov, _ = oracle.save_host_layout(oreg, m, obase, obase + m * bpb)
    oracle.process_save(oreg, ref, save_ids, ok_, ov if split else None)
    assert np.array_equal(got_host, ohost)
    if load_error is not None:
        with pytest.raises(_lib.PegaFlowError, match=load_error):
            ctx.load_layers([LayerTransfer(reg, block_array(load_ids, k, v if split else None))],
                            mode)
        ctx.synchronize()
        with pytest.raises(oracle.OracleError, match=load_error):
            oracle.process_load(oreg, ref, load_ids, ok_, ov if split else None)
        assert np.array_equal(dev.download(), ref)
        dev.close()
        host.close()
        return
    ctx.load_layers([LayerTransfer(reg, block_array(load_ids, k, v if split else None))], mode)
    ctx.synchronize()
    oracle.process_load(oreg, ref, load_ids, ok_, ov if split else None)
    assert np.array_equal(dev.download(), ref)
    dev.close()
    host.close()


@pytest.mark.parametrize("mode", list(MODES))
def test_edge_cases_vs_oracle(ctx, mode):
    m = MODES[mode]
    say(f"[gpu] edge cases mode={mode}")
    nb, bpb = 40, 256
    kv = nb * bpb
    # Every block, in reverse order, loaded in sorted order (maximal merging).
    _oracle_roundtrip_case(ctx, m, nb, bpb, 2, kv, 2 * kv, list(range(nb))[::-1],
                           list(range(nb)))
    # One block.
    _oracle_roundtrip_case(ctx, m, nb, bpb, 2, kv, 2 * kv, [7], [39])
    # Duplicate load targets: the later copy wins (in-order semantics).
    _oracle_roundtrip_case(ctx, m, nb, bpb, 2, kv, 2 * kv, [1, 2, 3, 4], [9, 9, 5, 9])
    # Host regions at an 8-byte (not 16-byte) offset: unaligned kernel path.
    _oracle_roundtrip_case(ctx, m, nb, bpb, 2, kv, 2 * kv, [3, 11, 20], [0, 1, 2],
                           host_offset=8)
    # Odd segment size (not a multiple of 16).
    _oracle_roundtrip_case(ctx, m, 30, 24, 2, 30 * 24 + 8, 30 * 24 * 2 + 8, [4, 5, 6],
                           [20, 0, 29])
    # Padded split layout (gap between K and V), blocks-first single segment.
    _oracle_roundtrip_case(ctx, m, nb, bpb, 2, kv + 3 * bpb, 2 * kv + 3 * bpb, [5, 6], [0, 39])
    _oracle_roundtrip_case(ctx, m, nb, 4608, 1, 0, nb * 4608, [9, 1, 30], [2, 3, 4])
    # Overlapping split layout (kv_stride < num_blocks * bytes_per_block) and a
    # strided layout (kv_stride < bytes_per_block): in-order semantics.
    _oracle_roundtrip_case(ctx, m, 10, 64, 2, 160, 160 + 640, [1, 2, 3], [4, 3, 2])
    _oracle_roundtrip_case(ctx, m, 10, 64, 2, 32, 9 * 64 + 32 + 64, [2, 5], [3, 4])


def _random_case(rng):
    """A random layer layout of every kind validation accepts (split,
    padded split, overlapping split, strided, contiguous two-segment,
    blocks-first), random save ids and load ids with repeats."""
    nb = int(rng.integers(1, 120))
    bpb = int(rng.choice([16, 24, 48, 256, 4096, 32768]))
    kind = rng.choice(["split", "padded", "overlap", "strided", "contig2", "single"])
    if kind == "single":
        segs, kv, size = 1, 0, nb * bpb
    elif kind == "contig2":
        segs, kv, size = 2, bpb, (nb + 1) * bpb
    elif kind == "strided":
        # The smallest size validation accepts, or room for whole blocks.
        segs, kv = 2, max(8, (bpb // 2) // 8 * 8)
        size = (nb - 1) * bpb + kv + bpb if rng.integers(2) else (nb + 1) * bpb
    elif kind == "overlap":
        segs, kv = 2, max(bpb, (nb * bpb // 2) // 8 * 8)
        size = kv + nb * bpb
    else:
        segs, kv = 2, nb * bpb + (int(rng.integers(1, 4)) * bpb if kind == "padded" else 0)
        size = kv + nb * bpb
    m = int(rng.integers(1, nb + 1))
    save_ids = rng.choice(nb, m, replace=False).tolist()
    load_ids = rng.choice(nb, m, replace=True).tolist()
    return kind, nb, bpb, segs, kv, size, save_ids, load_ids


@pytest.mark.parametrize("seed", range(12))
def test_random_layouts_vs_oracle(ctx, seed):
    """Seeded random layouts, ids and host offsets, every mode: the device
    bytes and the host regions equal the oracle's after save then load.  A
    whole-block load of a strided layout's last block at the smallest valid
    size would write past the tensor: both refuse it."""
    rng = np.random.Generator(np.random.PCG64(1000 + seed))
    for case in range(4):
        kind, nb, bpb, segs, kv, size, save_ids, load_ids = _random_case(rng)
        off = int(rng.choice([0, 8, 16, 4096]))
        past = kind == "strided" and any((b + 2) * bpb > size for b in load_ids)
        err = f"Block {max(load_ids)} exceeds registered memory" if past else None
        for name, m in MODES.items():
            say(f"[gpu] random seed={seed} case={case} {kind} nb={nb} bpb={bpb} kv={kv} "
                f"size={size} m={len(save_ids)} off={off} mode={name} error={past}")
            _oracle_roundtrip_case(ctx, m, nb, bpb, segs, kv, size, save_ids, load_ids,
                                   host_offset=off, seed=seed * 10 + case, load_error=err)


def test_pipelined_multi_layer_calls_vs_oracle(ctx):
    """Calls of at least 8 layers and 16384 chunks are issued in two parts
    (the first layers launched before the rest are planned).  16 layers of
    1024 blocks, one with overlapping K/V regions (copied in list order),
    loads naming blocks more than once (the later copy wins): every byte
    against the oracle.  A planning error in the second part fails the call
    with the reference's message and leaves nothing in flight."""
    say("[gpu] pipelined multi-layer calls vs oracle")
    L, nb, bpb, m = 16, 1100, 256, 1024
    rng = np.random.Generator(np.random.PCG64(11))
    host = PinnedBuffer(L * 2 * m * bpb)
    ohost = np.zeros(L * 2 * m * bpb, np.uint8)
    devs, refs, regs, oregs, saves, loads, osaves = [], [], [], [], [], [], []
    for l in range(L):
        kv = nb * bpb // 2 if l == 5 else nb * bpb
        size = kv + nb * bpb
        dev = DeviceBuffer(size)
        dev.fill_random(100 + l)
        ref = dev.download()
        reg = KVCacheRegistration.create(dev.ptr, size, nb, bpb, kv, 2)
        oreg = oracle.layout(ref.ctypes.data, size, nb, bpb, kv, 2)
        save_ids = rng.choice(nb, m, replace=False).tolist()
        load_ids = rng.choice(nb, m, replace=True).tolist()
        base, obase = host.ptr + l * 2 * m * bpb, ohost.ctypes.data + l * 2 * m * bpb
        k, v, split = oracle.save_host_layout(oreg, m, base, base + m * bpb)
        ok_, ov, _ = oracle.save_host_layout(oreg, m, obase, obase + m * bpb)
        saves.append(LayerTransfer(reg, block_array(save_ids, k, v if split else None)))
        loads.append(LayerTransfer(reg, block_array(load_ids, k, v if split else None)))
        osaves.append((oreg, ref, save_ids, load_ids, ok_, ov if split else None))
        devs.append(dev)
    host.array[:] = 0
    ctx.save_layers(saves, _lib.MODE_KERNEL)
    for oreg, ref, save_ids, _, ok_, ov in osaves:
        oracle.process_save(oreg, ref, save_ids, ok_, ov)
    assert np.array_equal(host.array, ohost)
    ctx.load_layers(loads, _lib.MODE_KERNEL)
    ctx.synchronize()
    for dev, (oreg, ref, _, load_ids, ok_, ov) in zip(devs, osaves):
        oracle.process_load(oreg, ref, load_ids, ok_, ov)
        assert np.array_equal(dev.download(), ref)
    # Three pipelined loads back to back, without waiting in between: each
    # call's descriptors must not be overwritten while an earlier call's
    # copies still read them.
    loads2, ids2 = [], []
    for lt in loads:
        b = lt.blocks.copy()
        ids = rng.choice(nb, m, replace=True)
        b["block_idx"] = ids
        loads2.append(LayerTransfer(lt.registration, b))
        ids2.append(ids.tolist())
    for batch in (loads, loads2, loads):
        ctx.load_layers(batch, _lib.MODE_KERNEL)
    ctx.synchronize()
    for l, (dev, (oreg, ref, _, load_ids, ok_, ov)) in enumerate(zip(devs, osaves)):
        for ids in (load_ids, ids2[l], load_ids):
            oracle.process_load(oreg, ref, ids, ok_, ov)
        assert np.array_equal(dev.download(), ref)
    # An out-of-range block in the last layer: found after the first part
    # was launched.
    bad = list(loads)
    b = bad[-1].blocks.copy()
    b["block_idx"][7] = nb
    bad[-1] = LayerTransfer(bad[-1].registration, b)
    for fn in (ctx.load_layers, ctx.save_layers):
        with pytest.raises(_lib.PegaFlowError, match="exceeds registered memory"):
            fn(bad, _lib.MODE_KERNEL)
        ctx.stream.synchronize()
    ctx.load_layers(loads, _lib.MODE_KERNEL)
    ctx.synchronize()
    for dev, (_, ref, _, _, _, _) in zip(devs, osaves):
        assert np.array_equal(dev.download(), ref)
    for dev in devs:
        dev.close()
    host.close()


def test_empty_and_errors(ctx, gpu):
    say("[gpu] empty and error paths")
    nb, bpb = 16, 512
    dev = DeviceBuffer(2 * nb * bpb)
    reg = KVCacheRegistration.create(dev.ptr, 2 * nb * bpb, nb, bpb, nb * bpb, 2)
    host = PinnedBuffer(1 << 16)
    for m in MODES.values():
        ctx.save_layers([], m)
        ctx.save_layers([LayerTransfer(reg, block_array([], []))], m)
        ctx.load_layers([LayerTransfer(reg, block_array([], []))], m)
    ctx.synchronize()
    # Out-of-range block: the reference's segment_offset message, before any copy.
    with pytest.raises(_lib.PegaFlowError, match="exceeds registered memory"):
        ctx.save_layers([LayerTransfer(reg, block_array([nb], [host.ptr]))], _lib.MODE_KERNEL)
    with pytest.raises(_lib.PegaFlowError, match="must be >= 0"):
        ctx.load_layers([LayerTransfer(reg, block_array([-1], [host.ptr]))], _lib.MODE_KERNEL)
    # Kernel mode refuses host memory that is not mapped for the device.
    pageable = np.zeros(4 * bpb, np.uint8)
    with pytest.raises(_lib.PegaFlowError, match="not device-accessible"):
        ctx.save_layers([LayerTransfer(reg, block_array([0], [pageable.ctypes.data]))],
                        _lib.MODE_KERNEL)
    # ...and a "layer tensor" that is not device memory.
    bad = KVCacheRegistration(data_ptr=pageable.ctypes.data, size_bytes=4 * bpb, num_blocks=2,
                              bytes_per_block=bpb, block_size_bytes=2 * bpb,
                              kv_stride_bytes=2 * bpb, segments=2)
    with pytest.raises(_lib.PegaFlowError, match="not inside one device allocation"):
        ctx.save_layers([LayerTransfer(bad, block_array([0], [host.ptr]))], _lib.MODE_KERNEL)
    # DMA modes accept pageable host memory, like cuMemcpy.
    dev.fill_random(5)
    ctx.save_layers([LayerTransfer(reg, block_array([3], [pageable.ctypes.data]))],
                    _lib.MODE_DMA_BATCHED)
    expect = oracle.random_words(bpb // 8, 5, 3 * bpb // 8).view(np.uint8)
    assert np.array_equal(pageable[:bpb], expect)
    # A staged transfer on a context without staging is an error.
    nostage = TransferContext(0, staging_bytes=0)
    with pytest.raises(_lib.PegaFlowError, match="no staging buffer"):
        nostage.save_layers([LayerTransfer(reg, block_array([0], [host.ptr]))],
                            _lib.MODE_STAGED)
    nostage.close()
    dev.close()
    host.close()


@pytest.mark.parametrize("shape", [(256, 1), (256, 2), (256, 4), (512, 8), (1024, 16),
                                   (64, 8)])
def test_kernel_shapes_and_nontemporal(ctx, shape):
    threads, unroll = shape
    say(f"[gpu] kernel shape threads={threads} unroll={unroll}")
    for nt in (0, _lib.KERNEL_NT_LOADS, _lib.KERNEL_NT_STORES, _lib.KERNEL_NONTEMPORAL):
        ctx.set_kernel_shape(threads, unroll | nt)
        _oracle_roundtrip_case(ctx, _lib.MODE_KERNEL, 64, 73728, 1, 0, 64 * 73728,
                               [5, 60, 2, 33], [0, 1, 63, 9], seed=threads + unroll)
        # Segments that end in a partial tile of every shape.
        _oracle_roundtrip_case(ctx, _lib.MODE_KERNEL, 20, 16 * 1000, 2, 20 * 16000,
                               40 * 16000, [3, 19, 0], [5, 6, 7], seed=nt + 1)
    ctx.reset_kernel_shape()
    ctx.set_max_grid(0)


@pytest.mark.parametrize("shape", [(512, 1), (256, 2), (64, 1)])
def test_xcd_major_tile_order(ctx, shape):
    threads, unroll = shape
    say(f"[gpu] xcd-major tile order threads={threads} unroll={unroll}")
    ctx.set_kernel_shape(threads, unroll | _lib.KERNEL_NONTEMPORAL | _lib.KERNEL_XCD_MAJOR)
    # Tile counts that are and are not multiples of 8.
    for nb, n in ((64, 13), (64, 64), (40, 7)):
        _oracle_roundtrip_case(ctx, _lib.MODE_KERNEL, nb, 32768, 2, nb * 32768, 2 * nb * 32768,
                               list(range(n)), list(range(nb - 1, nb - 1 - n, -1)), seed=n)
    ctx.reset_kernel_shape()


def test_capped_grid_loops_over_tiles(ctx):
    """A grid cap makes the fixed-map kernel loop over tiles (device routes:
    the staged mode's gather and scatter) and shrinks the queued kernel's
    persistent grid (host routes)."""
    say("[gpu] capped grid")
    for mode in (_lib.MODE_KERNEL, _lib.MODE_STAGED):
        for grid in (1, 7, 256):
            ctx.set_max_grid(grid)
            _oracle_roundtrip_case(ctx, mode, 64, 32768, 2, 64 * 32768, 128 * 32768,
                                   list(range(0, 64, 3)), list(range(63, -1, -3)),
                                   seed=grid + mode)
    ctx.set_max_grid(0)


@pytest.mark.parametrize("grid", [0, 1, 3, 32, 64, 5000])
def test_queued_host_routes(ctx, grid):
    """Work distribution over the host link: 0 = one workgroup per tile with
    the hardware's deal; N = N persistent workgroups pulling tiles from the
    queue, including a single workgroup and more workgroups than tiles.  The
    queue counter carries over from launch to launch, so several calls and
    several launches per call (layers of different chunk sizes) must all
    copy every tile exactly once."""
    say(f"[gpu] queued host routes grid={grid}")
    ctx.set_route_grid(_lib.ROUTE_SAVE_HOST, grid)
    ctx.set_route_grid(_lib.ROUTE_LOAD_HOST, grid)
    try:
        for rep in range(2):
            _oracle_roundtrip_case(ctx, _lib.MODE_KERNEL, 64, 32768, 2, 64 * 32768, 128 * 32768,
                                   list(range(0, 64, 3)), list(range(63, -1, -3)),
                                   seed=grid + rep)
            _oracle_roundtrip_case(ctx, _lib.MODE_KERNEL, 20, 16 * 1000, 2, 20 * 16000,
                                   40 * 16000, [3, 19, 0], [5, 6, 7], seed=grid + 7)
            _oracle_roundtrip_case(ctx, _lib.MODE_KERNEL, 64, 73728, 1, 0, 64 * 73728,
                                   [5, 60, 2, 33], [0, 1, 63, 9], seed=grid + 9)
        if grid:
            # Device routes queued too (the staged mode's gather and scatter).
            ctx.set_route_grid(_lib.ROUTE_SAVE_DEVICE, grid)
            ctx.set_route_grid(_lib.ROUTE_LOAD_DEVICE, grid)
            _oracle_roundtrip_case(ctx, _lib.MODE_STAGED, 64, 32768, 2, 64 * 32768,
                                   128 * 32768, list(range(0, 64, 5)), list(range(63, 0, -5)),
                                   seed=grid + 11)
    finally:
        ctx.reset_kernel_shape()


def _full_size(ctx, n_layers, nb, bpb, segs, n_blocks, save_mode, load_mode, seed=0):
    layers = Layers(n_layers, nb, bpb, segs, seed)
    rng = np.random.Generator(np.random.PCG64(seed))
    ids = rng.choice(nb, n_blocks, replace=False)
    rest = np.setdiff1d(np.arange(nb), ids)
    targets = rng.choice(rest, n_blocks, replace=False)
    host = PinnedBuffer(n_layers * n_blocks * bpb * segs)
    saved, _ = save_transfers(layers, ids.tolist(), host)
    ctx.save_layers(saved, save_mode)
    assert closed_form_host_check(layers, ids.tolist(), saved) == 0
    ctx.load_layers(load_transfers(layers, targets, saved), load_mode)
    ctx.synchronize()
    src_of = {int(t): int(s) for t, s in zip(targets, ids)}
    assert closed_form_tensor_check(layers, src_of) == 0
    layers.close()
    host.close()


@pytest.mark.parametrize("save_mode,load_mode", [("kernel", "kernel"), ("kernel", "staged"),
                                                  ("staged", "kernel"), ("auto", "auto"),
                                                  ("dma_batched", "dma_batched")])
def test_llama_10k_prefix_full_size(ctx, save_mode, load_mode):
    """Config 2: 32 bf16 layers [2,20000,16,8,128], 640 random blocks; the
    bench's own pairing (zero-copy save, zero-copy restore) first."""
    say(f"[gpu] llama full size save={save_mode} load={load_mode}")
    _full_size(ctx, 32, 20000, 32768, 2, 640, _lib.MODE_NAMES[save_mode],
               _lib.MODE_NAMES[load_mode])


@pytest.mark.parametrize("save_mode,load_mode", [("kernel", "kernel"), ("staged", "dma_batched")])
def test_llama_tp8_rank_full_size(ctx, save_mode, load_mode):
    """One TP=8 rank of Llama-3.1-8B: 32 layers [2,20000,16,1,128] (4 KiB
    segments), 640 random blocks."""
    say(f"[gpu] llama tp8 rank full size save={save_mode} load={load_mode}")
    _full_size(ctx, 32, 20000, 4096, 2, 640, MODES[save_mode], MODES[load_mode], seed=8)


@pytest.mark.parametrize("dtype_bytes", [2, 1])
def test_mla_latent_full_size(ctx, dtype_bytes):
    """Config 5: 61 layers [8192, 64, 576] (bf16 or fp8 bytes), 128 blocks."""
    say(f"[gpu] MLA full size dtype_bytes={dtype_bytes}")
    _full_size(ctx, 61, 8192, 64 * 576 * dtype_bytes, 1, 128, _lib.MODE_KERNEL,
               _lib.MODE_KERNEL, seed=dtype_bytes)


def test_layerwise_load_events_qwen3(ctx):
    """Config 3 shape: 36 layers [2,16000,16,8,128], 313 blocks, loaded one
    layer at a time; each layer's event gates a compute kernel on a second
    stream.  Events complete in layer order and the bytes are exact."""
    say("[gpu] qwen3 layer-wise events")
    n_layers, nb, bpb, n = 36, 16000, 32768, 313
    layers = Layers(n_layers, nb, bpb, 2, 9)
    rng = np.random.Generator(np.random.PCG64(9))
    ids = rng.choice(nb, n, replace=False)
    targets = rng.choice(np.setdiff1d(np.arange(nb), ids), n, replace=False)
    host = PinnedBuffer(n_layers * n * bpb * 2)
    saved, _ = save_transfers(layers, ids.tolist(), host)
    ctx.save_layers(saved, _lib.MODE_KERNEL)
    compute = Stream()
    # Layer l is copied on the compute stream right after its wait: an event
    # recorded for the wrong layer, or before its layer's copy, leaves a
    # snapshot without all of its restored blocks.
    snaps = [DeviceBuffer(layers.size) for _ in range(n_layers)]
    bpb, kv = layers.bpb, layers.kv
    for mode in (_lib.MODE_KERNEL, _lib.MODE_STAGED, _lib.MODE_DMA_BATCHED):
        evs = [Event() for _ in range(n_layers)]
        done = [Event() for _ in range(n_layers)]
        ctx.load_layers(load_transfers(layers, targets, saved), mode, layer_events=evs)
        for l in range(n_layers):
            compute.wait_event(evs[l])
            memcpy_async(snaps[l].ptr, layers.bufs[l].ptr, layers.size, compute)
            spin(compute, 50)
            done[l].record(compute)
        compute.synchronize()
        ctx.synchronize()
        for l in range(1, n_layers):
            assert evs[l - 1].elapsed_ms(evs[l]) >= 0.0
        t64, s64 = targets.astype(np.uint64), ids.astype(np.uint64)
        for l in range(n_layers):
            addrs = np.concatenate([snaps[l].ptr + t64 * bpb, snaps[l].ptr + kv + t64 * bpb])
            offs = np.concatenate([s64 * bpb // 8, (kv + s64 * bpb) // 8])
            assert verify_random_chunks(addrs, offs, bpb, layers.seeds[l]) == 0, \
                f"mode {mode}: layer {l}'s snapshot after its event misses restored bytes"
        src_of = {int(t): int(s) for t, s in zip(targets, ids)}
        assert closed_form_tensor_check(layers, src_of) == 0
        for l in range(n_layers):  # restore the targets for the next mode
            layers.bufs[l].fill_random(layers.seeds[l])
    for b in snaps:
        b.close()
    compute.close()
    layers.close()
    host.close()


def test_scatter_shape_chosen_on_evidence(ctx):
    """The scatter route times its two candidate shapes on a context's first
    scatters of at least 64 MiB (two each) and keeps the faster: every call's
    bytes are exact whichever shape ran, the choice is made after the trials,
    an explicit shape ends it and the defaults start it again."""
    say("[gpu] scatter shape chosen on evidence")
    n_layers, nb, bpb, n = 8, 4000, 32768, 640
    layers = Layers(n_layers, nb, bpb, 2, 21)
    rng = np.random.Generator(np.random.PCG64(21))
    ids = rng.choice(nb, n, replace=False)
    targets = rng.choice(np.setdiff1d(np.arange(nb), ids), n, replace=False)
    stage = DeviceBuffer(n_layers * n * 2 * bpb)  # 335 MB: one launch per call
    x = TransferContext(0)
    try:
        saved, _ = save_transfers(layers, ids.tolist(), stage)
        x.save_layers(saved, _lib.MODE_KERNEL)
        assert closed_form_host_check(layers, ids.tolist(), saved) == 0
        scatter = load_transfers(layers, targets, saved)
        src_of = {int(t): int(s) for t, s in zip(targets, ids)}
        assert x.route_shape(_lib.ROUTE_LOAD_DEVICE)[2] is False
        for call in range(6):
            x.load_layers(scatter, _lib.MODE_KERNEL)
            x.synchronize()
            assert closed_form_tensor_check(layers, src_of) == 0, f"call {call}"
            for l in range(n_layers):
                layers.bufs[l].fill_random(layers.seeds[l])
        threads, unroll, decided = x.route_shape(_lib.ROUTE_LOAD_DEVICE)
        assert decided and (threads, unroll) in (
            (512, 2 | _lib.KERNEL_NONTEMPORAL | _lib.KERNEL_XCD_MAJOR),
            (512, 1 | _lib.KERNEL_NONTEMPORAL))
        say(f"[gpu] scatter shape chosen: {threads} threads, unroll {unroll:#x}")
        x.set_kernel_shape_dir(_lib.ROUTE_LOAD_DEVICE, 256, 1)
        assert x.route_shape(_lib.ROUTE_LOAD_DEVICE) == (256, 1, True)
        x.load_layers(scatter, _lib.MODE_KERNEL)
        x.synchronize()
        assert closed_form_tensor_check(layers, src_of) == 0
        x.reset_kernel_shape()
        assert x.route_shape(_lib.ROUTE_LOAD_DEVICE)[2] is False
        with pytest.raises(_lib.PegaFlowError, match="scatter route only"):
            x.set_kernel_shape_dir(_lib.ROUTE_SAVE_DEVICE, 512, 1 | _lib.KERNEL_AUTO)
    finally:
        x.close()
        stage.close()
        layers.close()
