"""Seeded fuzz of PegaEngine's save and load by hash on the GPU.

Each seed builds an engine with a source instance and a target instance in
one namespace (random layer count, layout and segment size, some segment
sizes not 16-byte multiples; a third of the seeds with two tensor-parallel
ranks, registered on the one device with the same tensors), then runs a
random sequence of calls, each by a random rank and in transfer modes drawn
at random:
- saves of a random subset of layers, each layer with a list of its own or
  all sharing one, naming negative ids, hashes named twice, hashes sealed
  before and hashes an earlier call left part-way in flight;
- the source tensors refilled with new bits after every save, so a slot
  that keeps an earlier copy shows it;
- loads of random hashes into random targets of a random subset of layers,
  with negative and repeated targets and plain or layered LoadStates; some
  name a hash that is not sealed and must fail as a whole, writing nothing.

After every load each target tensor is compared byte for byte with a model
of the reference's rules:
- save (lib.rs:553-782, storage.rs:457-514): negative ids are skipped; a
  hash sealed before the call, or a slot already filled, is skipped; within
  one layer's list the first occurrence of a hash fills its slot; a block
  seals once the slot of every layer and rank has arrived;
- load (lib.rs:957-1069): every hash must be sealed or the call fails;
  negative ids are skipped; a rank loads its own slots; blocks are written
  in list order, so a target named twice ends with the later block.
At the end the engine's sealed and in-flight block counts must match the
model's.  A quarter of the seeds run on a pool of about ten blocks, so
saves evict: after each save the model drops the blocks the engine no
longer holds (asked one hash at a time, which leaves recency alone), and a
save that finds the pool held by blocks in flight must fail as exhausted,
publishing nothing.
"""

import hashlib
import random
import sys

import numpy as np
import pytest

from pegaflow_amd import _lib
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import PyLoadState
from pegaflow_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu
MiB = 1 << 20

LAYOUTS = ("kv_first", "kv_first_padded", "blocks_first")
SEGMENT_BYTES = (512, 1040, 4096, 16384, 200)   # one K or V segment (KV-first)
BLOCK_BYTES = (1024, 2080, 8192, 32768, 400)    # one whole block (blocks-first)
MODES = ("kernel", "staged", "auto", "dma_batched", "dma_reference")
NB = 48
HASHES = 24


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Tensors:
    """One instance's layers on device 0, registered with the engine."""

    def __init__(self, engine, inst, n_layers, layout, seg, seed, tp):
        self.layout = layout
        if layout == "blocks_first":
            self.bpb, self.kv, self.segments = seg, 0, 1
            self.size = NB * seg
        else:
            pad = 4096 if layout == "kv_first_padded" else 0
            self.bpb, self.kv, self.segments = seg, NB * seg + pad, 2
            self.size = self.kv + NB * seg
        self.names = [f"layer.{l}" for l in range(n_layers)]
        self.bufs = [DeviceBuffer(self.size) for _ in range(n_layers)]
        self.refill(seed)
        # Every rank registers the same tensors: one device holds one
        # registration per layer name (the last), as in the reference.
        for rank in range(tp):
            for name, b in zip(self.names, self.bufs):
                engine.register_context_layer(inst, "fuzz", 0, name, b.ptr, self.size, NB,
                                              self.bpb, self.kv, self.segments, rank, tp, n_layers)

    def refill(self, seed):
        for l, b in enumerate(self.bufs):
            b.fill_random(seed * 1000 + l)

    def download(self):
        return [b.download() for b in self.bufs]

    def slot(self, arr, b):
        """The bytes a save copies for block b of one layer."""
        s = self.bpb
        if self.segments == 1:
            return arr[b * s:(b + 1) * s].copy()
        v = self.kv + b * s
        return np.concatenate([arr[b * s:(b + 1) * s], arr[v:v + s]])

    def put(self, arr, b, data):
        """What a load of `data` into block b writes into one layer."""
        s = self.bpb
        if self.segments == 1:
            arr[b * s:(b + 1) * s] = data
        else:
            v = self.kv + b * s
            arr[b * s:(b + 1) * s] = data[:s]
            arr[v:v + s] = data[s:]

    def close(self):
        for b in self.bufs:
            b.close()


def h(seed, j):
    return hashlib.sha256(b"fuzz-%d-%d" % (seed, j)).digest()


def rand_ids(rng, n):
    return [-1 if rng.random() < 0.1 else rng.randrange(NB) for _ in range(n)]


@pytest.mark.parametrize("seed", range(96))
def test_engine_calls_vs_model(gpu, seed):
    rng = random.Random(seed)
    n_layers = rng.randint(1, 5)
    tp = 2 if 48 <= seed < 72 else 1
    evict = seed >= 72  # a pool of about ten blocks: saves evict
    layout = LAYOUTS[seed % len(LAYOUTS)]
    seg = rng.choice(BLOCK_BYTES if layout == "blocks_first" else SEGMENT_BYTES)
    say(f"[gpu] engine fuzz seed={seed}: {n_layers} layers, tp {tp}, {layout}, {seg} B segments"
        f"{', evicting' if evict else ''}")
    slot_bytes = seg * (1 if layout == "blocks_first" else 2)
    e = PegaEngine(pool_size=10 * n_layers * tp * slot_bytes + 4096 if evict else 64 * MiB)
    src = Tensors(e, "src", n_layers, layout, seg, seed * 7 + 1, tp)
    dst = Tensors(e, "dst", n_layers, layout, seg, seed * 7 + 2, tp)
    pool = [h(seed, j) for j in range(HASHES)]
    sealed = {}     # hash -> {(layer, rank): slot bytes}
    inflight = {}   # hash -> {(layer, rank): slot bytes}
    expect = dst.download()
    calls = {"saves": 0, "loads": 0, "failed_loads": 0, "exhausted_saves": 0}

    def resync():
        """Blocks the engine evicted are gone from the model too."""
        for k in list(sealed):
            if e.count_prefix_hit_blocks("src", [k]) == 0:
                del sealed[k]

    try:
        for step in range(40):
            save_mode, load_mode = rng.choice(MODES), rng.choice(MODES)
            e.set_transfer_modes(_lib.MODE_NAMES[save_mode], _lib.MODE_NAMES[load_mode])
            rank = rng.randrange(tp)
            if rng.random() < 0.5 or not sealed:
                # A save of a random subset of layers.
                if evict and rng.random() < 0.8:  # mostly whole blocks: fewer held in flight
                    layers = rng.sample(range(n_layers), n_layers)
                else:
                    layers = rng.sample(range(n_layers), rng.randint(1, n_layers))
                # One list for every layer (mostly, when the pool is small:
                # blocks left in flight hold memory that eviction cannot free).
                shared = rng.random() < (0.9 if evict else 0.5)
                n = rng.randint(1, 12)
                one = (rand_ids(rng, n), [rng.choice(pool) for _ in range(n)])
                lists = {l: one if shared else (rand_ids(rng, n), [rng.choice(pool)
                                                                   for _ in range(n)])
                         for l in layers}
                host = src.download()
                fresh = {}
                for l in layers:
                    ids, hashes = lists[l]
                    named = set()
                    for b, k in zip(ids, hashes):
                        if b < 0 or k in sealed or k in named:
                            continue
                        named.add(k)
                        if (l, rank) in inflight.get(k, {}):
                            continue
                        fresh.setdefault(k, {})[(l, rank)] = src.slot(host[l], b)
                try:
                    e.batch_save_kv_blocks("src", rank, 0, [(src.names[l], lists[l][0],
                                                             lists[l][1]) for l in layers])
                except _lib.PegaFlowError as err:
                    # Only a small pool may run out (blocks in flight hold
                    # memory eviction cannot free); such a save publishes
                    # nothing.
                    assert evict and "pinned pool exhausted" in str(err), err
                    calls["exhausted_saves"] += 1
                    fresh = {}
                for k, slots in fresh.items():
                    inflight.setdefault(k, {}).update(slots)
                    if len(inflight[k]) == n_layers * tp:
                        sealed[k] = inflight.pop(k)
                if evict:
                    resync()
                src.refill(seed * 7 + 100 + step)
                calls["saves"] += 1
                continue
            # A load of a random subset of layers.
            names_idx = rng.sample(range(n_layers), rng.randint(1, n_layers))
            n = rng.randint(1, 10)
            known = list(sealed)
            hashes = [rng.choice(known) for _ in range(n)]
            missing = rng.random() < 0.15 and len(sealed) < HASHES
            if missing:
                hashes[rng.randrange(n)] = rng.choice([k for k in pool if k not in sealed])
            targets = rand_ids(rng, n)
            layered = rng.random() < 0.5
            st = PyLoadState(num_layers=len(names_idx)) if layered else PyLoadState()
            names = [dst.names[l] for l in names_idx]
            try:
                e.batch_load_kv_blocks("dst", rank, 0, st.shm_name(), names, targets, hashes)
                raised = None
            except _lib.PegaFlowError as err:
                raised = err
            if missing:
                assert raised is not None and "missing KV block hash" in str(raised), raised
                assert st.get_state() == -1
                calls["failed_loads"] += 1
            else:
                assert raised is None, raised
                e.wait_idle()
                assert st.is_ready() and st.get_state() == 1
                if layered:
                    assert st.layers_done() == len(names_idx)
                for l in names_idx:
                    for t, k in zip(targets, hashes):
                        if t >= 0:
                            dst.put(expect[l], t, sealed[k][(l, rank)])
                calls["loads"] += 1
            got = dst.download()
            for l in range(n_layers):
                assert np.array_equal(got[l], expect[l]), (
                    f"step {step}: layer {l} differs after a load in {load_mode} mode "
                    f"(targets {targets})")
        s = e.stats()
        say(f"[gpu] engine fuzz seed={seed}: {calls}, model {len(sealed)} sealed / "
            f"{len(inflight)} in flight; engine {s['sealed_blocks']} / {s['inflight_blocks']}, "
            f"{s['evicted_blocks']} evicted")
        assert s["sealed_blocks"] == len(sealed) and s["inflight_blocks"] == len(inflight), s
        assert s["load_failures"] == 0, s
        if not evict:
            assert s["evicted_blocks"] == 0, s
    finally:
        e.close()
        src.close()
        dst.close()
