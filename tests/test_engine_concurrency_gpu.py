"""PegaEngine under concurrent use on the GPU.

Two saver threads keep sealing new batches of blocks, each from an instance
of its own (two save workers evicting from one pool), while two loader
threads restore recently sealed batches into disjoint target blocks of a
third instance (plain and layered LoadStates alternating) and a query
thread counts prefix hits.  The pool holds only a few batches, so eviction
runs all the time.  It runs with the zero-copy kernels both ways, with saves
staged on the copy engines beside kernel loads, with both directions staged,
and in the engine's default modes with TinyLFU admission and the
pre-eviction monitor on.

Every load that succeeds must leave its targets holding exactly the source
blocks' words, checked in closed form on the device.  A load that names a
hash already evicted must fail cleanly (an error from the call or a -1
LoadState), never with wrong bytes.  The engine's stats must add up at the
end, and once every block is evicted the pool must be empty.
"""

import hashlib
import os
import random
import sys
import threading
import time

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import PyLoadState
from pegaflow_amd.runtime import DeviceBuffer, verify_random_chunks

pytestmark = pytest.mark.gpu
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def h(batch, i):
    return hashlib.sha256(b"conc-%d-" % batch + int(i).to_bytes(8, "little")).digest()


class Layers:
    def __init__(self, n_layers, nb, bpb, seed):
        self.nb, self.bpb, self.kv, self.size = nb, bpb, nb * bpb, 2 * nb * bpb
        self.names = [f"layer.{l}" for l in range(n_layers)]
        self.seeds = [oracle.layer_seed(seed, l) for l in range(n_layers)]
        self.bufs = [DeviceBuffer(self.size) for _ in range(n_layers)]
        for b, s in zip(self.bufs, self.seeds):
            b.fill_random(s)

    def register(self, engine, inst):
        for name, b in zip(self.names, self.bufs):
            engine.register_context_layer(inst, "conc", 0, name, b.ptr, self.size, self.nb,
                                          self.bpb, self.kv, 2, 0, 1, len(self.names))

    def close(self):
        for b in self.bufs:
            b.close()


def check_targets(dst, src, sources, targets):
    """Mismatching words: dst block targets[j] must hold src block sources[j]
    (K and V segments) in every layer."""
    t = np.asarray(targets, np.uint64)
    s = np.asarray(sources, np.uint64)
    bad = 0
    for l, buf in enumerate(dst.bufs):
        addrs = np.concatenate([buf.ptr + t * dst.bpb, buf.ptr + dst.kv + t * dst.bpb])
        offs = np.concatenate([s * src.bpb // 8, (src.kv + s * src.bpb) // 8])
        bad += verify_random_chunks(addrs, offs, src.bpb, src.seeds[l])
    return bad


# (save mode, load mode, storage policy): the zero-copy kernels both ways;
# saves staged on the copy engines beside kernel loads; both directions
# staged; and AUTO both ways with TinyLFU admission and a pre-eviction
# monitor that wakes every millisecond, so blocks are refused and dropped
# by a thread of the engine's own while loads hold them.
MODES = [("kernel", "kernel", False), ("staged", "kernel", False), ("staged", "staged", False),
         ("auto", "auto", True)]


@pytest.mark.parametrize("save_mode,load_mode,policy", MODES,
                         ids=[f"{a}-{b}{'-policy' if c else ''}" for a, b, c in MODES])
def test_concurrent_saves_loads_and_queries(gpu, save_mode, load_mode, policy):
    say(f"[gpu] engine concurrency ({save_mode} saves, {load_mode} loads, storage policy "
        f"{'on' if policy else 'off'}): two savers, two loaders, a query thread, constant eviction")
    n_layers, nb, bpb, per_batch = 8, 512, 16384, 32
    batch_bytes = n_layers * per_batch * 2 * bpb  # 8 MiB
    e = PegaEngine(pool_size=6 * batch_bytes)      # room for about 6 batches
    e.set_transfer_modes(_lib.MODE_NAMES[save_mode], _lib.MODE_NAMES[load_mode])
    if policy:
        # Admission sized for one entry per block; the monitor keeps two
        # batches' bytes free once fewer than one batch's are.
        e.set_storage_policy(lfu_admission=True, value_size_hint=n_layers * 2 * bpb,
                             pre_evict=True, pre_evict_threshold=batch_bytes,
                             pre_evict_target=2 * batch_bytes, pre_evict_interval_ms=1)
    srcs = [Layers(n_layers, nb, bpb, seed=3), Layers(n_layers, nb, bpb, seed=5)]
    dst = Layers(n_layers, nb, bpb, seed=4)
    for k, src in enumerate(srcs):
        src.register(e, f"prefill{k}")
    dst.register(e, "decode")
    sealed = []            # (saver, batch, source block ids), in sealing order
    lock = threading.Lock()
    stop = threading.Event()
    errors = []
    stats = {"saves": 0, "loads_ok": 0, "loads_missing": 0, "queries": 0, "words_checked": 0}

    def saver(k):
        rng = random.Random(1 + k)
        src = srcs[k]
        batch = k  # saver k's batches are k, k + 2, ...: hashes differ between savers
        while not stop.is_set():
            ids = rng.sample(range(nb), per_batch)
            hashes = [h(batch, i) for i in ids]
            e.batch_save_kv_blocks(f"prefill{k}", 0, 0, [(n, ids, hashes) for n in src.names])
            with lock:
                sealed.append((k, batch, ids))
                stats["saves"] += 1
            batch += 2

    def loader(k):
        rng = random.Random(10 + k)
        # Loader k owns target blocks [k*256, k*256 + 256) of the decode instance.
        own = list(range(k * (nb // 2), (k + 1) * (nb // 2)))
        n = 0
        while not stop.is_set():
            with lock:
                recent = sealed[-4:]
            if not recent:
                time.sleep(0.001)
                continue
            ks, batch, ids = rng.choice(recent)
            pick = rng.sample(range(per_batch), 16)
            sources = [ids[j] for j in pick]
            hashes = [h(batch, i) for i in sources]
            targets = rng.sample(own, 16)
            st = PyLoadState(num_layers=n_layers) if n % 2 else PyLoadState()
            n += 1
            try:
                e.batch_load_kv_blocks("decode", 0, 0, st.shm_name(), dst.names, targets, hashes)
            except _lib.PegaFlowError as err:
                assert "missing KV block hash" in str(err), str(err)
                assert st.get_state() == -1
                with lock:
                    stats["loads_missing"] += 1
                continue
            t0 = time.monotonic()
            while not st.is_ready():
                assert time.monotonic() - t0 < 30, "load did not complete"
                time.sleep(0.0002)
            assert st.get_state() == 1
            if n % 2 == 0:  # layered state: every layer was published
                assert st.layers_done() == n_layers
            bad = check_targets(dst, srcs[ks], sources, targets)
            assert bad == 0, f"loader {k}: {bad} mismatching words (batch {batch})"
            with lock:
                stats["loads_ok"] += 1
                stats["words_checked"] += n_layers * 16 * 2 * bpb // 8

    def querier():
        while not stop.is_set():
            with lock:
                recent = sealed[-8:]
            for ks, batch, ids in recent:
                hits = e.count_prefix_hit_blocks(f"prefill{ks}", [h(batch, i) for i in ids])
                assert 0 <= hits <= per_batch
            with lock:
                stats["queries"] += 1
            time.sleep(0.0005)

    def guard(fn, *a):
        try:
            fn(*a)
        except BaseException as err:  # report any thread's failure in the test
            errors.append(err)
            stop.set()

    threads = [threading.Thread(target=guard, args=(saver, 0)),
               threading.Thread(target=guard, args=(saver, 1)),
               threading.Thread(target=guard, args=(loader, 0)),
               threading.Thread(target=guard, args=(loader, 1)),
               threading.Thread(target=guard, args=(querier,))]
    try:
        for t in threads:
            t.start()
        # PEGAFLOW_SOAK_SECONDS lengthens the run (6 s by default).
        deadline = time.monotonic() + float(os.environ.get("PEGAFLOW_SOAK_SECONDS", "6"))
        while time.monotonic() < deadline and not stop.is_set():
            time.sleep(0.05)
        stop.set()
        for t in threads:
            t.join(60)
            assert not t.is_alive(), "a worker thread did not stop"
        if errors:
            raise errors[0]
        e.wait_idle()
        s = e.stats()
        say(f"[gpu] concurrency: {stats}; engine {s}")
        assert stats["saves"] >= 10 and stats["loads_ok"] >= 10, stats
        assert s["evicted_blocks"] > 0, "the pool never filled"
        if policy:
            assert s["pre_evicted_blocks"] > 0, "the monitor never ran"
            assert s["pre_evicted_blocks"] <= s["evicted_blocks"]
        # With every block evicted (a monitor asked to free more than the
        # pool holds, then stopped), nothing may keep pool memory.
        everything = s["pool_total_bytes"] + 1
        e.set_storage_policy(pre_evict=True, pre_evict_threshold=everything,
                             pre_evict_target=everything, pre_evict_interval_ms=1)
        t0 = time.monotonic()
        while e.stats()["sealed_blocks"] and time.monotonic() - t0 < 10:
            time.sleep(0.005)
        e.set_storage_policy()  # joins the monitor
        s = e.stats()
        say(f"[gpu] after evicting everything: {s}")
        assert s["sealed_blocks"] == 0 and s["inflight_blocks"] == 0, s
        assert s["pool_used_bytes"] == 0, s
        assert s["load_failures"] == 0
        assert s["pool_used_bytes"] <= s["pool_total_bytes"]
        assert s["loaded_bytes"] == stats["loads_ok"] * n_layers * 16 * 2 * bpb
    finally:
        stop.set()
        e.close()
        for src in srcs:
            src.close()
        dst.close()
