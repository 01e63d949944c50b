"""The disk tier on the GPU: blocks saved from HBM are written to packed
files whose bytes match the oracle's packing (seal_offload.rs:379-448), a
fresh engine on the same directory indexes them, a prefix query reads them
back into its pinned pool (lib.rs:855-941), and a load by hash restores them
into HBM bit-exactly."""

import glob
import hashlib
import json
import os
import sys
import time

import numpy as np
import pytest

import oracle
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import PyLoadState
from pegaflow_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def h(i):
    return hashlib.sha256(b"ssd" + int(i).to_bytes(8, "little")).digest()


def wait(st, timeout=60.0):
    t0 = time.monotonic()
    while not st.is_ready():
        assert time.monotonic() - t0 < timeout, "load did not complete"
        time.sleep(0.0005)
    return st.get_state()


class Layers:
    """n_layers x tp_size layers on device 0 (slot = layer*tp + rank):
    KV-first (two segments of bpb bytes per block) or blocks-first (one
    segment of bpb bytes, packed whole)."""

    def __init__(self, n_layers, tp, nb, bpb, seed, segments=2):
        self.n_layers, self.tp, self.nb, self.bpb = n_layers, tp, nb, bpb
        self.segments = segments
        self.kv = nb * bpb if segments == 2 else 0
        self.size = nb * bpb * segments
        self.slot_bytes = bpb * segments
        self.names = [f"model.layers.{l}.self_attn" for l in range(n_layers)]
        self.bufs = {(l, r): DeviceBuffer(self.size) for l in range(n_layers) for r in range(tp)}
        self.fill(seed)

    def fill(self, seed):
        for (l, r), b in self.bufs.items():
            b.fill_random(oracle.layer_seed(seed + 1000 * r, l))

    def register(self, engine, inst, ns, rank=0):
        """Registers one rank's layers.  The engine keeps one registration per
        layer name per device, as the reference does (its ranks sit on their
        own GPUs), so on one GPU the ranks take turns: register, then save
        or load that rank."""
        for l in range(self.n_layers):
            b = self.bufs[(l, rank)]
            engine.register_context_layer(inst, ns, 0, self.names[l], b.ptr, self.size, self.nb,
                                          self.bpb, self.kv, self.segments, rank, self.tp,
                                          self.n_layers)

    def host(self):
        return {k: b.download() for k, b in self.bufs.items()}

    def saved_slots(self, host, ids):
        """Per block: the (K, V) of every slot, from the oracle's save path."""
        per = {}
        m = len(ids)
        split = self.segments == 2
        for key, buf in host.items():
            buf = buf.copy()
            reg = oracle.layout(buf.ctypes.data, self.size, self.nb, self.bpb, self.kv,
                                self.segments)
            region = np.zeros(m * self.slot_bytes, np.uint8)
            k, v, is_split = oracle.save_host_layout(reg, m, region.ctypes.data,
                                                     region.ctypes.data + m * self.bpb)
            assert is_split == split
            oracle.process_save(reg, buf, ids, k, v)
            per[key] = region
        out = []
        for j in range(m):
            slots = []
            for l in range(self.n_layers):
                for r in range(self.tp):
                    reg_ = per[(l, r)]
                    slots.append((reg_[j * self.bpb:(j + 1) * self.bpb].tobytes(),
                                  reg_[(m + j) * self.bpb:(m + j + 1) * self.bpb].tobytes()
                                  if split else None))
            out.append(slots)
        return out

    def expected(self, before, clobbered, ids, targets):
        out = {}
        m = len(ids)
        for key in self.bufs:
            src, dst = before[key].copy(), clobbered[key].copy()
            region = np.zeros(m * self.slot_bytes, np.uint8)
            reg_s = oracle.layout(src.ctypes.data, self.size, self.nb, self.bpb, self.kv,
                                  self.segments)
            k, v, _ = oracle.save_host_layout(reg_s, m, region.ctypes.data,
                                              region.ctypes.data + m * self.bpb)
            oracle.process_save(reg_s, src, ids, k, v)
            reg_d = oracle.layout(dst.ctypes.data, self.size, self.nb, self.bpb, self.kv,
                                  self.segments)
            oracle.process_load(reg_d, dst, targets, k, v)
            out[key] = dst
        return out

    def close(self):
        for b in self.bufs.values():
            b.close()


def check_files(root, ns, hashes, want_slots):
    """Every block named in a sidecar matches the oracle's packing, and each
    file is exactly the packing of its blocks in sidecar order."""
    by_hash = {hh: j for j, hh in enumerate(hashes)}
    seen = set()
    for side in glob.glob(os.path.join(root, ns, "*.json")):
        meta = json.load(open(side))
        assert meta["namespace"] == ns and meta["version"] == 1
        data = open(os.path.join(root, ns, meta["file"]), "rb").read()
        assert len(data) == meta["size"]
        blocks = []
        for b in meta["blocks"]:
            j = by_hash[bytes.fromhex(b["hash"])]
            m = b["meta"]
            slots = [(s["is_split"], s["size"]) for s in m["slots"]]
            size = sum(sz for _, sz in slots)
            assert oracle.unpack_block(data[m["offset"]:m["offset"] + size], slots) == \
                want_slots[j]
            assert json.dumps(m, separators=(",", ":")) == oracle.block_meta_json(
                meta["file"], m["offset"], slots, m["total_slots"])
            blocks.append(want_slots[j])
            seen.add(j)
        packed, offs = oracle.pack_blocks(blocks)
        assert packed == data and offs == [b["meta"]["offset"] for b in meta["blocks"]]
    assert seen == set(range(len(hashes)))


@pytest.mark.parametrize("tp,segments", [(1, 2), (2, 2), (1, 1)],
                         ids=["kv_first-tp1", "kv_first-tp2", "blocks_first-tp1"])
def test_offload_restart_prefetch_load(gpu, tmp_path, tp, segments):
    say(f"[gpu] disk tier offload -> restart -> prefetch -> load tp={tp} segments={segments}")
    root = str(tmp_path / "pega")
    layers = Layers(4, tp, 64, 4096 * (3 - segments), seed=17 + tp + (10 if segments == 1 else 0),
                    segments=segments)
    ids = [5, 17, 3, 60, 41, 8, 9, 10, 11, 12]
    hashes = [h(i + 100 * tp) for i in ids]
    try:
        e1 = PegaEngine(pool_size=128 * MiB)
        e1.enable_disk(root, max_pack_blocks=4)
        before = layers.host()
        for r in range(tp):
            layers.register(e1, "inst", "llama", r)
            e1.batch_save_kv_blocks("inst", r, 0, [(n, ids, hashes) for n in layers.names])
        e1.flush_disk()
        s = e1.disk_stats()
        slot_bytes = layers.slot_bytes
        assert s["offloaded_blocks"] == len(ids) and s["failures"] == 0
        assert s["written_bytes"] == len(ids) * 4 * tp * slot_bytes == s["bytes"]
        assert s["files"] >= 3  # at most 4 blocks per file
        check_files(root, "llama", hashes, layers.saved_slots(before, ids))
        e1.close()

        e2 = PegaEngine(pool_size=128 * MiB)
        e2.enable_disk(root)
        assert e2.disk_stats()["indexed_blocks"] == len(ids)
        layers.register(e2, "inst2", "llama")
        layers.fill(seed=999)
        clobbered = layers.host()
        q = e2.count_prefix_hit_blocks_with_prefetch("inst2", hashes)
        assert q["prefetch_state"] == "loading" and q["loading_blocks"] == len(ids)
        e2.wait_prefetch()
        q = e2.count_prefix_hit_blocks_with_prefetch("inst2", hashes)
        assert q["prefetch_state"] == "ready" and q["hit_blocks"] == len(ids)
        targets = [0, 1, 2, 63, 62, 40, 39, 38, 20, 21]
        for r in range(tp):
            layers.register(e2, "inst2", "llama", r)
            st = PyLoadState(num_layers=layers.n_layers)
            e2.batch_load_kv_blocks("inst2", r, 0, st.shm_name(), layers.names, targets, hashes)
            assert wait(st) == 1
        exp = layers.expected(before, clobbered, ids, targets)
        for key, b in layers.bufs.items():
            assert np.array_equal(b.download(), exp[key]), f"layer/rank {key}"
        # Blocks read back are not written again.
        assert e2.disk_stats()["offloaded_blocks"] == 0
        e2.close()
    finally:
        layers.close()


def test_load_rejects_blocks_of_another_shape(gpu, tmp_path):
    say("[gpu] disk tier: a stored block of another size is refused at load")
    root = str(tmp_path / "pega")
    a = Layers(2, 1, 32, 2048, seed=3)
    b = Layers(2, 1, 32, 1024, seed=4)
    try:
        e1 = PegaEngine(pool_size=64 * MiB)
        e1.enable_disk(root)
        a.register(e1, "a", "shared")
        e1.batch_save_kv_blocks("a", 0, 0, [(n, [1, 2], [h(1), h(2)]) for n in a.names])
        e1.close()
        e2 = PegaEngine(pool_size=64 * MiB)
        e2.enable_disk(root)
        b.register(e2, "b", "shared")
        e2.count_prefix_hit_blocks_with_prefetch("b", [h(1), h(2)])
        e2.wait_prefetch()
        before = b.host()
        st = PyLoadState()
        with pytest.raises(RuntimeError, match="holds 4096 split bytes .* registered with "
                                               "2048 split bytes"):
            e2.batch_load_kv_blocks("b", 0, 0, st.shm_name(), b.names, [0, 1], [h(1), h(2)])
        assert st.get_state() == -1
        after = b.host()
        assert all(np.array_equal(before[k], after[k]) for k in before)
        e2.close()
    finally:
        a.close()
        b.close()
