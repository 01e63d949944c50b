"""PegaEngine on the GPU: save by hash, load by hash with LoadState, seal
visibility across layers and TP ranks, dedup, prefix counting, eviction, and
per-layer progress — bytes checked against the oracle or in closed form."""

import hashlib
import sys
import time

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import PyLoadState
from pegaflow_amd.runtime import DeviceBuffer
from pegaflow_amd.workload import LLAMA3_8B, DeviceLayers, draw_blocks, verify_restored

pytestmark = pytest.mark.gpu
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def h(i, salt=b"blk"):
    return hashlib.sha256(salt + int(i).to_bytes(8, "little")).digest()


def wait(st: PyLoadState, timeout=60.0):
    t0 = time.monotonic()
    while not st.is_ready():
        assert time.monotonic() - t0 < timeout, "load did not complete"
        time.sleep(0.0005)
    return st.get_state()


class Model:
    """n_layers KV-first layers [2, nb, ...] on device 0, registered with an
    engine as instance `inst` (tp_rank of tp_size)."""

    def __init__(self, engine, inst, n_layers, nb, bpb, seed=1, tp_rank=0, tp_size=1,
                 prefix="layer", total_layers=None):
        self.nb, self.bpb, self.n_layers = nb, bpb, n_layers
        self.kv = nb * bpb
        self.size = 2 * self.kv
        self.names = [f"{prefix}.{l}" for l in range(n_layers)]
        self.seeds = [oracle.layer_seed(seed, l) for l in range(n_layers)]
        self.bufs = []
        for l in range(n_layers):
            b = DeviceBuffer(self.size)
            b.fill_random(self.seeds[l])
            self.bufs.append(b)
            engine.register_context_layer(inst, "ns", 0, self.names[l], b.ptr, self.size, nb, bpb,
                                          self.kv, 2, tp_rank, tp_size,
                                          total_layers or n_layers)

    def host_copies(self):
        return [b.download() for b in self.bufs]

    def close(self):
        for b in self.bufs:
            b.close()


def expected_after_load(model, originals, ids, targets):
    """Oracle: save(ids) then load(targets) on each host copy."""
    out = []
    for l, ref in enumerate(originals):
        ref = ref.copy()
        reg = oracle.layout(ref.ctypes.data, model.size, model.nb, model.bpb, model.kv, 2)
        m = len(ids)
        host = np.zeros(2 * m * model.bpb, np.uint8)
        k, v, _ = oracle.save_host_layout(reg, m, host.ctypes.data,
                                          host.ctypes.data + m * model.bpb)
        oracle.process_save(reg, ref, ids, k, v)
        oracle.process_load(reg, ref, targets, k, v)
        out.append(ref)
    return out


@pytest.fixture
def engine(gpu):
    e = PegaEngine(pool_size=256 * MiB)
    yield e
    e.close()


@pytest.mark.parametrize("save_mode,load_mode", [
    ("kernel", "kernel"), ("kernel", "dma_batched"), ("kernel", "dma_reference"),
    ("staged", "staged"), ("auto", "auto")])
def test_save_then_load_by_hash(engine, save_mode, load_mode):
    say(f"[gpu] engine save/load by hash save_mode={save_mode} load_mode={load_mode}")
    engine.set_transfer_modes(_lib.MODE_NAMES[save_mode], _lib.MODE_NAMES[load_mode])
    m = Model(engine, "inst", 6, 64, 4096)
    orig = m.host_copies()
    ids = [5, 17, 3, 60, 41, 8]
    hashes = [h(i) for i in ids]
    engine.batch_save_kv_blocks("inst", 0, 0, [(n, ids, hashes) for n in m.names])
    assert engine.count_prefix_hit_blocks("inst", hashes) == len(ids)
    targets = [0, 1, 2, 63, 62, 40]
    st = PyLoadState(num_layers=m.n_layers)
    engine.batch_load_kv_blocks("inst", 0, 0, st.shm_name(), m.names, targets, hashes)
    assert wait(st) == 1
    assert st.layers_done() == m.n_layers
    exp = expected_after_load(m, orig, ids, targets)
    for l in range(m.n_layers):
        assert np.array_equal(m.bufs[l].download(), exp[l]), f"layer {l}"
    s = engine.stats()
    assert s["sealed_blocks"] == len(ids) and s["inflight_blocks"] == 0
    assert s["saved_bytes"] == s["loaded_bytes"] == m.n_layers * len(ids) * 2 * m.bpb
    m.close()


def test_seal_visibility_dedup_and_prefix(engine):
    say("[gpu] engine seal visibility / dedup / prefix")
    m = Model(engine, "inst", 4, 32, 2048)
    ids = list(range(10))
    hashes = [h(i) for i in ids]
    # Half the layers: blocks are inflight, not visible (storage.rs:136-208).
    engine.batch_save_kv_blocks("inst", 0, 0, [(n, ids, hashes) for n in m.names[:2]])
    assert engine.count_prefix_hit_blocks("inst", hashes) == 0
    assert engine.stats()["inflight_blocks"] == 10
    used = engine.stats()["pool_used_bytes"]
    # Re-saving the same layers is a no-op (slot already inflight).
    engine.batch_save_kv_blocks("inst", 0, 0, [(n, ids, hashes) for n in m.names[:2]])
    assert engine.stats()["pool_used_bytes"] == used
    engine.batch_save_kv_blocks("inst", 0, 0, [(n, ids, hashes) for n in m.names[2:]])
    assert engine.count_prefix_hit_blocks("inst", hashes) == 10
    s = engine.stats()
    assert s["sealed_blocks"] == 10 and s["inflight_blocks"] == 0
    # Sealed blocks are skipped entirely.
    used = s["pool_used_bytes"]
    engine.batch_save_kv_blocks("inst", 0, 0, [(n, ids, hashes) for n in m.names])
    assert engine.stats()["pool_used_bytes"] == used
    # Prefix counting stops at the first miss (lib.rs:803-838).
    assert engine.count_prefix_hit_blocks("inst", hashes[:3] + [h(99)] + hashes[3:]) == 3
    # Another namespace sees nothing.
    engine.register_context_layer("other", "ns2", 0, "x", m.bufs[0].ptr, m.size, m.nb, m.bpb,
                                  m.kv, 2, 0, 1, 1)
    assert engine.count_prefix_hit_blocks("other", hashes) == 0
    m.close()


def _expect_per_layer(model, orig, pairs_per_layer):
    """Oracle: for each layer, save the listed source blocks and load them
    into the listed targets (pairs_per_layer[l] = (sources, targets))."""
    out = []
    for l, ref in enumerate(orig):
        src, dst = pairs_per_layer[l]
        out.append(expected_after_load(model, [ref], src, dst)[0])
    return out


def test_duplicate_hash_in_one_save_keeps_first(engine):
    """One save batch names a hash twice with different blocks.  Both are
    copied, the first occurrence fills the slot and the second is dropped
    (lib.rs:590-621; storage.rs:181-184, 483-486): the whole-batch path."""
    say("[gpu] engine duplicate hash in one save (whole batch)")
    m = Model(engine, "dup", 4, 32, 2048, seed=12)
    orig = m.host_copies()
    ids, hashes = [3, 7, 12], [h(1), h(2), h(1)]
    engine.batch_save_kv_blocks("dup", 0, 0, [(n, ids, hashes) for n in m.names])
    s = engine.stats()
    assert s["sealed_blocks"] == 2 and s["inflight_blocks"] == 0
    st = PyLoadState()
    engine.batch_load_kv_blocks("dup", 0, 0, st.shm_name(), m.names, [20, 21], [h(1), h(2)])
    assert wait(st) == 1
    exp = _expect_per_layer(m, orig, [([3, 7], [20, 21])] * m.n_layers)
    for l in range(m.n_layers):
        assert np.array_equal(m.bufs[l].download(), exp[l]), f"layer {l}"
    m.close()


def test_duplicate_hash_slot_by_slot_keeps_first(engine):
    """The same rule when an earlier call left the block partly in flight,
    which sends the batch through the slot-by-slot path: layer 0's slot
    keeps the earlier call's block, the other layers the first occurrence."""
    say("[gpu] engine duplicate hash in one save (slot by slot)")
    m = Model(engine, "dup2", 4, 32, 2048, seed=13)
    orig = m.host_copies()
    engine.batch_save_kv_blocks("dup2", 0, 0, [(m.names[0], [5], [h(1)])])
    assert engine.stats()["inflight_blocks"] == 1
    ids, hashes = [3, 7, 12], [h(1), h(2), h(1)]
    engine.batch_save_kv_blocks("dup2", 0, 0, [(n, ids, hashes) for n in m.names])
    s = engine.stats()
    assert s["sealed_blocks"] == 2 and s["inflight_blocks"] == 0
    st = PyLoadState(num_layers=m.n_layers)
    engine.batch_load_kv_blocks("dup2", 0, 0, st.shm_name(), m.names, [20, 21], [h(1), h(2)])
    assert wait(st) == 1
    exp = _expect_per_layer(m, orig, [([5, 7], [20, 21])] +
                            [([3, 7], [20, 21])] * (m.n_layers - 1))
    for l in range(m.n_layers):
        assert np.array_equal(m.bufs[l].download(), exp[l]), f"layer {l}"
    m.close()


def _save_request(inst, layers):
    """SaveRequest wire bytes; each layer is (name, ids, hashes) or raw
    SaveLayer bytes."""
    from pegaflow_amd.rpc import proto

    out = proto.SaveRequest(instance_id=inst, tp_rank=0, device_id=0).SerializeToString()
    for layer in layers:
        if not isinstance(layer, bytes):
            name, ids, hashes = layer
            layer = proto.SaveLayer(layer_name=name, block_ids=ids,
                                    block_hashes=hashes).SerializeToString()
        out += b"\x22" + _varint(len(layer)) + layer  # field 4, length-delimited
    return out


def _varint(n):
    out = bytearray()
    while True:
        b, n = n & 0x7F, n >> 7
        out.append(b | (0x80 if n else 0))
        if not n:
            return bytes(out)


def test_save_requests_share_repeated_lists(engine):
    """The request decoder shares a layer's id and hash lists with the
    previous layer's when their bytes are equal (the whole message after the
    name, or either field alone), and decodes them otherwise: reversed lists,
    a layer with an unknown field first and its name last, ids that differ
    under shared hashes.  Every (hash, layer) slot must hold the block that
    layer's own lists name."""
    from pegaflow_amd.rpc import proto

    say("[gpu] engine save requests with shared and distinct per-layer lists")
    m = Model(engine, "req", 6, 64, 2048, seed=21)
    orig = m.host_copies()
    H = [h(i, b"req") for i in range(8)]
    A = [5, 17, 3, 60, 41, 8, 22, 30]
    B = [1, 2, 9, 10, 33, 34, 50, 63]
    odd = (b"\x48\x01" +  # field 9, varint: skipped
           proto.SaveLayer(block_ids=B, block_hashes=H).SerializeToString() +
           proto.SaveLayer(layer_name=m.names[3]).SerializeToString())
    req = _save_request("req", [
        (m.names[0], A, H),
        (m.names[1], A, H),              # the same bytes after the name
        (m.names[2], B[::-1], H[::-1]),  # both lists differ
        odd,                             # name last: decoded in full
        (m.names[4], A, H),              # hashes equal to the layer before's
        (m.names[5], B, H),              # hashes shared along the chain
    ])
    engine.serve_request(_lib.REQUEST_SAVE, req)
    want_ids = [A, A, B, B, A, B]
    # A second request whose layers are all alike.
    H2 = [h(i, b"req2") for i in range(5)]
    C = [11, 12, 13, 14, 15]
    engine.serve_request(_lib.REQUEST_SAVE, _save_request("req", [(n, C, H2) for n in m.names]))
    assert engine.stats()["sealed_blocks"] == len(H) + len(H2)
    for hashes, per_layer in ((H, want_ids), (H2, [C] * m.n_layers)):
        for l in range(m.n_layers):
            for i, hh in enumerate(hashes):
                b = per_layer[l][i]
                k, v = engine.read_block_slot("ns", hh, l)
                assert k == orig[l][b * m.bpb:(b + 1) * m.bpb].tobytes(), f"layer {l} block {i} K"
                assert v == orig[l][m.kv + b * m.bpb:m.kv + (b + 1) * m.bpb].tobytes(), \
                    f"layer {l} block {i} V"
    # A layer whose lists differ in length is refused as the reference does.
    bad = _save_request("req", [(m.names[0], A, H), (m.names[1], A[:3], H)])
    with pytest.raises(RuntimeError, match="block_ids length 3 does not match block_hashes 8"):
        engine.serve_request(_lib.REQUEST_SAVE, bad)
    m.close()


def test_load_pairs_ids_with_hashes_up_to_the_shorter_list(engine):
    """lib.rs:1008-1043 pairs ids with hashes as zip does: extra hashes get no
    target, extra ids are dropped; every hash is still looked up, so an
    unpaired hash must be sealed too."""
    say("[gpu] engine load pairs ids and hashes up to the shorter list")
    m = Model(engine, "zip", 2, 32, 2048, seed=21)
    orig = m.host_copies()
    ids = [3, 7, 12, 20]
    hashes = [h(i, b"zip") for i in ids]
    engine.batch_save_kv_blocks("zip", 0, 0, [(n, ids, hashes) for n in m.names])
    st = PyLoadState()  # two targets for four hashes
    engine.batch_load_kv_blocks("zip", 0, 0, st.shm_name(), m.names, [30, 31], hashes)
    assert wait(st) == 1
    exp = _expect_per_layer(m, orig, [([3, 7], [30, 31])] * m.n_layers)
    for l in range(m.n_layers):
        assert np.array_equal(m.bufs[l].download(), exp[l]), f"layer {l}"
    st = PyLoadState()  # four targets for two hashes
    engine.batch_load_kv_blocks("zip", 0, 0, st.shm_name(), m.names, [28, 29, 0, 1],
                                hashes[2:])
    assert wait(st) == 1
    exp = _expect_per_layer(m, exp, [([12, 20], [28, 29])] * m.n_layers)
    for l in range(m.n_layers):
        assert np.array_equal(m.bufs[l].download(), exp[l]), f"layer {l}"
    st = PyLoadState()
    with pytest.raises(RuntimeError, match="missing KV block hash at index 1"):
        engine.batch_load_kv_blocks("zip", 0, 0, st.shm_name(), m.names, [30],
                                    [hashes[0], h(99, b"zip")])
    assert st.get_state() == -1
    for l in range(m.n_layers):
        assert np.array_equal(m.bufs[l].download(), exp[l]), f"layer {l} written by a failed load"
    m.close()


def test_load_missing_hash_fails_whole_call(engine):
    say("[gpu] engine load with a missing hash")
    m = Model(engine, "inst", 2, 16, 1024)
    engine.batch_save_kv_blocks("inst", 0, 0, [(n, [1, 2], [h(1), h(2)]) for n in m.names])
    st = PyLoadState()
    with pytest.raises(RuntimeError, match="missing KV block hash at index 1"):
        engine.batch_load_kv_blocks("inst", 0, 0, st.shm_name(), m.names, [3, 4],
                                    [h(1), h(7)])
    assert st.get_state() == -1
    m.close()


def test_tp2_blocks_seal_when_both_ranks_saved(engine):
    say("[gpu] engine tp_size=2")
    r0 = Model(engine, "tp", 2, 16, 1024, seed=3, tp_rank=0, tp_size=2, prefix="a")
    with pytest.raises(RuntimeError, match="topology mismatch"):
        engine.register_context_layer("tp", "ns", 0, "zz", r0.bufs[0].ptr, r0.size, 16, 1024,
                                      r0.kv, 2, 0, 2, 3)
    # The second rank registers the same layer names with its own tensors.
    r1_bufs = []
    for l, name in enumerate(r0.names):
        b = DeviceBuffer(r0.size)
        b.fill_random(oracle.layer_seed(77, l))
        r1_bufs.append(b)
        engine.register_context_layer("tp", "ns", 0, name, b.ptr, r0.size, 16, 1024, r0.kv, 2, 1,
                                      2, 2)
    ids, hashes = [4, 9], [h(4), h(9)]
    # Registration of rank 1 replaced the device-0 registration of these layer
    # names, as in the reference (one registration per layer name per device).
    engine.batch_save_kv_blocks("tp", 0, 0, [(n, ids, hashes) for n in r0.names])
    assert engine.count_prefix_hit_blocks("tp", hashes) == 0  # rank 1 slots missing
    engine.batch_save_kv_blocks("tp", 1, 0, [(n, ids, hashes) for n in r0.names])
    assert engine.count_prefix_hit_blocks("tp", hashes) == 2
    for b in r1_bufs:
        b.close()
    r0.close()


def test_eviction_under_pool_pressure(gpu):
    say("[gpu] engine eviction")
    nb, bpb, layers = 64, 32768, 2
    per_batch = layers * 8 * 2 * bpb  # 8 blocks, K and V, 2 layers = 1 MiB
    e = PegaEngine(pool_size=3 * per_batch)
    m = Model(e, "ev", layers, nb, bpb, seed=5)
    orig = m.host_copies()
    batches = [[8 * k + i for i in range(8)] for k in range(4)]
    for k, ids in enumerate(batches):
        e.batch_save_kv_blocks("ev", 0, 0, [(n, ids, [h(i) for i in ids]) for n in m.names])
    s = e.stats()
    assert s["evicted_blocks"] >= 8
    # The oldest batch was evicted (LRU); the newest is present.
    assert e.count_prefix_hit_blocks("ev", [h(i) for i in batches[0]]) == 0
    assert e.count_prefix_hit_blocks("ev", [h(i) for i in batches[3]]) == 8
    # Restore the newest batch into other blocks and check the bytes.
    targets = list(range(40, 48))
    st = PyLoadState()
    e.batch_load_kv_blocks("ev", 0, 0, st.shm_name(), m.names, targets,
                           [h(i) for i in batches[3]])
    assert wait(st) == 1
    exp = expected_after_load(m, orig, batches[3], targets)
    for l in range(layers):
        assert np.array_equal(m.bufs[l].download(), exp[l])
    m.close()
    e.close()


def test_layerwise_progress_and_negative_ids(engine):
    say("[gpu] engine per-layer progress")
    m = Model(engine, "lw", 8, 256, 32768, seed=11)
    ids = list(range(0, 200, 2))
    hashes = [h(i, b"lw") for i in ids]
    engine.batch_save_kv_blocks("lw", 0, 0, [(n, ids, hashes) for n in m.names])
    targets = [-1 if i % 10 == 0 else 255 - i // 2 for i in range(len(ids))]
    st = PyLoadState(num_layers=m.n_layers)
    engine.batch_load_kv_blocks("lw", 0, 0, st.shm_name(), m.names, targets, hashes)
    seen = []
    while not st.is_ready():
        seen.append(st.layers_done())
    assert st.get_state() == 1 and st.layers_done() == m.n_layers
    assert seen == sorted(seen)  # monotonic
    for l in range(m.n_layers):
        assert st.wait_for_layer(l, timeout_s=1)
    kept = [(t, s) for t, s in zip(targets, ids) if t >= 0]
    src = np.arange(m.nb)
    for t, s in kept:
        src[t] = s
    from pegaflow_amd.runtime import verify_random_chunks
    blocks = np.arange(m.nb, dtype=np.uint64)
    for l, b in enumerate(m.bufs):
        addrs = np.concatenate([b.ptr + blocks * m.bpb, b.ptr + m.kv + blocks * m.bpb])
        offs = np.concatenate([src.astype(np.uint64) * m.bpb // 8,
                               (m.kv + src.astype(np.uint64) * m.bpb) // 8])
        assert verify_random_chunks(addrs, offs, m.bpb, m.seeds[l]) == 0
    m.close()


def test_llama_prefix_through_engine(gpu):
    """Config 2 through the engine: 32 layers, 640 blocks saved by hash and
    restored into 640 other blocks; closed-form check of every block."""
    say("[gpu] engine llama full size")
    e = PegaEngine(pool_size=1400 * MiB)
    layers = DeviceLayers(LLAMA3_8B, base_seed=0)
    names = [f"model.layers.{l}.self_attn" for l in range(LLAMA3_8B.layers)]
    for name, r in zip(names, layers.regs):
        e.register_context_layer("llama", "ns", 0, name, r.data_ptr, r.size_bytes, r.num_blocks,
                                 r.bytes_per_block, r.kv_stride_bytes, r.segments, 0, 1,
                                 LLAMA3_8B.layers)
    ids, targets = draw_blocks(LLAMA3_8B.num_blocks, 640, 0)
    hashes = [h(i, b"llama") for i in ids]
    t0 = time.perf_counter()
    e.batch_save_kv_blocks("llama", 0, 0, [(n, ids, hashes) for n in names])
    t1 = time.perf_counter()
    assert e.count_prefix_hit_blocks("llama", hashes) == 640
    st = PyLoadState(num_layers=len(names))
    t2 = time.perf_counter()
    e.batch_load_kv_blocks("llama", 0, 0, st.shm_name(), names, targets, hashes)
    assert wait(st) == 1
    t3 = time.perf_counter()
    P = 640 * 32 * 65536
    say(f"[gpu] engine save {P / (t1 - t0) / 1e9:.1f} GB/s, load {P / (t3 - t2) / 1e9:.1f} GB/s")
    assert verify_restored(layers, ids, targets) == 0
    layers.close()
    e.close()


def _wait_words(words, value, n, timeout=10.0):
    """The device words, once all of them hold `value` (written asynchronously
    by the load thread)."""
    t0 = time.monotonic()
    while True:
        got = words.buf.download().view(np.uint64)[:n]
        if (got == value).all() or time.monotonic() - t0 > timeout:
            return got.tolist()
        time.sleep(0.001)


def test_device_words_gate_consumer_per_layer(engine):
    """A layered load with the consumer's device words (same process): the
    engine's one marked launch writes word l as layer l lands; a consumer
    stream waits on each word and snapshots its layer, and every snapshot
    holds the restored bytes.  A failed load (unknown hash) and an empty load
    (every id negative) still write every word, so no device wait is left
    hanging; the LoadState tells them apart."""
    from pegaflow_amd.load_state import LayerWords
    from pegaflow_amd.runtime import Stream, memcpy_async

    say("[gpu] engine layer words: device-side per-layer gating")
    engine.set_transfer_modes(_lib.MODE_KERNEL, _lib.MODE_KERNEL)
    m = Model(engine, "words", 8, 256, 32768, seed=31)
    words = LayerWords(m.n_layers, local=True)
    flag = DeviceBuffer(4 * m.n_layers)
    snaps = [DeviceBuffer(m.size) for _ in range(m.n_layers)]
    stream = Stream()
    try:
        orig = m.host_copies()
        ids = list(range(0, 160, 2))
        hashes = [h(i, b"words") for i in ids]
        engine.batch_save_kv_blocks("words", 0, 0, [(n, ids, hashes) for n in m.names])
        targets = list(range(255, 95, -2))
        exp = expected_after_load(m, orig, ids, targets)
        for rnd in range(2):  # the same words serve consecutive loads
            for l, b in enumerate(m.bufs):
                b.fill_random(m.seeds[l])
            flag.memset(0)
            st = PyLoadState(layer_words=words)
            engine.batch_load_kv_blocks("words", 0, 0, st.shm_name(), m.names, targets, hashes)
            for l in range(m.n_layers):
                assert st.wait_for_layer_on_device(
                    l, lambda i: words.wait_on_device(stream, i, 20_000_000, flag.ptr + 4 * i))
                memcpy_async(snaps[l].ptr, m.bufs[l].ptr, m.size, stream)
            stream.synchronize()
            assert wait(st) == 1 and st.layers_done() == m.n_layers
            assert not flag.download().any(), f"round {rnd}: a device wait timed out"
            for l in range(m.n_layers):
                assert np.array_equal(snaps[l].download(), exp[l]), f"round {rnd} layer {l}"
        # Unknown hash: the call fails, the state says so, the words are written.
        st = PyLoadState(layer_words=words)
        with pytest.raises(_lib.PegaFlowError):
            engine.batch_load_kv_blocks("words", 0, 0, st.shm_name(), m.names, targets[:2],
                                        [hashes[0], h(10**6, b"words")])
        assert st.get_state() == -1
        assert _wait_words(words, words.value, m.n_layers) == [words.value] * m.n_layers
        # Nothing to copy: completed at once, words written.
        st = PyLoadState(layer_words=words)
        engine.batch_load_kv_blocks("words", 0, 0, st.shm_name(), m.names, [-1, -1],
                                    hashes[:2])
        assert wait(st) == 1
        assert _wait_words(words, words.value, m.n_layers) == [words.value] * m.n_layers
    finally:
        stream.close()
        for b in snaps:
            b.close()
        flag.close()
        words.close()
        m.close()


def test_local_layer_events_gate_consumer_per_layer(engine):
    """The engine's per-layer-event branch run in one process: the consumer
    puts one of its own events per layer in the LoadState (the in-process
    variant of the interprocess event block).  The load thread issues one
    launch per layer, records layer l's event after it, publishes
    events_recorded once every record is queued, then layers_done as the
    events fire.  A consumer stream waits on each event and snapshots its
    layer at once; every snapshot must hold the restored bytes.  The same
    events serve a second load; a failed load ends without a device wait."""
    from pegaflow_amd.runtime import Event, Stream, memcpy_async

    say("[gpu] engine local layer events: device-side per-layer gating")
    engine.set_transfer_modes(_lib.MODE_KERNEL, _lib.MODE_KERNEL)
    m = Model(engine, "levents", 8, 256, 32768, seed=37)
    evs = [Event() for _ in range(m.n_layers)]
    snaps = [DeviceBuffer(m.size) for _ in range(m.n_layers)]
    stream = Stream()
    try:
        orig = m.host_copies()
        ids = list(range(1, 161, 2))
        hashes = [h(i, b"levents") for i in ids]
        engine.batch_save_kv_blocks("levents", 0, 0, [(n, ids, hashes) for n in m.names])
        targets = list(range(254, 94, -2))
        exp = expected_after_load(m, orig, ids, targets)
        for rnd in range(2):
            for l, b in enumerate(m.bufs):
                b.fill_random(m.seeds[l])
            st = PyLoadState(num_layers=m.n_layers, layer_events=evs)
            assert st.inner.events_local()
            engine.batch_load_kv_blocks("levents", 0, 0, st.shm_name(), m.names, targets,
                                        hashes)
            for l in range(m.n_layers):
                assert st.wait_for_layer_on_device(l, lambda i: stream.wait_event(evs[i]))
                memcpy_async(snaps[l].ptr, m.bufs[l].ptr, m.size, stream)
            stream.synchronize()
            assert wait(st) == 1
            assert st.events_recorded() and st.layers_done() == m.n_layers
            for l in range(m.n_layers):
                assert np.array_equal(snaps[l].download(), exp[l]), f"round {rnd} layer {l}"
        # An unknown hash fails the call before any record: no device wait.
        st = PyLoadState(num_layers=m.n_layers, layer_events=evs)
        with pytest.raises(_lib.PegaFlowError):
            engine.batch_load_kv_blocks("levents", 0, 0, st.shm_name(), m.names, targets[:2],
                                        [hashes[0], h(10**6, b"levents")])
        calls = []
        assert not st.wait_for_layer_on_device(0, calls.append) and calls == []
    finally:
        stream.close()
        for s in snaps:
            s.close()
        m.close()


@pytest.mark.parametrize("mode", ["kernel", "staged"])
@pytest.mark.parametrize("completion", ["plain", "layered", "events"])
def test_split_load_matches_oracle(engine, completion, mode):
    """A load of 8 layers x 1024 split blocks (16384 chunks) is split: the
    lists of its first two layers are submitted while the others are built,
    and the transfer issues them once they are published.  Bytes against the
    oracle for each way the load thread publishes completion, by the kernel
    and staged (a load with per-layer events runs the kernel mode either
    way)."""
    from pegaflow_amd.runtime import Event, Stream

    say(f"[gpu] engine split load ({completion}, {mode})")
    engine.set_transfer_modes(_lib.MODE_KERNEL, _lib.MODE_NAMES[mode])
    m = Model(engine, "split", 8, 2100, 1024, seed=41)
    evs = [Event() for _ in range(m.n_layers)] if completion == "events" else None
    stream = Stream() if completion == "events" else None
    try:
        orig = m.host_copies()
        perm = np.random.default_rng(41).permutation(2100)
        ids, targets = [int(i) for i in perm[:1024]], [int(i) for i in perm[1024:2048]]
        hashes = [h(i, b"split") for i in ids]
        engine.batch_save_kv_blocks("split", 0, 0, [(n, ids, hashes) for n in m.names])
        exp = expected_after_load(m, orig, ids, targets)
        for l, b in enumerate(m.bufs):
            b.fill_random(m.seeds[l])
        if completion == "plain":
            st = PyLoadState()
        elif completion == "layered":
            st = PyLoadState(num_layers=m.n_layers)
        else:
            st = PyLoadState(num_layers=m.n_layers, layer_events=evs)
        engine.batch_load_kv_blocks("split", 0, 0, st.shm_name(), m.names, targets, hashes)
        if completion == "events":
            for l in range(m.n_layers):
                assert st.wait_for_layer_on_device(l, lambda i: stream.wait_event(evs[i]))
            stream.synchronize()
        assert wait(st) == 1
        if completion != "plain":
            assert st.layers_done() == m.n_layers
        got = m.host_copies()
        for l in range(m.n_layers):
            assert np.array_equal(got[l], exp[l]), f"layer {l}"
    finally:
        if stream is not None:
            stream.close()
        m.close()


@pytest.mark.parametrize("mode", ["kernel", "staged"])
def test_split_load_error_in_later_layers(engine, mode):
    """A split load whose later layer is registered with another block size
    than the stored blocks hold: the call fails with the size message after
    the first layer was submitted, the LoadState reads failed, the later
    layers' destinations are untouched and the load thread serves the next
    load (the first layer may have been copied already)."""
    say(f"[gpu] engine split load: error in a later layer ({mode})")
    engine.set_transfer_modes(_lib.MODE_KERNEL, _lib.MODE_NAMES[mode])
    a = Model(engine, "splita", 8, 2100, 2048, seed=43)
    b = odd = None
    try:
        ids = list(range(1024))
        hashes = [h(i, b"splite") for i in ids]
        engine.batch_save_kv_blocks("splita", 0, 0, [(n, ids, hashes) for n in a.names])
        # Instance b shares the namespace; its layer 7 holds 1024-byte halves.
        # With 4096-byte blocks the first part is layer 0 alone.
        b = Model(engine, "splitb", 7, 2100, 2048, seed=44, prefix="b", total_layers=8)
        odd = DeviceBuffer(2 * 2100 * 1024)
        odd.fill_random(45)
        engine.register_context_layer("splitb", "ns", 0, "b.7", odd.ptr, 2 * 2100 * 1024, 2100,
                                      1024, 2100 * 1024, 2, 0, 1, 8)
        names = b.names + ["b.7"]
        before = [x.download() for x in b.bufs[1:]] + [odd.download()]
        targets = list(range(1024, 2048))
        st = PyLoadState(num_layers=8)
        with pytest.raises(RuntimeError, match="holds 4096 split bytes for layer b.7, which is "
                                               "registered with 2048 split bytes"):
            engine.batch_load_kv_blocks("splitb", 0, 0, st.shm_name(), names, targets, hashes)
        assert wait(st) == -1
        after = [x.download() for x in b.bufs[1:]] + [odd.download()]
        assert all(np.array_equal(x, y) for x, y in zip(before, after))
        # The worker is free: a load of the matching layers completes, and so
        # does one that reports each layer (its marks count from 0 again).
        st = PyLoadState()
        engine.batch_load_kv_blocks("splitb", 0, 0, st.shm_name(), b.names, targets, hashes)
        assert wait(st) == 1
        st = PyLoadState(num_layers=len(b.names))
        engine.batch_load_kv_blocks("splitb", 0, 0, st.shm_name(), b.names, targets, hashes)
        assert wait(st) == 1
        assert st.layers_done() == len(b.names)
    finally:
        a.close()
        if b is not None:
            b.close()
        if odd is not None:
            odd.close()


@pytest.mark.parametrize("save_mode", ["kernel", "staged", "auto"])
def test_pipelined_save_matches_oracle(engine, save_mode):
    """A save of 8 layers x 1024 split blocks (16,384 chunks) is pipelined:
    the regions and lists of its first layers are made and their copy
    started before the others are made.  A first save of half the blocks,
    then a save of all of them (the saved half filtered out, so the kept
    lists differ from the ids); every block restored into other blocks
    equals the oracle's, and the store holds all 1024 blocks sealed."""
    say(f"[gpu] engine pipelined save ({save_mode})")
    engine.set_transfer_modes(_lib.MODE_NAMES[save_mode], _lib.MODE_KERNEL)
    m = Model(engine, "psave", 8, 2100, 1024, seed=51)
    try:
        orig = m.host_copies()
        perm = np.random.default_rng(51).permutation(2100)
        ids, targets = [int(i) for i in perm[:1024]], [int(i) for i in perm[1024:2048]]
        hashes = [h(i, b"psave") for i in ids]
        engine.batch_save_kv_blocks("psave", 0, 0,
                                    [(n, ids[::2], hashes[::2]) for n in m.names])
        engine.batch_save_kv_blocks("psave", 0, 0, [(n, ids, hashes) for n in m.names])
        assert engine.count_prefix_hit_blocks("psave", hashes) == 1024
        s = engine.stats()
        assert s["sealed_blocks"] == 1024 and s["inflight_blocks"] == 0
        st = PyLoadState()
        engine.batch_load_kv_blocks("psave", 0, 0, st.shm_name(), m.names, targets, hashes)
        assert wait(st) == 1
        exp = expected_after_load(m, orig, ids, targets)
        got = m.host_copies()
        for l in range(m.n_layers):
            assert np.array_equal(got[l], exp[l]), f"layer {l}"
    finally:
        m.close()


@pytest.mark.parametrize("save_mode", ["kernel", "staged"])
def test_pipelined_save_pool_exhausted_in_later_layer(gpu, save_mode):
    """A pipelined save whose pool holds its first layers' regions but not
    the rest: the call fails with the pool's message once the first
    layers' copy has drained, nothing is published, and a save that fits
    then completes and restores correctly."""
    say(f"[gpu] engine pipelined save, pool exhausted in a later layer ({save_mode})")
    e = PegaEngine(pool_size=5 * MiB)  # 2 MiB per layer of 1024 split 1 KiB blocks
    e.set_transfer_modes(_lib.MODE_NAMES[save_mode], _lib.MODE_KERNEL)
    m = Model(e, "pex", 8, 2100, 1024, seed=53)
    try:
        orig = m.host_copies()
        ids = list(range(1024))
        hashes = [h(i, b"pex") for i in ids]
        with pytest.raises(RuntimeError, match="pinned pool exhausted while allocating"):
            e.batch_save_kv_blocks("pex", 0, 0, [(n, ids, hashes) for n in m.names])
        s = e.stats()
        assert s["sealed_blocks"] == 0 and s["inflight_blocks"] == 0
        assert s["pool_used_bytes"] == 0
        assert e.count_prefix_hit_blocks("pex", hashes) == 0
        small, tg = ids[:200], list(range(1500, 1700))
        e.batch_save_kv_blocks("pex", 0, 0, [(n, small, hashes[:200]) for n in m.names])
        st = PyLoadState()
        e.batch_load_kv_blocks("pex", 0, 0, st.shm_name(), m.names, tg, hashes[:200])
        assert wait(st) == 1
        exp = expected_after_load(m, orig, small, tg)
        got = m.host_copies()
        for l in range(m.n_layers):
            assert np.array_equal(got[l], exp[l]), f"layer {l}"
    finally:
        m.close()
        e.close()


def test_tinylfu_admission_refuses_colder_blocks(gpu):
    """With TinyLFU admission on (set_storage_policy, cache.rs:71-95; a
    sketch sized wide through the value-size hint), a batch saved after the
    least recently used batch has been loaded twice is colder than it and is
    refused: its hashes are not counted, loading them fails, and the
    refusals are counted.  Saved twice more it is as warm and enters; every
    byte it loads then equals the oracle's.  Admission off: a colder batch
    enters at once."""
    say("[gpu] engine TinyLFU admission")
    e = PegaEngine(pool_size=64 * MiB)
    m = Model(e, "lfu", 2, 64, 4096, seed=61)
    try:
        e.set_storage_policy(lfu_admission=True, value_size_hint=4096)
        orig = m.host_copies()
        a_ids, b_ids = [1, 2, 3], [10, 11, 12]
        a_h, b_h = [h(i, b"lfuA") for i in a_ids], [h(i, b"lfuB") for i in b_ids]
        e.batch_save_kv_blocks("lfu", 0, 0, [(n, a_ids, a_h) for n in m.names])
        for _ in range(2):
            st = PyLoadState()
            e.batch_load_kv_blocks("lfu", 0, 0, st.shm_name(), m.names, [40, 41, 42], a_h)
            assert wait(st) == 1
        e.batch_save_kv_blocks("lfu", 0, 0, [(n, b_ids, b_h) for n in m.names])
        assert e.count_prefix_hit_blocks("lfu", b_h) == 0
        assert e.stats()["admission_rejections"] == 3
        st = PyLoadState()
        with pytest.raises(RuntimeError, match="missing KV block hash at index 0"):
            e.batch_load_kv_blocks("lfu", 0, 0, st.shm_name(), m.names, [50, 51, 52], b_h)
        assert st.get_state() == -1
        # Recorded on every offer: the third offer is as warm as batch A.
        e.batch_save_kv_blocks("lfu", 0, 0, [(n, b_ids, b_h) for n in m.names])
        assert e.count_prefix_hit_blocks("lfu", b_h) == 0
        e.batch_save_kv_blocks("lfu", 0, 0, [(n, b_ids, b_h) for n in m.names])
        assert e.count_prefix_hit_blocks("lfu", b_h) == 3
        assert e.stats()["admission_rejections"] == 6
        st = PyLoadState()
        e.batch_load_kv_blocks("lfu", 0, 0, st.shm_name(), m.names, [50, 51, 52], b_h)
        assert wait(st) == 1
        exp = expected_after_load(m, orig, a_ids, [40, 41, 42])
        exp = expected_after_load(m, exp, b_ids, [50, 51, 52])
        got = m.host_copies()
        for l in range(m.n_layers):
            assert np.array_equal(got[l], exp[l]), f"layer {l}"
        # Admission off: a new, colder batch enters at once.
        e.set_storage_policy(lfu_admission=False)
        c_h = [h(i, b"lfuC") for i in b_ids]
        e.batch_save_kv_blocks("lfu", 0, 0, [(n, b_ids, c_h) for n in m.names])
        assert e.count_prefix_hit_blocks("lfu", c_h) == 3
    finally:
        e.close()
        m.close()


def test_pre_eviction_keeps_free_space(gpu):
    """The pre-eviction monitor (storage.rs:646-688): once the pool's free
    bytes fall below the threshold, it evicts least-recently-used blocks
    until the target is free; the oldest batches go first and the newest
    stays loadable."""
    say("[gpu] engine pre-eviction")
    e = PegaEngine(pool_size=8 * MiB)
    m = Model(e, "pre", 2, 256, 4096, seed=62)
    try:
        # 8 batches of 16 blocks x 2 layers x 8 KiB = 256 KiB each: 2 MiB.
        batches = [([b * 16 + i for i in range(16)], [h(b * 16 + i, b"pre") for i in range(16)])
                   for b in range(8)]
        for ids, hs in batches:
            e.batch_save_kv_blocks("pre", 0, 0, [(n, ids, hs) for n in m.names])
        s = e.stats()
        free = s["pool_total_bytes"] - s["pool_used_bytes"]
        assert s["sealed_blocks"] == 128 and free < 7 * MiB
        e.set_storage_policy(pre_evict=True, pre_evict_threshold=7 * MiB,
                             pre_evict_target=7 * MiB + 512 * 1024, pre_evict_interval_ms=10)
        t0 = time.monotonic()
        while e.stats()["pre_evicted_blocks"] == 0:
            assert time.monotonic() - t0 < 10, "the monitor evicted nothing"
            time.sleep(0.01)
        time.sleep(0.05)
        e.set_storage_policy()  # stops the monitor
        s = e.stats()
        assert s["pool_total_bytes"] - s["pool_used_bytes"] >= 7 * MiB + 512 * 1024
        assert s["pre_evicted_blocks"] == s["evicted_blocks"] > 0
        assert e.count_prefix_hit_blocks("pre", batches[0][1]) == 0
        assert e.count_prefix_hit_blocks("pre", batches[-1][1]) == 16
        st = PyLoadState()
        e.batch_load_kv_blocks("pre", 0, 0, st.shm_name(), m.names,
                               list(range(200, 216)), batches[-1][1])
        assert wait(st) == 1
    finally:
        e.close()
        m.close()


def test_engine_on_cu_masked_contexts(gpu, monkeypatch):
    """PEGAFLOW_CUS_PER_XCD masks the contexts the engine creates: a save
    and a layer-by-layer load through them (staged, each slice's scatter on
    2 CUs per XCD) equal the oracle, every layer published."""
    say("[gpu] engine on CU-masked contexts")
    monkeypatch.setenv("PEGAFLOW_CUS_PER_XCD", "2")
    e = PegaEngine(pool_size=64 * MiB)
    m = Model(e, "cum", 4, 256, 8192, seed=63)
    try:
        orig = m.host_copies()
        ids = list(range(0, 200, 3))
        targets = list(range(1, 200, 3))
        hashes = [h(i, b"cum") for i in ids]
        e.batch_save_kv_blocks("cum", 0, 0, [(n, ids, hashes) for n in m.names])
        st = PyLoadState(num_layers=m.n_layers)
        e.batch_load_kv_blocks("cum", 0, 0, st.shm_name(), m.names, targets, hashes)
        assert wait(st) == 1 and st.layers_done() == m.n_layers
        exp = expected_after_load(m, orig, ids, targets)
        got = m.host_copies()
        for l in range(m.n_layers):
            assert np.array_equal(got[l], exp[l]), f"layer {l}"
    finally:
        e.close()
        m.close()
