"""The disk tier on the CPU: the packed block format (seal_offload.rs:379-448,
869-909) pinned by a numpy brute-force fixture, and the engine's reader,
index, prefetch states (lib.rs:855-941) and quota over files built from that
fixture.  Writing needs saved blocks, hence a GPU (tests/test_disk_gpu.py).

The reference has no tests of this format; the fixture's expected file is
the array [block, slot, K|V, bytes] flattened (tests/golden/make_golden.py),
a formulation independent of the oracle's offset walk."""

import hashlib
import json
import os

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.engine import PegaEngine

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "packed_tiny.npz")
SPLIT_UUID = "00000000-0000-4000-8000-000000000001"
CONTIG_UUID = "00000000-0000-4000-8000-000000000002"


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


def h(i, salt=b"disk"):
    return hashlib.sha256(salt + int(i).to_bytes(8, "little")).digest()


def split_slots(g, ids):
    """Per block, per slot (layer * 2 + rank): (K, V) from the oracle's save path."""
    nb, bpb = 8, 32
    per_slot = []
    for l in range(2):
        for r in range(2):
            buf = g[f"split_input_{l}_{r}"].copy()
            reg = oracle.layout(buf.ctypes.data, buf.nbytes, nb, bpb, nb * bpb, 2)
            host = np.zeros(2 * len(ids) * bpb, np.uint8)
            k, v, split = oracle.save_host_layout(reg, len(ids), host.ctypes.data,
                                                  host.ctypes.data + len(ids) * bpb)
            assert split
            oracle.process_save(reg, buf, ids, k, v)
            per_slot.append([(host[j * bpb:(j + 1) * bpb].tobytes(),
                              host[(len(ids) + j) * bpb:(len(ids) + j + 1) * bpb].tobytes())
                             for j in range(len(ids))])
    return [[per_slot[s][j] for s in range(4)] for j in range(len(ids))]


def contig_slots(g, ids):
    buf = g["contig_input"].copy()
    reg = oracle.layout(buf.ctypes.data, buf.nbytes, 6, 64, 0, 1)
    host = np.zeros(len(ids) * 64, np.uint8)
    k, v, split = oracle.save_host_layout(reg, len(ids), host.ctypes.data, 0)
    assert not split
    oracle.process_save(reg, buf, ids, k, None)
    return [[(host[j * 64:(j + 1) * 64].tobytes(), None)] for j in range(len(ids))]


# ---------------------------------------------------------------------------
# The oracle against the fixture.
# ---------------------------------------------------------------------------
def test_oracle_pack_matches_fixture(g):
    ids = g["split_ids"].tolist()
    data, offs = oracle.pack_blocks(split_slots(g, ids))
    assert data == g["split_file"].tobytes()
    assert offs == g["split_offsets"].tolist()
    for j, off in enumerate(offs):
        assert oracle.block_meta_json(SPLIT_UUID + ".bin", off, [(True, 64)] * 4, 4) == \
            str(g["split_meta"][j])
    ids = g["contig_ids"].tolist()
    data, offs = oracle.pack_blocks(contig_slots(g, ids))
    assert data == g["contig_file"].tobytes()
    assert oracle.block_meta_json(CONTIG_UUID + ".bin", offs[1], [(False, 64)], 1) == \
        str(g["contig_meta"][1])


def test_planted_mistakes_fail_the_fixture(g):
    ids = g["split_ids"].tolist()
    blocks = split_slots(g, ids)
    want = g["split_file"].tobytes()
    kv_swapped = [[(v, k) for k, v in b] for b in blocks]
    rank_major = [[b[0], b[2], b[1], b[3]] for b in blocks]
    block_order = blocks[::-1]
    for wrong in (kv_swapped, rank_major, block_order):
        assert oracle.pack_blocks(wrong)[0] != want


@settings(max_examples=40, deadline=None)
@given(st.lists(st.lists(st.tuples(st.integers(1, 40), st.booleans()), min_size=3, max_size=3),
                min_size=1, max_size=5), st.integers(0, 2**32))
def test_unpack_inverts_pack(shape, seed):
    rng = np.random.default_rng(seed)
    blocks = [[(rng.bytes(n), rng.bytes(n) if split else None) for n, split in b] for b in shape]
    data, offs = oracle.pack_blocks(blocks)
    ends = offs[1:] + [len(data)]
    for b, (o, e) in enumerate(zip(offs, ends)):
        metas = [(v is not None, len(k) * (2 if v is not None else 1)) for k, v in blocks[b]]
        assert oracle.unpack_block(data[o:e], metas) == blocks[b]


# ---------------------------------------------------------------------------
# The engine's reader over fixture files.
# ---------------------------------------------------------------------------
def write_packed(root, ns_dir, namespace, uuid, file_bytes, metas, hashes, mtime=None):
    d = os.path.join(root, ns_dir)
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, uuid + ".bin"), "wb") as f:
        f.write(file_bytes)
    side = {"version": 1, "namespace": namespace, "file": uuid + ".bin", "size": len(file_bytes),
            "blocks": [{"hash": hh.hex(), "meta": json.loads(m)} for hh, m in zip(hashes, metas)]}
    p = os.path.join(d, uuid + ".json")
    with open(p, "w") as f:
        json.dump(side, f)
    if mtime is not None:
        os.utime(p, (mtime, mtime))


@pytest.fixture
def golden_root(tmp_path, g):
    root = str(tmp_path / "pega")
    hs = [h(i) for i in range(3)]
    write_packed(root, "llama", "llama", SPLIT_UUID, g["split_file"].tobytes(),
                 [str(m) for m in g["split_meta"]], hs)
    write_packed(root, "ns-612f62", "a/b", CONTIG_UUID, g["contig_file"].tobytes(),
                 [str(m) for m in g["contig_meta"]], [h(10), h(11)])
    return root, hs


def engine_on(root, pool=64 << 20, **kw):
    e = PegaEngine(pool_size=pool, host_pool=True)
    e.enable_disk(root, **kw)
    return e


def reg(e, inst, ns, layers, tp, nb=8, bpb=32, segments=2):
    size = 2 * nb * bpb if segments == 2 else nb * bpb
    e.register_context_layer(inst, ns, 0, "l0", 0x10000, size, nb, bpb,
                             nb * bpb if segments == 2 else 0, segments, 0, tp, layers)


def test_engine_indexes_and_prefetches_fixture_files(golden_root, g):
    root, hs = golden_root
    e = engine_on(root)
    s = e.disk_stats()
    assert (s["files"], s["indexed_blocks"], s["failures"]) == (2, 5, 0)
    assert s["bytes"] == g["split_file"].nbytes + g["contig_file"].nbytes
    reg(e, "vllm", "llama", 2, 2)
    q = e.count_prefix_hit_blocks_with_prefetch("vllm", hs)
    assert q["prefetch_state"] == "loading" and (q["hit_blocks"], q["loading_blocks"]) == (0, 3)
    e.wait_prefetch()
    q = e.count_prefix_hit_blocks_with_prefetch("vllm", hs)
    assert q == {"prefetch_state": "ready", "state": 0, "hit_blocks": 3, "loading_blocks": 0,
                 "missing_blocks": 0}
    assert e.count_prefix_hit_blocks("vllm", hs) == 3
    want = split_slots(g, g["split_ids"].tolist())
    for b in range(3):
        for slot in range(4):
            assert e.read_block_slot("llama", hs[b], slot) == want[b][slot]
    s = e.disk_stats()
    assert s["prefetched_blocks"] == 3 and s["read_bytes"] == g["split_file"].nbytes
    # The contiguous namespace lives in an escaped directory.
    reg(e, "other", "a/b", 1, 1, nb=6, bpb=64, segments=1)
    e.count_prefix_hit_blocks_with_prefetch("other", [h(10), h(11)])
    e.wait_prefetch()
    want = contig_slots(g, g["contig_ids"].tolist())
    assert e.read_block_slot("a/b", h(11), 0) == (want[1][0][0], b"")
    e.close()


def test_prefetch_of_page_sized_slots(tmp_path):
    """Blocks whose slot halves are 4 KiB (as a bf16 head of 16 tokens x 128
    dims is), packed by the oracle: five adjacent blocks are one read run
    into five pool allocations, and every slot holds the file's bytes."""
    rng = np.random.default_rng(7)
    seg, n_blocks, n_slots = 4096, 5, 2
    blocks = [[(rng.bytes(seg), rng.bytes(seg)) for _ in range(n_slots)]
              for _ in range(n_blocks)]
    data, offs = oracle.pack_blocks(blocks)
    assert all(o % 4096 == 0 for o in offs)
    uuid = "00000000-0000-4000-8000-000000000003"
    metas = [json.dumps({"file": uuid + ".bin", "offset": o,
                         "slots": [{"is_split": True, "size": 2 * seg}] * n_slots,
                         "total_slots": n_slots}, separators=(",", ":")) for o in offs]
    hs = [h(i, b"aligned") for i in range(n_blocks)]
    root = str(tmp_path / "pega")
    write_packed(root, "llama", "llama", uuid, data, metas, hs)
    e = engine_on(root)
    reg(e, "vllm", "llama", 2, 1, nb=8, bpb=seg)
    q = e.count_prefix_hit_blocks_with_prefetch("vllm", hs)
    assert q["prefetch_state"] == "loading"
    e.wait_prefetch()
    assert e.count_prefix_hit_blocks("vllm", hs) == n_blocks
    for b in range(n_blocks):
        for slot in range(n_slots):
            assert e.read_block_slot("llama", hs[b], slot) == blocks[b][slot]
    s = e.disk_stats()
    assert (s["prefetched_blocks"], s["read_bytes"], s["failures"]) == (n_blocks, len(data), 0)
    e.close()


def test_query_states_follow_the_reference(golden_root):
    root, hs = golden_root
    e = engine_on(root)
    reg(e, "vllm", "llama", 2, 2)
    # First miss not on disk: partial miss, nothing read (lib.rs:905-921).
    q = e.count_prefix_hit_blocks_with_prefetch("vllm", [h(99)] + hs)
    assert (q["prefetch_state"], q["hit_blocks"], q["missing_blocks"]) == ("partial_miss", 0, 4)
    assert e.disk_stats()["pending_blocks"] == 0
    # The rest of the prefix is read, skipping what is not on disk.
    q = e.count_prefix_hit_blocks_with_prefetch("vllm", [hs[0], h(99), hs[2]])
    assert (q["prefetch_state"], q["loading_blocks"]) == ("loading", 3)
    e.wait_prefetch()
    q = e.count_prefix_hit_blocks_with_prefetch("vllm", [hs[0], h(99), hs[2]])
    assert (q["prefetch_state"], q["hit_blocks"], q["missing_blocks"]) == ("partial_miss", 1, 2)
    assert e.count_prefix_hit_blocks("vllm", [hs[2]]) == 1
    # Other namespaces see nothing.
    reg(e, "x", "elsewhere", 2, 2)
    q = e.count_prefix_hit_blocks_with_prefetch("x", hs)
    assert q["prefetch_state"] == "partial_miss" and q["missing_blocks"] == 3
    with pytest.raises(RuntimeError, match="instance nope not found"):
        e.count_prefix_hit_blocks_with_prefetch("nope", hs)
    e.close()


def test_without_a_disk_tier_the_query_is_the_plain_count():
    e = PegaEngine(pool_size=1 << 20, host_pool=True)
    reg(e, "i", "ns", 2, 2)
    assert e.count_prefix_hit_blocks_with_prefetch("i", [h(0)]) == {
        "prefetch_state": "ready", "state": 0, "hit_blocks": 0, "loading_blocks": 0,
        "missing_blocks": 0}
    assert e.disk_stats()["files"] == 0
    e.close()


def test_bad_sidecars_are_skipped(tmp_path, g):
    root = str(tmp_path / "pega")
    data = g["split_file"].tobytes()
    metas = [str(m) for m in g["split_meta"]]
    u = "00000000-0000-4000-8000-0000000000%02d"
    write_packed(root, "ns", "ns", u % 1, data, metas, [h(0), h(1), h(2)])  # fine
    write_packed(root, "ns", "ns", u % 2, data[:-1], metas, [h(3), h(4), h(5)])  # short file
    d = os.path.join(root, "ns")
    with open(os.path.join(d, (u % 3) + ".json"), "w") as f:
        f.write("{not json")
    write_packed(root, "ns", "ns", u % 4, data, metas, [h(6), h(7), h(8)])
    side = os.path.join(d, (u % 4) + ".json")  # metas name another file
    e = engine_on(root)
    s = e.disk_stats()
    assert s["files"] == 1 and s["indexed_blocks"] == 3 and s["failures"] == 3
    e.close()
    assert os.path.exists(side)  # skipped, never deleted


def test_quota_drops_the_oldest_files_first(tmp_path, g):
    root = str(tmp_path / "pega")
    data = g["contig_file"].tobytes()
    metas = [str(m) for m in g["contig_meta"]]
    old, new = CONTIG_UUID, "00000000-0000-4000-8000-000000000003"
    write_packed(root, "ns", "ns", old, data, metas, [h(0), h(1)], mtime=1_000_000)
    metas_new = [m.replace(CONTIG_UUID, new) for m in metas]
    write_packed(root, "ns", "ns", new, data, metas_new, [h(1), h(2)], mtime=2_000_000)
    e = engine_on(root, quota_bytes=len(data))
    s = e.disk_stats()
    assert (s["files"], s["evicted_files"], s["indexed_blocks"]) == (1, 1, 2)
    assert not os.path.exists(os.path.join(root, "ns", old + ".bin"))
    assert os.path.exists(os.path.join(root, "ns", new + ".bin"))
    reg(e, "i", "ns", 1, 1, nb=6, bpb=64, segments=1)
    q = e.count_prefix_hit_blocks_with_prefetch("i", [h(0)])
    assert q["prefetch_state"] == "partial_miss"
    e.count_prefix_hit_blocks_with_prefetch("i", [h(1), h(2)])
    e.wait_prefetch()
    assert e.count_prefix_hit_blocks("i", [h(1), h(2)]) == 2
    e.close()


def test_prefetch_that_does_not_fit_the_pool_fails_cleanly(golden_root):
    root, hs = golden_root
    e = engine_on(root, pool=256)  # one unit: no 256-byte block fits with the others
    reg(e, "vllm", "llama", 2, 2)
    e.count_prefix_hit_blocks_with_prefetch("vllm", hs)
    e.wait_prefetch()
    s = e.disk_stats()
    assert s["prefetched_blocks"] + s["failures"] == 3 and s["pending_blocks"] == 0
    assert e.stats()["pool_used_bytes"] <= 256
    e.close()


def test_enable_disk_errors(tmp_path):
    e = PegaEngine(pool_size=1 << 20, host_pool=True)
    with pytest.raises(RuntimeError, match="empty disk root") as ei:
        e.enable_disk("")
    assert ei.value.code == _lib.PF_ERR_INVALID_ARGUMENT
    blocker = tmp_path / "file"
    blocker.write_text("x")
    with pytest.raises(RuntimeError, match="cannot create disk root"):
        e.enable_disk(str(blocker / "sub"))
    e.enable_disk(str(tmp_path / "ok"))
    with pytest.raises(RuntimeError, match="already enabled"):
        e.enable_disk(str(tmp_path / "ok"))
    with pytest.raises(RuntimeError, match="block not cached"):
        e.read_block_slot("ns", b"nope", 0)
    e.close()


def test_query_rpc_reports_prefetch(golden_root):
    """service.rs:258-330 over the wire: loading while the disk read runs,
    then ready."""
    from pegaflow_amd import ipc
    from pegaflow_amd.rpc.client import EngineRpcClient
    from pegaflow_amd.rpc.server import Server

    root, hs = golden_root
    srv = Server("127.0.0.1:0", engine=PegaEngine(pool_size=64 << 20, host_pool=True),
                 dfs_root=root).start()
    try:
        with EngineRpcClient(f"http://{srv.addr}") as c:
            assert c.register_context("vllm", "llama", 0, 2, 0, 2, "l0",
                                      ipc.local_tensor(0x10000, 512, 0), 8, 32, 256, 2)[0]
            q = c.query("vllm", hs)
            assert (q["prefetch_state"], q["loading_blocks"]) == ("loading", 3)
            srv.engine.wait_prefetch()
            q = c.query("vllm", hs)
            assert (q["prefetch_state"], q["hit_blocks"]) == ("ready", 3)
            q = c.query("vllm", [h(77)])
            assert (q["prefetch_state"], q["missing_blocks"]) == ("partial_miss", 1)
    finally:
        srv.stop()
