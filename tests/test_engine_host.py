"""Host logic of the engine, without a GPU: the pool allocator (the
reference's allocator.rs tests plus a model check) and the engine's
registration / validation / lookup rules (lib.rs:303-484, 803-838) on an
engine whose pool is plain host memory."""

import ctypes

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from pegaflow_amd import _lib
from pegaflow_amd.engine import PegaEngine, ScaledOffsetAllocator, _block_ids, _hashes
from pegaflow_amd.load_state import PyLoadState

GiB = 1 << 30


# ---------------------------------------------------------------------------
# allocator.rs:183-238.
# ---------------------------------------------------------------------------
def test_creates_allocator_with_scaled_capacity():
    a = ScaledOffsetAllocator(10 * GiB, 64)
    assert a.unit_size == 64
    assert a.total_bytes == 10 * GiB  # 10 GiB / 64 units of 64 B


def test_allocate_rounds_up_to_unit_size():
    a = ScaledOffsetAllocator(1024, 64)
    assert a.allocate(1) == (0, 64)
    assert a.storage_report() == (960, 960)


def test_reuse_after_free_merges_neighboring_regions():
    a = ScaledOffsetAllocator(256, 64)
    x = a.allocate(64)
    y = a.allocate(64)
    a.free(x[0])
    a.free(y[0])
    assert a.allocate(128) == (0, 128)


def test_rejects_unreasonably_large_requests():
    a = ScaledOffsetAllocator(1024 * 1024, 1)
    with pytest.raises(_lib.PegaFlowError) as ei:
        a.allocate((2**32 - 1) * 2)
    assert ei.value.code == _lib.PF_ERR_INVALID_ARGUMENT
    assert "overflows u32 backing allocator" in str(ei.value)


def test_rejects_invalid_unit_size():
    with pytest.raises(_lib.PegaFlowError, match="unit size must be greater than zero"):
        ScaledOffsetAllocator(1024, 0)


def test_auto_unit_keeps_32_bit_units():
    # 30 GiB pool: smallest unit with <= u32::MAX units is 8 bytes (allocator.rs:77-86).
    assert ScaledOffsetAllocator(30 * GiB).unit_size == 8
    assert ScaledOffsetAllocator(4096).unit_size == 1
    assert ScaledOffsetAllocator(0).allocate(1) is None
    assert ScaledOffsetAllocator(4096).allocate(0) is None  # Ok(None) for zero bytes


@settings(max_examples=100, deadline=None)
@given(st.lists(st.tuples(st.booleans(), st.integers(1, 300)), max_size=60),
       st.sampled_from([1, 8, 64]))
def test_allocator_model(ops, unit):
    """Against a unit bitmap: allocations are unit-rounded, in range and never
    overlap; free-byte accounting is exact; freeing everything coalesces the
    whole region back into one."""
    total = 2048
    a = ScaledOffsetAllocator(total, unit)
    live = {}
    for is_alloc, size in ops:
        if is_alloc or not live:
            r = a.allocate(size)
            if r is None:
                continue
            off, got = r
            assert got == -(-size // unit) * unit and off % unit == 0 and off + got <= total
            for o2, g2 in live.items():
                assert off + got <= o2 or o2 + g2 <= off
            live[off] = got
        else:
            off = sorted(live)[size % len(live)]
            a.free(off)
            del live[off]
        free, largest = a.storage_report()
        assert free == a.total_bytes - sum(live.values())
        assert largest <= free
    for off in list(live):
        a.free(off)
    assert a.storage_report() == (a.total_bytes, a.total_bytes)


# ---------------------------------------------------------------------------
# Engine host logic (plain host pool, no transfers).
# ---------------------------------------------------------------------------
@pytest.fixture
def engine():
    e = PegaEngine(pool_size=64 << 20, host_pool=True)
    yield e
    e.close()


def reg(engine, layer="l0", inst="i0", ns="ns", device=0, tp_rank=0, tp_size=1, layers=2,
        nb=16, bpb=512, segments=2, ptr=0x10000):
    kv = nb * bpb if segments == 2 else 0
    size = kv + nb * bpb if segments == 2 else nb * bpb
    engine.register_context_layer(inst, ns, device, layer, ptr, size, nb, bpb, kv, segments,
                                  tp_rank, tp_size, layers)


def test_register_validation_messages(engine):
    with pytest.raises(RuntimeError, match="invalid KV cache layout for layer bad"):
        engine.register_context_layer("i", "ns", 0, "bad", 0x1000, 100, 0, 10, 10, 2, 0, 1, 1)
    with pytest.raises(RuntimeError, match="kv_stride_bytes must be > 0 when segments > 1"):
        engine.register_context_layer("i", "ns", 0, "bad", 0x1000, 100, 10, 10, 0, 2, 0, 1, 1)
    with pytest.raises(RuntimeError, match="device_id must be >= 0"):
        engine.register_context_layer("i", "ns", -1, "bad", 0x1000, 1000, 10, 10, 100, 2, 0, 1, 1)
    with pytest.raises(RuntimeError, match="registered memory too small"):
        engine.register_context_layer("i", "ns", 0, "bad", 0x1000, 199, 10, 10, 100, 2, 0, 1, 1)


def test_topology_mismatch_and_instances(engine):
    reg(engine, "l0")
    reg(engine, "l1")
    with pytest.raises(RuntimeError, match="topology mismatch: instance i0 exists with "
                                           "layers=2, tp=1; requested layers=3, tp=1") as ei:
        reg(engine, "l2", layers=3)
    assert ei.value.code == _lib.PF_ERR_TOPOLOGY_MISMATCH
    with pytest.raises(RuntimeError, match="instance nope not found"):
        engine.count_prefix_hit_blocks("nope", [b"a"])
    assert engine.count_prefix_hit_blocks("i0", [b"a", b"b"]) == 0
    assert engine.count_prefix_hit_blocks("i0", []) == 0
    engine.unregister_instance("i0")
    with pytest.raises(RuntimeError, match="instance i0 not found"):
        engine.unregister_instance("i0")


def test_save_errors_before_any_transfer(engine):
    reg(engine, "l0")
    with pytest.raises(RuntimeError, match="device 3 not found in instance i0"):
        engine.batch_save_kv_blocks("i0", 0, 3, [("l0", [0], [b"h"])])
    with pytest.raises(RuntimeError, match="layer zz unknown"):
        engine.batch_save_kv_blocks("i0", 0, 0, [("zz", [0], [b"h"])])
    with pytest.raises(RuntimeError, match="block 16 out of range for layer l0"):
        engine.batch_save_kv_blocks("i0", 0, 0, [("l0", [16], [b"h"])])
    with pytest.raises(RuntimeError, match="tp_rank 1 out of range"):
        engine.batch_save_kv_blocks("i0", 1, 0, [("l0", [1], [b"h"])])
    with pytest.raises(RuntimeError, match="does not match block_hashes"):
        engine.batch_save_kv_blocks("i0", 0, 0, [("l0", [1, 2], [b"h"])])
    # Negative ids only: nothing to save, no transfer needed.
    engine.batch_save_kv_blocks("i0", 0, 0, [("l0", [-1, -5], [b"a", b"b"])])
    # A real save needs a device-mapped pool.
    with pytest.raises(RuntimeError, match="not mapped for a device") as ei:
        engine.batch_save_kv_blocks("i0", 0, 0, [("l0", [1], [b"h"])])
    assert ei.value.code == _lib.PF_ERR_UNSUPPORTED
    assert engine.stats()["pool_used_bytes"] == 0  # the failed save released its regions


def test_save_marshalling(engine):
    """A save's layer array is built as pf_save_layer's 64-bit words: each
    layer reaches the engine with its own name, ids and hashes (the errors
    name the second layer), from lists or numpy ids; hashes of one length
    get arithmetic offsets, mixed lengths their running sums."""
    assert ctypes.sizeof(_lib.SaveLayer) == 40
    assert [getattr(_lib.SaveLayer, f).offset for f, _ in _lib.SaveLayer._fields_] == \
        [0, 8, 16, 24, 32]
    data, offs = _hashes([b"ab", b"cd", b"ef"])
    assert bytes(data) == b"abcdef" and offs.tolist() == [0, 2, 4, 6]
    data, offs = _hashes([b"a", b"bcd", b""])
    assert bytes(data) == b"abcd" and offs.tolist() == [0, 1, 4, 4]
    data, offs = _hashes([b"", b""])
    assert offs.tolist() == [0, 0, 0]
    data, offs = _hashes([])
    assert offs.tolist() == [0]
    for ids in ([3, -1, 7], np.array([3, -1, 7], np.int64)):
        keep, addr, n = _block_ids(ids)
        assert n == 3 and (ctypes.c_int32 * 3).from_address(addr)[:] == [3, -1, 7]
    reg(engine, "l0")
    reg(engine, "l1")
    with pytest.raises(RuntimeError, match="block 17 out of range for layer l1"):
        engine.batch_save_kv_blocks("i0", 0, 0, [("l0", [-1], [b"h"]),
                                                 ("l1", np.array([17]), [b"hh"])])
    with pytest.raises(RuntimeError, match="layer zz unknown"):
        engine.batch_save_kv_blocks("i0", 0, 0, [("l0", [-1, -2], [b"a", b"bcd"]),
                                                 ("zz", [0], [b"h"])])
    # Negative ids only, hashes of mixed lengths, and an empty batch: no copy.
    engine.batch_save_kv_blocks("i0", 0, 0, [("l0", np.array([-1, -2]), [b"a", b"bcd"]),
                                             ("l1", [-3], [b"xyz"])])
    engine.batch_save_kv_blocks("i0", 0, 0, [])
    assert engine.stats()["pool_used_bytes"] == 0


def test_load_errors_set_the_load_state(engine):
    reg(engine, "l0")
    st = PyLoadState()
    with pytest.raises(RuntimeError, match="missing KV block hash at index 0 "
                                           r"\(namespace=ns, hash_len=3\)"):
        engine.batch_load_kv_blocks("i0", 0, 0, st.shm_name(), ["l0"], [1], [b"abc"])
    assert st.get_state() == -1 and st.is_ready()
    st2 = PyLoadState()
    with pytest.raises(RuntimeError, match="instance zz not found"):
        engine.batch_load_kv_blocks("zz", 0, 0, st2.shm_name(), ["l0"], [1], [b"abc"])
    assert st2.get_state() == -1
    # Nothing to load: completes immediately (lib.rs:1055-1060).
    st3 = PyLoadState()
    engine.batch_load_kv_blocks("i0", 0, 0, st3.shm_name(), ["l0"], [], [])
    assert st3.get_state() == 1
    with pytest.raises(RuntimeError, match="failed to open shared memory"):
        engine.batch_load_kv_blocks("i0", 0, 0, "pega_load_does_not_exist", ["l0"], [], [])


def test_storage_policy_settings(engine):
    """set_storage_policy (StorageConfig, storage.rs:43-111): admission and
    the pre-eviction monitor turn on and off again; a monitor without an
    interval is refused; the stats carry their counters (0 on an engine
    that has stored nothing)."""
    engine.set_storage_policy(lfu_admission=True, value_size_hint=4096)
    engine.set_storage_policy(pre_evict=True, pre_evict_threshold=1 << 20,
                              pre_evict_target=2 << 20, pre_evict_interval_ms=5)
    with pytest.raises(RuntimeError, match="pre-eviction interval of 0 ms"):
        engine.set_storage_policy(pre_evict=True, pre_evict_interval_ms=0)
    engine.set_storage_policy()
    s = engine.stats()
    assert s["admission_rejections"] == 0 and s["pre_evicted_blocks"] == 0
