"""The C-ABI library: loads, exports every declared symbol, and its host-side
logic (layout validation, segment offsets, run merging, LoadState) agrees
with the oracle and the reference's own unit tests.  No GPU calls here."""

import ctypes
import os
import re
import struct

import pytest
from hypothesis import given, settings, strategies as st

import oracle
from pegaflow_amd import _lib
from pegaflow_amd.load_state import LoadState, PyLoadState
from pegaflow_amd.transfer import (KVCacheRegistration, count_merged_runs, derive_layout,
                                   is_contiguous_layout, segment_offset)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pegaflow_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pf_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = declared_symbols()
    assert len(syms) > 50
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    unbound = [s for s in syms if s not in _lib.SIGNATURES]
    assert not unbound, unbound
    assert lib.pf_version().decode().startswith("pegaflow_hip")


def test_library_is_gfx950_build():
    with open(_lib.LIB_PATH, "rb") as fh:
        blob = fh.read()
    assert b"gfx950" in blob


def _reg(*args):
    return KVCacheRegistration.create(*args)


@settings(max_examples=300, deadline=None)
@given(st.integers(0, 2**40), st.integers(0, 2**36), st.integers(0, 3000),
       st.integers(0, 70000), st.integers(0, 2**31), st.integers(0, 3))
def test_layout_init_matches_oracle(ptr, size, nb, bpb, stride, segs):
    try:
        expect = oracle.layout(ptr, size, nb, bpb, stride, segs)
    except oracle.OracleError:
        expect = None
    try:
        got = _reg(ptr, size, nb, bpb, stride, segs)
    except _lib.PegaFlowError as e:
        assert e.code == _lib.PF_ERR_INVALID_ARGUMENT
        got = None
    assert (expect is None) == (got is None)
    if got is not None:
        assert got.block_size_bytes == expect.block_size_bytes
        assert got.size_bytes == expect.size_bytes


@settings(max_examples=300, deadline=None)
@given(st.integers(1, 5000), st.integers(1, 70000), st.integers(0, 3), st.integers(1, 2),
       st.integers(0, 6000), st.integers(0, 2))
def test_segment_offset_matches_oracle(nb, bpb, pad, segs, block, seg):
    stride = (nb + pad) * bpb if segs == 2 else 0
    size = stride + nb * bpb
    o = oracle.layout(0, size, nb, bpb, stride, segs)
    r = _reg(0, size, nb, bpb, stride, segs)
    try:
        expect = oracle.segment_offset(o, block, seg)
    except oracle.OracleError as e:
        expect = str(e)
    try:
        got = segment_offset(r, block, seg)
    except _lib.PegaFlowError as e:
        got = str(e).split("storage error: ", 1)[1]
    assert got == expect
    assert is_contiguous_layout(r) == oracle.is_contiguous(o)
    assert r.kind == oracle.layout_kind(o)


@settings(max_examples=200, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 3), st.integers(0, 3)), max_size=50))
def test_merged_runs_match_oracle(steps):
    seg = 64
    g, c, x, y = [], [], 0, 10**6
    for dg, dc in steps:
        x += dg * seg
        y += dc * seg
        g.append(x)
        c.append(y)
    assert count_merged_runs(g, c, seg) == len(oracle.merge_runs(g, c, seg))


def test_derive_layout_rules():
    # worker.py:104-115 on vLLM's KV-first [2, nb, bs, h, d] bf16 tensor.
    shape = (2, 20000, 16, 8, 128)
    stride = (20000 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128, 128, 1)
    assert derive_layout(shape, stride, 2) == (20000, 32768, 655_360_000, 2)
    # Blocks-first MLA latent [8192, 64, 576].
    assert derive_layout((8192, 64, 576), (64 * 576, 576, 1), 1) == (8192, 36864, 0, 1)
    # A blocks-first tensor whose first dimension happens to be 2 is taken as
    # KV-first, exactly as the reference does.
    assert derive_layout((2, 64, 576), (64 * 576, 576, 1), 2)[3] == 2
    with pytest.raises(ValueError):
        derive_layout((4, 0), (0, 1), 2)


def test_derive_layout_from_torch_tensor():
    torch = pytest.importorskip("torch")
    t = torch.empty((2, 12, 16, 4, 64), dtype=torch.float16)
    assert derive_layout(t.shape, t.stride(), t.element_size()) == (12, 16 * 4 * 64 * 2,
                                                                    12 * 16 * 4 * 64 * 2, 2)


def test_error_message_is_per_call():
    with pytest.raises(_lib.PegaFlowError, match="kv_stride_bytes must be > 0"):
        _reg(0, 1000, 10, 10, 0, 2)
    assert "kv_stride" in _lib.last_error()


# ---------------------------------------------------------------------------
# LoadState (sync_state.rs:294-340 tests plus the byte layout of :19-43).
# ---------------------------------------------------------------------------
def test_load_state_round_trip():
    st_ = LoadState.new()
    assert st_.get() == 0
    name = st_.shm_name()
    assert re.fullmatch(r"pega_load_[0-9a-f]{32}", name)
    st_.set_completed()
    att = LoadState.attach(name)
    assert att.get() == 1
    att.set_error()
    assert st_.get() == -1
    att.close()
    st_.close()
    assert not os.path.exists("/dev/shm/" + name)


def test_load_state_byte_layout_matches_reference():
    st_ = LoadState.new()
    path = "/dev/shm/" + st_.shm_name()
    raw = open(path, "rb").read()
    assert len(raw) == 32
    off, = struct.unpack_from("<Q", raw, 0)
    assert off == 8
    magic, version, state = struct.unpack_from("<IIq", raw, off)
    assert (magic, version, state) == (0x50464C44, 1, 0)
    st_.set_completed()
    assert struct.unpack_from("<q", open(path, "rb").read(), off + 8)[0] == 1
    st_.close()


def _make_shm(name, data: bytes):
    fd = os.open("/dev/shm/" + name, os.O_CREAT | os.O_RDWR, 0o600)
    os.write(fd, data)
    os.close(fd)


def test_load_state_attach_rejects_too_small_mapping():
    name = "pega_test_small_" + os.urandom(8).hex()
    _make_shm(name, b"\0")
    try:
        with pytest.raises(_lib.PegaFlowError, match="shared memory too small"):
            LoadState.attach(name)
    finally:
        os.unlink("/dev/shm/" + name)


def test_load_state_attach_rejects_invalid_header():
    st_ = LoadState.new()
    path = "/dev/shm/" + st_.shm_name()
    with open(path, "r+b") as fh:
        fh.seek(8)
        fh.write(struct.pack("<I", 0xDEADBEEF))
    with pytest.raises(_lib.PegaFlowError, match="invalid LoadState header"):
        LoadState.attach(st_.shm_name())
    st_.close()


def test_load_state_reads_a_reference_written_mapping():
    # A mapping laid out by the reference's init_new_mapping (offset 8).
    name = "pega_load_" + os.urandom(16).hex()
    _make_shm(name, struct.pack("<QIIq", 8, 0x50464C44, 1, -1) + b"\0" * 8)
    try:
        st_ = LoadState.attach(name)
        assert st_.get() == -1 and st_.num_layers() == 0
        st_.close()
    finally:
        os.unlink("/dev/shm/" + name)


def test_layered_load_state():
    p = PyLoadState(num_layers=36)
    assert p.get_state() == 0 and not p.is_ready() and p.layers_done() == 0
    srv = LoadState.attach(p.shm_name())
    assert srv.num_layers() == 36
    srv.set_layers_done(5)
    assert p.layers_done() == 5
    assert p.wait_for_layer(4, timeout_s=1.0)
    assert not p.wait_for_layer(5, timeout_s=0.01)
    srv.set_completed()
    assert p.is_ready() and p.get_state() == 1 and p.layers_done() == 36
    # The first 32 bytes keep the reference's record.
    raw = open("/dev/shm/" + p.shm_name(), "rb").read()
    assert len(raw) == 48
    assert struct.unpack_from("<QIIq", raw, 0) == (8, 0x50464C44, 1, 1)
    assert struct.unpack_from("<IIq", raw, 32) == (0x50464C58, 36, 36)
    srv.close()


def test_pinned_zero_size_rejected_without_device():
    # pinned_mem.rs:285-288: zero size fails before any driver call.
    h, d = ctypes.c_void_p(), ctypes.c_uint64()
    rc = _lib.load().pf_pinned_allocate(0, 0, ctypes.byref(h), ctypes.byref(d))
    assert rc == _lib.PF_ERR_ZERO_SIZE


def test_huge_page_size_parse():
    # pinned_mem.rs:291-306: Hugepagesize is present on Linux and a power of two.
    from pegaflow_amd.runtime import huge_page_size
    size = huge_page_size()
    assert size >= 2 * 1024 * 1024 and size & (size - 1) == 0


def test_xcd_major_remap_is_a_bijection():
    """The load kernel's tile order (tile_of in pf_kernels.hip): workgroup b
    runs on XCD b mod 8 and takes tile x*q + min(x, r) + i.  It must visit
    every tile of [0, n) exactly once, with XCD x owning one contiguous range
    of q or q+1 tiles, for every tile count up to 1024 and some large ones
    (the Llama gather has 40960 tiles)."""
    for n in list(range(1, 1025)) + [4096, 4097, 40960, 40967]:
        q, r = n >> 3, n & 7
        seen = bytearray(n)
        owner = [[] for _ in range(8)]
        for b in range(n):
            x, i = b & 7, b >> 3
            t = x * q + min(x, r) + i
            assert 0 <= t < n and not seen[t], (n, b, t)
            seen[t] = 1
            owner[x].append(t)
        for x in range(8):
            ts = owner[x]
            assert ts == list(range(ts[0], ts[0] + len(ts))) if ts else True
            assert len(ts) == q + (1 if x < r else 0)


def test_load_state_event_block_layout():
    """The optional block of per-layer event handles after the layered
    extension: {'PFLE', count, events_recorded} at byte 48, handles at 64."""
    from pegaflow_amd.load_state import LoadState, PyLoadState

    handles = [bytes([7 + i]) * 64 for i in range(5)]
    p = PyLoadState(num_layers=5, layer_events=handles)
    raw = open("/dev/shm/" + p.shm_name(), "rb").read()
    assert len(raw) == 64 + 5 * 64
    assert struct.unpack_from("<QIIq", raw, 0) == (8, 0x50464C44, 1, 0)
    assert struct.unpack_from("<IIq", raw, 32) == (0x50464C58, 5, 0)
    assert struct.unpack_from("<IIq", raw, 48) == (0x50464C45, 5, 0)
    assert raw[64:] == b"".join(handles)
    srv = LoadState.attach(p.shm_name())
    assert srv.event_handles() == handles and not p.events_recorded()
    calls = []
    # Nothing recorded and the load finished (nothing to load): no device wait.
    srv.set_completed()
    assert p.wait_for_layer_on_device(2, calls.append) and calls == []
    srv.set_events_recorded(5)
    assert p.events_recorded()
    assert p.wait_for_layer_on_device(2, calls.append) and calls == [2]
    srv.close()
    # A failed load ends the wait without a device wait.
    q = PyLoadState(num_layers=2, layer_events=handles[:2])
    LoadState.attach(q.shm_name()).set_error()
    assert not q.wait_for_layer_on_device(0, calls.append) and calls == [2]
    # Plain and layered states carry no handles; mismatched lists are refused.
    assert LoadState.attach(PyLoadState(num_layers=3).shm_name()).event_handles() == []
    with pytest.raises(ValueError):
        PyLoadState(num_layers=3, layer_events=handles[:2])


def _words_record(kind, value, address=0, alloc_size=0, offset=0, handle=b""):
    w = _lib.LayerWords()
    w.kind, w.value, w.address, w.alloc_size, w.offset = kind, value, address, alloc_size, offset
    ctypes.memmove(w.handle, handle.ljust(64, b"\0"), 64)
    return w


class _HostWords:
    """Stands in for LayerWords (which needs device memory): the record only."""

    def __init__(self, num_layers, record):
        self.num_layers, self._record = num_layers, record

    def next_load(self):
        return self._record


def test_load_state_words_block_layout():
    """The optional block of layer words after the layered extension, at byte
    48: {'PFLW', count, value, kind, 0, address, alloc_size, offset, handle}."""
    handle = bytes(range(64))
    rec = _words_record(_lib.LAYER_WORDS_IPC, 9, alloc_size=1 << 21, offset=512, handle=handle)
    p = PyLoadState(layer_words=_HostWords(6, rec))
    raw = open("/dev/shm/" + p.shm_name(), "rb").read()
    assert len(raw) == 48 + 112
    assert struct.unpack_from("<QIIq", raw, 0) == (8, 0x50464C44, 1, 0)
    assert struct.unpack_from("<IIq", raw, 32) == (0x50464C58, 6, 0)
    assert struct.unpack_from("<IIQIIQQQ", raw, 48) == (0x50464C57, 6, 9, 0, 0, 0, 1 << 21, 512)
    assert raw[96:160] == handle
    srv = LoadState.attach(p.shm_name())
    w, n = srv.layer_words()
    assert n == 6 and w.value == 9 and w.kind == 0 and w.offset == 512
    assert bytes(w.handle) == handle and srv.event_handles() == []
    # Words need no "recorded" handshake: the wait is queued at once...
    calls = []
    assert p.wait_for_layer_on_device(4, calls.append) and calls == [4]
    # ...and not at all once the load has failed.
    srv.set_error()
    assert not p.wait_for_layer_on_device(1, calls.append) and calls == [4]
    srv.close()
    # A local record keeps its address; states without words report none.
    q = PyLoadState(layer_words=_HostWords(2, _words_record(_lib.LAYER_WORDS_LOCAL, 1,
                                                            address=0x7000)))
    w, n = LoadState.attach(q.shm_name()).layer_words()
    assert n == 2 and w.kind == 1 and w.address == 0x7000
    assert LoadState.attach(PyLoadState(num_layers=3).shm_name()).layer_words() == (None, 0)
    ev = PyLoadState(num_layers=1, layer_events=[b"\1" * 64])
    assert LoadState.attach(ev.shm_name()).layer_words() == (None, 0)


@pytest.mark.parametrize("rec,n", [
    (dict(kind=0, value=0, alloc_size=4096), 2),          # value 0
    (dict(kind=0, value=1, alloc_size=4096, offset=4), 2),  # misaligned
    (dict(kind=0, value=1, alloc_size=16, offset=8), 2),  # past the allocation
    (dict(kind=1, value=1, address=0x1004), 2),           # misaligned address
    (dict(kind=2, value=1, address=0x1000), 2),           # unknown kind
    (dict(kind=1, value=1, address=0x1000), 0),           # no layers
])
def test_load_state_words_block_rejects(rec, n):
    with pytest.raises(_lib.PegaFlowError):
        LoadState.new(n, None, _words_record(**rec))
