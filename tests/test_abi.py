"""The C-ABI library: loads, exports every declared symbol, and its host-side
logic (layout validation, segment offsets, run merging, LoadState) agrees
with the oracle and the reference's own unit tests.  No GPU calls here."""

import ctypes
import os
import re
import struct

import numpy as np
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


def header_constants():
    """Every integer #define and enum value of the header, by name."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    raw = dict(re.findall(r"^#define (PF_[A-Z0-9_]+) (.+)$", text, flags=re.M))
    raw.update(re.findall(r"(PF_[A-Z0-9_]+) = (-?[^,}\n]+)", text))
    values = {}
    for _ in range(4):  # definitions that use other definitions
        for name, expr in raw.items():
            e = re.sub(r"(0x[0-9a-fA-F]+|\d+)(ull|u)\b", r"\1", expr.strip())
            e = re.sub(r"PF_[A-Z0-9_]+", lambda m: str(values.get(m.group(0), "?")), e)
            if re.fullmatch(r"-?[0-9a-fx()|<+ ]+", e):
                values[name] = eval(e)  # digits and | << + only
    return values


def test_python_constants_match_the_header():
    values = header_constants()
    assert len(values) > 60, sorted(values)
    checked = 0
    for name, value in values.items():
        for attr in (name, name[3:]):
            if hasattr(_lib, attr) and isinstance(getattr(_lib, attr), int):
                assert getattr(_lib, attr) == value, (attr, getattr(_lib, attr), value)
                checked += 1
    assert checked > 30
    assert _lib.STAGED_HEAD_ENGINE == values["PF_STAGED_HEAD_ENGINE"]


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


def test_load_state_local_event_block_layout():
    """The in-process variant of the event block: {'PFLL', count,
    events_recorded} at byte 48, then per layer a 64-byte slot holding the
    event's address and zeros; an attacher sees it as local."""
    from types import SimpleNamespace

    from pegaflow_amd.load_state import LoadState, PyLoadState

    evs = [SimpleNamespace(handle=0x7F0000001000 + 0x40 * i) for i in range(3)]
    p = PyLoadState(num_layers=3, layer_events=evs)
    raw = open("/dev/shm/" + p.shm_name(), "rb").read()
    assert len(raw) == 64 + 3 * 64
    assert struct.unpack_from("<IIq", raw, 32) == (0x50464C58, 3, 0)
    assert struct.unpack_from("<IIq", raw, 48) == (0x50464C4C, 3, 0)
    for i, e in enumerate(evs):
        slot = raw[64 + 64 * i: 128 + 64 * i]
        assert struct.unpack_from("<Q", slot)[0] == e.handle and slot[8:] == bytes(56)
    srv = LoadState.attach(p.shm_name())
    assert srv.events_local() and p.inner.events_local()
    assert len(srv.event_handles()) == 3
    srv.set_events_recorded(3)
    calls = []
    assert p.wait_for_layer_on_device(1, calls.append) and calls == [1]
    srv.close()
    # An IPC event block is not local; a null event is refused.
    q = PyLoadState(num_layers=1, layer_events=[b"\x01" * 64])
    assert not LoadState.attach(q.shm_name()).events_local()
    with pytest.raises(_lib.PegaFlowError, match="null event for layer 1"):
        PyLoadState(num_layers=2, layer_events=[evs[0], SimpleNamespace(handle=0)])


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


# ---------------------------------------------------------------------------
# The transfer.rs primitives' error paths, which return before any HIP call.
# ---------------------------------------------------------------------------
def _last_error():
    return _lib.load().pf_last_error().decode()


def test_copy_primitives_buffer_too_small():
    """copy_cpu_to_gpu_async refuses a CPU buffer shorter than the copy with
    the reference's message (transfer.rs:89-95); copy_gpu_to_cpu does too."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 100)()
    rc = lib.pf_copy_cpu_to_gpu_async(0x1000, 0, ctypes.addressof(buf), 100, 101, None)
    assert rc == _lib.PF_ERR_STORAGE
    assert _last_error() == "CPU buffer too small: 100 bytes, need 101 bytes"
    rc = lib.pf_copy_gpu_to_cpu(0x1000, 64, ctypes.addressof(buf), 99, 100)
    assert rc == _lib.PF_ERR_STORAGE
    assert _last_error() == "CPU buffer too small: 99 bytes, need 100 bytes"
    rc = lib.pf_copy_cpu_to_gpu_async(0x1000, 0, None, 0, 16, None)
    assert rc == _lib.PF_ERR_INVALID_ARGUMENT and _last_error() == "null CPU buffer"


def test_batch_copy_segments_argument_errors():
    lib = _lib.load()
    pu = ctypes.POINTER(ctypes.c_uint64)
    g = (ctypes.c_uint64 * 2)(0, 64)
    c = (ctypes.c_uint64 * 2)(0x10000, 0x10040)
    out = ctypes.c_uint64(7)
    rc = lib.pf_batch_copy_segments_to_gpu(ctypes.cast(g, pu), ctypes.cast(c, pu), 2, 64, None,
                                           None, ctypes.byref(out))
    assert rc == _lib.PF_ERR_INVALID_ARGUMENT and _last_error() == "null layout"
    assert out.value == 0
    reg = _reg(0x100000, 1 << 20, 64, 4096, 64 * 4096 // 2, 2).to_c()
    rc = lib.pf_batch_copy_segments_to_gpu(None, None, 2, 64, ctypes.byref(reg), None,
                                           ctypes.byref(out))
    assert rc == _lib.PF_ERR_INVALID_ARGUMENT and _last_error() == "null transfer list"
    # An empty list issues nothing (transfer.rs:122-126).
    rc = lib.pf_batch_copy_segments_to_gpu(None, None, 0, 64, ctypes.byref(reg), None,
                                           ctypes.byref(out))
    assert rc == _lib.PF_OK and out.value == 0
    # segment_size * run length overflowing is the reference's error.
    big = (ctypes.c_uint64 * 2)(0, 1 << 63)
    bigc = (ctypes.c_uint64 * 2)(0x10000, 0x10000 + (1 << 63))
    rc = lib.pf_batch_copy_segments_to_gpu(ctypes.cast(big, pu), ctypes.cast(bigc, pu), 2,
                                           1 << 63, ctypes.byref(reg), None, ctypes.byref(out))
    assert rc == _lib.PF_ERR_STORAGE
    assert _last_error() == "batch_copy_segments_to_gpu: total_size overflow"


def test_copy_block_gpu_to_cpu_errors_from_segment_offset():
    """copy_block_gpu_to_cpu passes segment_offset's errors up unchanged
    (transfer.rs:207, 227), for contiguous and strided layouts; a contiguous
    whole block past the tensor gets the same offset/size/limit detail."""
    lib = _lib.load()
    dst = (ctypes.c_uint8 * 8192)()
    # Split KV-first layout (not contiguous): block 128's first segment
    # already starts at the end of the tensor.
    split = _reg(0x100000, 2 * 64 * 4096, 64, 4096, 64 * 4096, 2)
    rc = lib.pf_copy_block_gpu_to_cpu(ctypes.byref(split.to_c()), 128, ctypes.addressof(dst))
    assert rc == _lib.PF_ERR_STORAGE
    assert _last_error() == ("Block 128 segment 0 exceeds registered memory "
                             "(offset 524288, size 4096, limit 524288)")
    # Single-segment (contiguous) layout.
    single = _reg(0x100000, 10 * 4096, 10, 4096, 0, 1)
    rc = lib.pf_copy_block_gpu_to_cpu(ctypes.byref(single.to_c()), 10, ctypes.addressof(dst))
    assert rc == _lib.PF_ERR_STORAGE
    assert _last_error() == ("Block 10 segment 0 exceeds registered memory "
                             "(offset 40960, size 4096, limit 40960)")
    # Contiguous two-segment layout (kv_stride == bytes_per_block) at the
    # smallest size validation accepts, (num_blocks + 1) segments: block 10's
    # first segment passes segment_offset, its whole block does not fit.
    contig2 = _reg(0x100000, 11 * 4096, 10, 4096, 4096, 2)
    assert is_contiguous_layout(contig2)
    assert segment_offset(contig2, 10, 0) == 40960
    rc = lib.pf_copy_block_gpu_to_cpu(ctypes.byref(contig2.to_c()), 10, ctypes.addressof(dst))
    assert rc == _lib.PF_ERR_STORAGE
    assert _last_error() == ("Block 10 exceeds registered memory "
                             "(offset 40960, size 8192, limit 45056)")
    rc = lib.pf_copy_block_gpu_to_cpu(None, 0, ctypes.addressof(dst))
    assert rc == _lib.PF_ERR_INVALID_ARGUMENT and _last_error() == "null layout"
    assert lib.pf_layout_kind(None) == -1


def test_layer_array_reuses_and_refreshes_the_c_structs():
    """_layer_array makes each layer's pf_layer_xfer once per (registration,
    blocks array) and reuses it; a new blocks array or registration rebuilds
    it, in-place edits of the array are seen through the same pointer, and a
    pickled layer leaves the struct behind."""
    import pickle

    from pegaflow_amd import transfer as T

    reg = _reg(0x10000, 2 * 16 * 64, 16, 64, 16 * 64, 2)
    lt = T.LayerTransfer(reg, T.block_array([1, 2, 3], [0x9000, 0x9040, 0x9080]))
    arr, keep = T._layer_array([lt, lt])
    first = arr[0].blocks
    assert arr[1].blocks == first and arr[0].num_blocks == 3
    assert arr[0].layout.num_blocks == 16 and arr[0].layout.kv_stride_bytes == 16 * 64
    arr2, _ = T._layer_array([lt])
    assert arr2[0].blocks == first  # reused
    lt.blocks["block_idx"][0] = 7  # in place: the same memory
    assert np.frombuffer((ctypes.c_int64 * 1).from_address(first), np.int64)[0] == 7
    lt.blocks = T.block_array([4, 5], [0xA000, 0xA040])
    arr3, keep3 = T._layer_array([lt])
    assert arr3[0].num_blocks == 2 and arr3[0].blocks == keep3[0].ctypes.data != first
    reg2 = _reg(0x20000, 2 * 8 * 64, 8, 64, 8 * 64, 2)
    lt.registration = reg2
    arr4, _ = T._layer_array([lt])
    assert arr4[0].layout.data_ptr == 0x20000 and arr4[0].layout.num_blocks == 8
    back = pickle.loads(pickle.dumps(lt))
    assert "_c" not in back.__dict__
    assert back.registration == reg2 and back.blocks.tolist() == lt.blocks.tolist()
    arr5, keep5 = T._layer_array([back])
    assert arr5[0].blocks == keep5[0].ctypes.data
