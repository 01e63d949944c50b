"""The `pegaflow.Engine` wire surface on the CPU: schema encodings, the
tensor-handle record, the server's CLI size parser, and a live in-process
server over a plain host pool (no transfers).

The reference's own tests for this surface are the parse_memory_size cases
(pegaflow-server/src/utils.rs:42-57); the encodings below are fixed by the
field numbers and types of pegaflow-proto/proto/engine.proto:5-115 and the
protobuf wire format (tag = field << 3 | wire type; packed varints for
repeated int32; two's-complement 10-byte varints for negative int32).
"""

import os

import grpc
import pytest

from pegaflow_amd import _lib, ipc
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import PyLoadState
from pegaflow_amd.rpc import proto
from pegaflow_amd.rpc.client import EngineRpcClient
from pegaflow_amd.rpc.server import Server, TensorRegistry, parse_memory_size


# ---------------------------------------------------------------------------
# Wire encodings.
# ---------------------------------------------------------------------------
def test_register_request_encoding():
    m = proto.RegisterContextRequest(instance_id="a", device_id=1, num_blocks=300, segments=2,
                                     namespace="ns")
    # 0a 01 'a' | 10 01 | 28 ac02 (300) | 40 02 | 62 02 'ns'
    assert m.SerializeToString().hex() == "0a0161100128ac02400262026e73"


def test_save_layer_encoding_packs_ids_and_sign_extends():
    m = proto.SaveLayer(layer_name="l", block_ids=[1, 2, -1], block_hashes=[b"xy"])
    assert m.SerializeToString().hex() == "0a016c120c0102ffffffffffffffffff011a027879"
    back = proto.SaveLayer.FromString(bytes.fromhex("0a016c120c0102ffffffffffffffffff011a027879"))
    assert list(back.block_ids) == [1, 2, -1] and list(back.block_hashes) == [b"xy"]


def test_query_response_encoding():
    m = proto.QueryResponse(hit_blocks=5, prefetch_state=proto.PREFETCH_LOADING)
    assert m.SerializeToString().hex() == "10051801"
    # proto3 omits defaults: an all-default status still marks presence.
    m2 = proto.HealthResponse(status=proto.ResponseStatus(ok=False))
    assert m2.SerializeToString().hex() == "0a00" and m2.HasField("status")


def test_every_field_number_and_service_path():
    d = proto.LoadRequest.DESCRIPTOR
    assert [(f.name, f.number) for f in d.fields] == [
        ("instance_id", 1), ("tp_rank", 2), ("device_id", 3), ("load_state_shm", 4),
        ("layer_names", 5), ("block_ids", 6), ("block_hashes", 7)]
    d = proto.RegisterContextRequest.DESCRIPTOR
    assert [f.number for f in d.fields] == list(range(1, 13))
    assert proto.method_path("Query") == "/pegaflow.Engine/Query"
    svc = proto.FILE.services_by_name["Engine"]
    assert [m.name for m in svc.methods] == ["RegisterContext", "Save", "Load", "Query",
                                             "UnregisterContext", "Shutdown", "Health"]


# ---------------------------------------------------------------------------
# parse_memory_size: utils.rs:42-57 plus the unit table of utils.rs:22-29.
# ---------------------------------------------------------------------------
def test_parse_memory_size_basic():
    assert parse_memory_size("1024") == 1024
    assert parse_memory_size("1gb") == 1 << 30
    assert parse_memory_size("1.5gb") == int(1.5 * 1024 * 1024 * 1024)
    assert parse_memory_size(" 500MB ") == 500 << 20
    assert parse_memory_size("1TB") == 1 << 40
    assert parse_memory_size("512kb") == 512 << 10
    assert parse_memory_size("7b") == 7


def test_cli_accepts_the_reference_launch_command():
    """Every option of the reference's server (pegaflow-server/src/lib.rs:38-113)
    parses, with its defaults; --redis-url turns the disk tier on at the
    reference's default root, and options without effect are reported."""
    from pegaflow_amd.rpc.server import DEFAULT_DFS_ROOT, parse_args, unsupported_options

    d = parse_args([])
    assert (d.addr, d.device, d.pool_size, d.log_level) == ("127.0.0.1:50055", 0, 30 << 30, "info")
    assert d.dfs_root is None and d.dfs_quota == 50 << 30 and unsupported_options(d) == []
    assert (d.pre_evict_threshold, d.pre_evict_target, d.pre_evict_interval_ms) == \
        (5 << 30, 8 << 30, 100)
    a = parse_args(["--addr", "0.0.0.0:50055", "--device", "1", "--pool-size", "10gb",
                    "--hint-value-size", "64kb", "--use-hugepages", "--pre-evict",
                    "--pre-evict-threshold", "1gb", "--pre-evict-target", "2gb",
                    "--pre-evict-interval-ms", "50", "--disable-lfu-admission",
                    "--metrics-otel-endpoint", "", "--metrics-period-secs", "10",
                    "--log-level", "debug", "--redis-url", "redis://127.0.0.1:6379",
                    "--dfs-quota", "1tb", "--dfs-scan-interval-ms", "200"])
    assert a.pool_size == 10 << 30 and a.hint_value_size == 64 << 10 and a.device == 1
    assert a.dfs_root == DEFAULT_DFS_ROOT and a.dfs_quota == 1 << 40
    notes = unsupported_options(a)
    assert len(notes) == 1 and notes[0].startswith("--use-hugepages")
    assert a.pre_evict and (a.pre_evict_threshold, a.pre_evict_target) == (1 << 30, 2 << 30)
    assert a.disable_lfu_admission and not a.lfu_admission and not d.lfu_admission
    assert parse_args(["--lfu-admission"]).lfu_admission
    assert parse_args(["--dfs-root", "/mnt/x"]).dfs_root == "/mnt/x"


def test_parse_memory_size_invalid():
    for bad in ("", "abc", "-10gb", "10pb", "1_000"):
        with pytest.raises(ValueError):
            parse_memory_size(bad)


# ---------------------------------------------------------------------------
# The tensor-handle record.
# ---------------------------------------------------------------------------
def test_local_tensor_record_round_trip():
    rec = ipc.local_tensor(0x7F0000001000, 4096, 3)
    assert len(rec) == ipc.RECORD_BYTES == 104
    t = ipc.open_tensor(rec)
    assert (t.data_ptr, t.size_bytes, t.device_id, t.mapped_base) == (0x7F0000001000, 4096, 3, 0)


def test_record_rejections_happen_before_any_device_call():
    rec = bytearray(ipc.local_tensor(0x1000, 64, 0))
    with pytest.raises(ValueError, match="must be 104 bytes"):
        ipc.open_tensor(bytes(rec[:-1]))
    bad = bytes(b"XXXXXXXX") + bytes(rec[8:])
    with pytest.raises(ValueError, match="not a pegaflow tensor handle"):
        ipc.open_tensor(bad)
    past = ipc._HEAD.pack(ipc.MAGIC_PTR, 0, 0, 100, 64, 64) + bytes(64)
    with pytest.raises(ValueError, match="extends past"):
        ipc.open_tensor(past)
    big = ipc._HEAD.pack(ipc.MAGIC_IPC, 0, 0, 1 << 31, 0, 64) + bytes(64)
    with pytest.raises(ValueError, match="2 GiB"):
        ipc.open_tensor(big)


def test_registry_keys_and_drop():
    r = TensorRegistry()
    k0 = TensorRegistry.context_key("inst", 0, 0)
    assert k0 == "inst:tp0:dev0"
    r.register_layer(k0, "l0", 0, ipc.local_tensor(0x1000, 64, 0))
    r.register_layer(k0, "l0", 0, ipc.local_tensor(0x2000, 64, 0))  # replaces
    r.register_layer(TensorRegistry.context_key("inst", 1, 0), "l0", 0,
                     ipc.local_tensor(0x3000, 64, 0))
    r.register_layer(TensorRegistry.context_key("inst2", 0, 0), "l0", 0,
                     ipc.local_tensor(0x4000, 64, 0))
    with pytest.raises(ValueError, match="pinned to device 0"):
        r.register_layer(k0, "l1", 1, ipc.local_tensor(0x5000, 64, 1))
    assert r.drop_instance("inst") == 2
    assert r.drop_instance("inst") == 0
    assert r.drop_instance("inst2") == 1


def test_reregistration_keeps_the_mapping_the_engine_uses(monkeypatch):
    """A layer registered again: the engine gets the new address first, the
    old mapping is closed only after the engine's queued loads drained, and a
    registration the engine refuses closes the new mapping and keeps the
    old one (the engine still points there)."""
    from pegaflow_amd import frontend as fe

    events = []

    class Mapping:
        def __init__(self, addr):
            self.data_ptr, self.size_bytes, self.device_id = addr, 64, 0

        def close(self):
            events.append(("close", self.data_ptr))

    monkeypatch.setattr(fe, "open_tensor", lambda raw: Mapping(int(raw)))

    class Engine:
        refuse = False

        def register_context_layer(self, inst, ns, dev, name, ptr, *rest):
            if self.refuse:
                raise _lib.PegaFlowError(_lib.PF_ERR_TOPOLOGY_MISMATCH, "topology mismatch")
            events.append(("engine", ptr))

        def wait_idle(self):
            events.append(("drain",))

    eng = Engine()
    f = fe.EngineFrontend(eng)
    args = ("inst", "ns", 0, 1, 0, 2, "l0")
    f.register_context(*args, b"4096", 16, 512, 8192, 2)
    f.register_context(*args, b"8192", 16, 512, 8192, 2)
    assert events == [("engine", 4096), ("engine", 8192), ("drain",), ("close", 4096)]
    events.clear()
    eng.refuse = True
    with pytest.raises(_lib.PegaFlowError, match="topology mismatch"):
        f.register_context(*args, b"12288", 16, 512, 8192, 2)
    assert events == [("close", 12288)]
    key = TensorRegistry.context_key("inst", 0, 0)
    assert f.registry.tensor(key, "l0").data_ptr == 8192


# ---------------------------------------------------------------------------
# A live server over a plain host pool.
# ---------------------------------------------------------------------------
@pytest.fixture(params=["native", "python"])
def served(request):
    srv = Server("127.0.0.1:0", engine=PegaEngine(pool_size=64 << 20, host_pool=True),
                 grpc_impl=request.param).start()
    client = EngineRpcClient(f"http://{srv.addr}")
    yield srv, client
    client.close()
    srv.stop()


def _register(client, layer, nb=16, bpb=512, layers=2, inst="i0", tp_size=1, ptr=0x10000):
    size = 2 * nb * bpb
    return client.register_context(inst, "ns", 0, tp_size, 0, layers, layer,
                                   ipc.local_tensor(ptr, size, 0), nb, bpb, nb * bpb, 2)


def test_health_and_endpoint(served):
    srv, client = served
    assert client.health() == (True, "")
    assert client.endpoint() == f"http://{srv.addr}"


def test_register_query_unregister(served):
    srv, client = served
    assert _register(client, "l0") == (True, "")
    assert _register(client, "l1") == (True, "")
    q = client.query("i0", [b"a", b"b"])
    assert q == {"ok": True, "message": "", "hit_blocks": 0, "prefetch_state": "ready",
                 "loading_blocks": 0, "missing_blocks": 0}
    assert client.unregister_context("i0") == (True, "")
    with pytest.raises(RuntimeError, match=r"unregister_context RPC failed: .*FAILED_PRECONDITION"
                                           r".*instance i0 not found"):
        client.unregister_context("i0")


def test_error_codes_follow_engine_errors(served):
    srv, client = served
    _register(client, "l0")
    with pytest.raises(RuntimeError, match=r"FAILED_PRECONDITION.*topology mismatch"):
        _register(client, "l2", layers=3)
    with pytest.raises(RuntimeError, match=r"INVALID_ARGUMENT.*out of range for layer l0"):
        client.save("i0", 0, 0, [("l0", [16], [b"h"])])
    with pytest.raises(RuntimeError, match=r"query RPC failed: .*FAILED_PRECONDITION"
                                           r".*instance zz not found"):
        client.query("zz", [b"a"])
    with pytest.raises(RuntimeError, match=r"register_context RPC failed: .*INTERNAL"
                                           r".*register tensor failed"):
        client.register_context("i0", "ns", 0, 1, 0, 2, "l9", b"short", 16, 512, 8192, 2)
    # Negative ids only: nothing to transfer.
    assert client.save("i0", 0, 0, [("l0", [-1], [b"a"])]) == (True, "")


def test_load_failure_reaches_the_load_state(served):
    srv, client = served
    _register(client, "l0")
    st = PyLoadState()
    with pytest.raises(RuntimeError, match=r"load RPC failed: .*missing KV block hash"):
        client.load("i0", 0, 0, st.shm_name(), ["l0"], [1], [b"abc"])
    assert st.get_state() == -1
    st2 = PyLoadState()
    assert client.load("i0", 0, 0, st2.shm_name(), ["l0"], [], []) == (True, "")
    assert st2.get_state() == 1


def test_shutdown_sets_the_event(served):
    srv, client = served
    assert client.shutdown() == (True, "")
    assert srv.service.shutdown_event.is_set()


def test_client_fails_fast_without_a_server():
    with pytest.raises(RuntimeError, match="failed to connect to engine server"):
        EngineRpcClient("http://127.0.0.1:1", connect_timeout_s=0.3)


def test_server_speaks_to_a_raw_channel(served):
    """A client built only from the wire format (as the reference's tonic
    client is) gets the same answers."""
    srv, _ = served
    ch = grpc.insecure_channel(srv.addr)
    call = ch.unary_unary("/pegaflow.Engine/Health", request_serializer=lambda b: b,
                          response_deserializer=lambda b: b)
    assert call(b"", timeout=5) == bytes.fromhex("0a020801")  # status{ok=true}
    ch.close()


def test_save_request_from_shared_and_generated_lists():
    """EngineRpcClient.save converts a list shared by several layers once, and
    a generator of fresh per-layer lists (whose ids Python may reuse) still
    yields every layer's own values."""
    from pegaflow_amd.rpc import proto
    from pegaflow_amd.rpc.client import EngineRpcClient

    c = EngineRpcClient.__new__(EngineRpcClient)
    sent = []
    ok = proto.SaveResponse()
    ok.status.ok = True
    c._call = lambda rpc, method, req: sent.append(req) or ok
    ids, hs = [4, 5, 6], [bytes([i]) * 32 for i in range(3)]
    assert c.save("inst", 0, 0, [("a", ids, hs), ("b", ids, hs)]) == (True, "")
    gen = ((f"l{i}", [i, i + 1], [bytes([i]) * 32, bytes([i + 1]) * 32]) for i in range(6))
    assert c.save("inst", 0, 0, gen) == (True, "")
    first, second = (proto.SaveRequest.FromString(r) for r in sent)
    assert first.instance_id == "inst" and [s.layer_name for s in first.saves] == ["a", "b"]
    assert [list(s.block_ids) for s in first.saves] == [ids, ids]
    assert [list(s.block_hashes) for s in first.saves] == [hs, hs]
    assert [list(s.block_ids) for s in second.saves] == [[i, i + 1] for i in range(6)]
    assert [list(s.block_hashes) for s in second.saves] == \
        [[bytes([i]) * 32, bytes([i + 1]) * 32] for i in range(6)]


def test_save_request_encoding_matches_the_message():
    """The client's pre-encoded SaveRequest is byte-identical to the message
    built field by field, for shared, distinct and empty lists; the service
    hands equal consecutive lists to the engine as one object."""
    from pegaflow_amd.rpc import proto
    from pegaflow_amd.rpc.client import encode_save_request
    from pegaflow_amd.rpc.server import EngineService

    ids, hs = [7, -1, 300000], [bytes([i]) * 32 for i in range(3)]
    other = [1, 2, 3]
    saves = [("a", ids, hs), ("", ids, hs), ("c" * 200, other, hs), ("d", ids, hs),
             ("e", [], [])]
    ref = proto.SaveRequest(instance_id="inst", tp_rank=2, device_id=1)
    for n, i, h in saves:
        ref.saves.add(layer_name=n, block_ids=i, block_hashes=h)
    wire = encode_save_request("inst", 2, 1, saves)
    assert wire == ref.SerializeToString()
    assert proto.SaveRequest.FromString(wire) == ref

    got = {}

    class Frontend:
        def save(self, *a):
            got["saves"] = a[3]

    svc = EngineService.__new__(EngineService)
    svc.frontend = Frontend()
    for req in (proto.SaveRequest.FromString(wire),):
        svc.Save(req, None)
        out = got["saves"]
        assert [(n, list(i), list(h)) for n, i, h in out] == [(n, i, h) for n, i, h in saves]
        assert out[1][1] is out[0][1] and out[1][2] is out[0][2]   # "" after "a": shared
        assert out[2][1] is not out[1][1]                           # other ids
        assert out[3][1] is not out[2][1]                           # changes back


def _ld(field, payload):
    """One length-delimited record."""
    from pegaflow_amd.rpc.client import _varint
    return _varint(field << 3 | 2) + _varint(len(payload)) + payload


def test_engine_decoder_matches_the_full_parse(served):
    """The engine's request decoder (the native gRPC server's Save and Load,
    pf_engine_serve_request) gives what protobuf's full parse gives (the service's Python
    path) for the canonical encoding and for unpacked ids, the name after
    the lists, a second name record (the last wins), unknown fields, the
    header last and an empty layer: each variant's result or error text is
    the same, and the error names the layer that was decoded.  Malformed
    bytes (truncated, a name that is not UTF-8, a string with the wrong wire
    type, a bad length) fail on both."""
    from google.protobuf.message import DecodeError

    from pegaflow_amd.rpc import proto
    from pegaflow_amd.rpc.client import _varint as varint

    srv, slow = served
    _register(slow, "l0")
    _register(slow, "l1")

    def python_path(method, msg_cls, wire):
        got = []

        class Context:
            def abort(self, code, detail):
                got.append((code.name, detail))
                raise RuntimeError(detail)

        handler = srv.service.Save if method == 2 else srv.service.Load
        try:
            handler(msg_cls.FromString(wire), Context())
        except RuntimeError:
            pass
        return got[0] if got else ("OK", "")

    def native(method, wire):
        status, msg = _serve(srv.engine, method, wire)
        return ("OK", "") if status == 0 else (_STATUS_NAMES.get(status, "INTERNAL"), msg)

    hs = [b"x" * 32, b"y" * 32]
    head = proto.SaveRequest(instance_id="i0", tp_rank=0, device_id=0).SerializeToString()
    lists = proto.SaveLayer(block_ids=[5, 16], block_hashes=hs).SerializeToString()  # 16: out of range
    unpacked = b"".join(varint(2 << 3) + varint(v & (2**64 - 1)) for v in (5, 16))
    hashes = b"".join(_ld(3, h) for h in hs)
    saves = [
        head + _ld(4, _ld(1, b"l0") + lists),                          # canonical
        head + _ld(4, _ld(1, b"l0") + unpacked + hashes),              # ids not packed
        head + _ld(4, lists + _ld(1, b"l1")),                          # name after the lists
        head + _ld(4, _ld(1, b"l0") + lists + _ld(1, b"l1")),          # second name wins
        head + _ld(4, _ld(1, b"l1") + lists + _ld(1, b"")),            # ... also when empty
        head + _ld(4, _ld(1, b"l0") + lists) + varint(9 << 3) + varint(7),  # unknown field
        _ld(4, _ld(1, b"l1") + lists) + head,                          # header last
        head + _ld(4, b""),                                            # an empty layer
        head + _ld(4, _ld(1, b"l0") + _ld(2, varint(5)) + _ld(3, b"a")),  # a good one
    ]
    # Several layers: the decoder shares a layer's lists with the previous
    # layer's when their bytes are equal, and must still see every layer's own.
    def layer(name, ids, hl=hs, name_last=False):
        body = proto.SaveLayer(block_ids=ids, block_hashes=hl).SerializeToString()
        return _ld(4, body + _ld(1, name) if name_last else _ld(1, name) + body)

    mixed = b"".join(_ld(3, h) + varint(2 << 3) + varint(v) for h, v in zip(hs, (1, 2)))
    saves += [
        head + layer(b"l0", [1, 2]) + layer(b"l1", [1, 2]) + layer(b"l0", [1, 16]),
        head + layer(b"l0", [1, 2]) + layer(b"l1", [1]),                  # fewer ids
        head + layer(b"l0", [1, 2]) + layer(b"l1", [1, 2], hs[:1]),       # fewer hashes
        head + layer(b"l0", [1, 2]) + layer(b"l1", [1, 2], name_last=True) +
        layer(b"l1", [1, 2]) + layer(b"l0", [3, 16]),                     # after a name-last one
        head + _ld(4, _ld(1, b"l0") + mixed) + _ld(4, _ld(1, b"l1") + mixed) +
        layer(b"l1", [1, 2, 3]),                                          # interleaved lists
        head + layer(b"l0", [2, 1], hs[::-1]) + layer(b"l1", [1, 2]) + layer(b"l1", [16, 2]),
    ]
    outcomes = []
    for i, w in enumerate(saves):
        want = python_path(2, proto.SaveRequest, w)
        assert native(2, w) == want, f"save variant {i}: {want}"
        outcomes.append(want)
    assert "layer l0" in outcomes[0][1] and "layer l1" in outcomes[3][1]
    assert outcomes[8] == ("OK", "") or outcomes[8][0] != "INVALID_ARGUMENT"
    lhead = proto.LoadRequest(instance_id="i0", tp_rank=0, device_id=0,
                              load_state_shm="pega_load_none").SerializeToString()
    loads = [
        lhead + _ld(5, b"l0") + _ld(7, b"abc"),                        # missing shm, then hash
        _ld(7, b"abc") + _ld(5, b"zz") + lhead,                        # header last
        lhead + _ld(5, b"l0") + varint(6 << 3) + varint(3) + _ld(7, b"a"),  # unpacked id
    ]
    for i, w in enumerate(loads):
        want = python_path(1, proto.LoadRequest, w)
        assert native(1, w) == want, f"load variant {i}: {want}"
    canon = saves[0]
    bad = [canon[:-3], head + _ld(4, _ld(1, b"\xff\xfe") + lists), b"\x22\xff"]
    for i, w in enumerate(bad):
        with pytest.raises(DecodeError):
            proto.SaveRequest.FromString(w)
        assert native(2, w) == ("INTERNAL", "malformed SaveRequest"), f"bad {i}"
    # A known field with another wire type: the reference server's decoder
    # (prost) refuses the message, as the engine's does; protobuf's Python
    # parser keeps the record as an unknown field instead.
    assert native(2, head + _ld(4, varint(1 << 3) + varint(7))) == \
        ("INTERNAL", "malformed SaveRequest")
    # Over gRPC the same bytes fail as a message that does not parse.
    from pegaflow_amd.rpc.client import _serialize
    stub = slow._channel.unary_unary(proto.method_path("Save"), request_serializer=_serialize,
                                     response_deserializer=proto.SaveResponse.FromString)
    with pytest.raises(grpc.RpcError) as err:
        stub(bad[0], timeout=10)
    assert err.value.code() == grpc.StatusCode.INTERNAL
    assert err.value.details() == "malformed SaveRequest"


# ---------------------------------------------------------------------------
# The engine's decoder of request bytes (pf_engine_serve_request), which the
# native gRPC server hands Load and Save to.
# ---------------------------------------------------------------------------
# Engine status -> the gRPC status the service reports it as (service.rs:77-88).
_STATUS_NAMES = {1: "INVALID_ARGUMENT", 4: "FAILED_PRECONDITION", 5: "FAILED_PRECONDITION",
                 6: "FAILED_PRECONDITION"}


def _serve(engine, method, payload):
    """(status, error message) of one request through the engine's decoder."""
    from pegaflow_amd._lib import last_error, load
    rc = load().pf_engine_serve_request(engine._h, method, payload, len(payload))
    return rc, ("" if rc == 0 else last_error())


def _error(fn):
    with pytest.raises(RuntimeError) as e:
        fn()
    return str(e.value)


class _Decoded:
    """The service object called with decoded messages (its Python path, as
    a caller of the service object takes it), errors formatted as the
    client formats an RPC error.  Over gRPC the server hands Load and Save
    to the engine's own decoder instead."""

    def __init__(self, svc):
        self.svc = svc

    @staticmethod
    def _run(method, handler, req):
        class Context:
            def abort(self, code, detail):
                raise RuntimeError(f"{method} RPC failed: status: {code}, message: {detail!r}")

        handler(req, Context())
        return True, ""

    def save(self, *args):
        from pegaflow_amd.rpc import proto
        from pegaflow_amd.rpc.client import encode_save_request
        req = proto.SaveRequest.FromString(encode_save_request(*args))
        return self._run("save", self.svc.Save, req)

    def load(self, *args):
        from pegaflow_amd.rpc import proto
        from pegaflow_amd.rpc.client import encode_load_request
        req = proto.LoadRequest.FromString(encode_load_request(*args))
        return self._run("load", self.svc.Load, req)


def test_grpc_gives_the_service_results_and_errors(served):
    """Each request gives the same result and error text over gRPC (native:
    decoded by the engine; python: by protobuf) and through the service's
    Python path for decoded messages."""
    srv, slow = served
    decoded = _Decoded(srv.service)
    assert slow.health() == (True, "")
    _register(slow, "l0")
    _register(slow, "l1")
    cases = [
        lambda c: c.save("i0", 0, 0, [("l0", [16], [b"h"])]),                 # id out of range
        lambda c: c.save("i0", 0, 0, [("l0", [1, 2], [b"h"])]),               # length mismatch
        lambda c: c.save("i0", 0, 0, [("l1", [3], [b"h"])]),                  # host pool
        lambda c: c.save("zz", 0, 0, [("l0", [1], [b"h"])]),                  # no instance
        lambda c: c.save("i0", 0, 0, [("nope", [1], [b"h"])]),                # unknown layer
        lambda c: c.load("zz", 0, 0, PyLoadState().shm_name(), ["l0"], [1], [b"a"]),
        lambda c: c.load("i0", 0, 0, PyLoadState().shm_name(), ["l0"], [1], [b"abc"]),
        # More hashes than ids: every hash is still looked up (lib.rs:1008-1011).
        lambda c: c.load("i0", 0, 0, PyLoadState().shm_name(), ["l0"], [], [b"abc"]),
        lambda c: c.load("i0", 0, 0, "pega_load_missing", ["l0"], [1], [b"a"]),
    ]
    for i, case in enumerate(cases):
        want = _error(lambda: case(decoded))
        assert _error(lambda: case(slow)) == want, f"case {i}: {want}"
    assert "INVALID_ARGUMENT" in _error(lambda: cases[0](slow))
    assert "block_ids length 2 does not match block_hashes 1" in _error(lambda: cases[1](slow))
    assert "FAILED_PRECONDITION" in _error(lambda: cases[3](slow))
    # Negative ids only, and an empty load: nothing to do, the same on both.
    assert slow.save("i0", 0, 0, [("l0", [-1], [b"a"])]) == (True, "")
    st = PyLoadState()
    assert slow.load("i0", 0, 0, st.shm_name(), ["l0"], [], []) == (True, "")
    assert st.get_state() == 1
    st = PyLoadState()
    with pytest.raises(RuntimeError, match="missing KV block hash"):
        slow.load("i0", 0, 0, st.shm_name(), ["l0"], [1], [b"abc"])
    assert st.get_state() == -1  # the failure reaches the LoadState


def _varint(n):
    n &= (1 << 64) - 1
    out = bytearray()
    while True:
        b, n = n & 0x7F, n >> 7
        if not n:
            out.append(b)
            return bytes(out)
        out.append(b | 0x80)


def _field(num, wt, payload):
    if wt == 0:
        return _varint(num << 3) + _varint(payload)
    return _varint(num << 3 | wt) + (_varint(len(payload)) + payload if wt == 2 else payload)


def test_decoder_handles_every_encoding(served):
    """Hand-built requests through the engine's decoder: fields out of order,
    ids packed and unpacked, negative ids as 10-byte varints, unknown fields
    of every wire type; and malformed and unknown requests are errors."""
    srv, slow = served
    eng = srv.engine
    _register(slow, "l0")
    _register(slow, "l1")
    layer = (_field(3, 2, b"h1") + _field(2, 0, 5) + _field(2, 0, -3) + _field(1, 2, b"l0") +
             _field(3, 2, b"h2") + _field(3, 2, b"h3") + _field(2, 2, _varint(16)) +
             _field(9, 0, 7) + _field(10, 1, b"\0" * 8) + _field(11, 5, b"\0" * 4))
    req = _field(4, 2, layer) + _field(3, 0, 0) + _field(1, 2, b"i0") + _field(2, 0, 0)
    status, msg = _serve(eng, 2, req)
    # ids [5, -3, 16]: the negative id is skipped, 16 is out of range on l0.
    assert status == 1 and msg == "invalid argument: block 16 out of range for layer l0 " \
                                  "(16 blocks registered)"
    load = (_field(7, 2, b"zz") + _field(5, 2, b"l1") + _field(1, 2, b"i0") +
            _field(6, 2, _varint(1) + _varint(-2)) + _field(4, 2, b"pega_load_x") +
            _field(12, 2, b"ignored"))
    status, msg = _serve(eng, 1, load)
    assert status != 0 and "LoadState" in msg  # decoded through to the shm attach
    st = PyLoadState()
    load = (_field(5, 2, b"l1") + _field(1, 2, b"i0") + _field(7, 2, b"a") +
            _field(6, 0, 3) + _field(4, 2, st.shm_name().encode()) + _field(7, 2, b"b"))
    status, msg = _serve(eng, 1, load)
    assert status == 3 and "missing KV block hash at index 0" in msg
    assert st.get_state() == -1
    # Malformed: a length running past the message, a group wire type.
    assert _serve(eng, 2, _field(1, 2, b"i0")[:-1]) == (11, "malformed SaveRequest")
    assert _serve(eng, 1, _varint(1 << 3 | 3)) == (11, "malformed LoadRequest")
    assert _serve(eng, 9, b"") == (1, "unknown method 9")
    assert _serve(eng, 3, b"") == (0, "")  # Health
    assert slow.health() == (True, "")
