"""The library's native gRPC server (pf_grpc.cpp) on a host-memory engine:
calls multiplexed on one connection from many threads, requests that span
many frames and outgrow the connection's flow-control window, a refused
message encoding, and clients that break the protocol.  The RPCs' results,
codes and messages are checked against grpcio's server in test_rpc.py (its
live-server tests run on both)."""

import hashlib
import socket
import struct
import threading
import time

import grpc
import pytest

from pegaflow_amd import ipc
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import PyLoadState
from pegaflow_amd.rpc.client import EngineRpcClient
from pegaflow_amd.rpc.server import Server

PREFACE = b"PRI * HTTP/2.0\r\n\r\nSM\r\n\r\n"


@pytest.fixture
def native():
    srv = Server("127.0.0.1:0", engine=PegaEngine(pool_size=64 << 20, host_pool=True)).start()
    assert srv.grpc_impl == "native"
    yield srv
    srv.stop()


def _register(client, layer, layers=2, nb=16, bpb=512):
    return client.register_context("i0", "ns", 0, 1, 0, layers, layer,
                                   ipc.local_tensor(0x10000, 2 * nb * bpb, 0), nb, bpb,
                                   nb * bpb, 2)


def _frame(ftype, flags, sid, payload=b""):
    return struct.pack(">I", len(payload))[1:] + bytes([ftype, flags]) + struct.pack(
        ">I", sid) + payload


def _frames(data):
    """(type, flags, stream, payload) of each whole frame in data."""
    out, off = [], 0
    while off + 9 <= len(data):
        n = int.from_bytes(data[off:off + 3], "big")
        if off + 9 + n > len(data):
            break
        out.append((data[off + 3], data[off + 4],
                    int.from_bytes(data[off + 5:off + 9], "big") & 0x7fffffff,
                    data[off + 9:off + 9 + n]))
        off += 9 + n
    return out


def _read_until_closed(s, timeout=5.0):
    s.settimeout(timeout)
    got = b""
    t0 = time.monotonic()
    while time.monotonic() - t0 < timeout:
        try:
            d = s.recv(65536)
        except socket.timeout:
            break
        except ConnectionResetError:
            return got, True
        if not d:
            return got, True
        got += d
    return got, False


def test_calls_from_many_threads_share_one_connection(native):
    """8 threads x 60 rounds of Health, Query (the Python handler), Save and
    Load (the engine's decoder) and a failing Load, on one client."""
    client = EngineRpcClient(f"http://{native.addr}")
    assert _register(client, "l0") == (True, "")
    assert _register(client, "l1") == (True, "")
    errors = []

    def worker(k):
        try:
            for i in range(60):
                assert client.health() == (True, "")
                assert client.query("i0", [b"h%d-%d" % (k, i)])["hit_blocks"] == 0
                assert client.save("i0", 0, 0, [("l0", [-1], [b"x"])]) == (True, "")
                st = PyLoadState()
                assert client.load("i0", 0, 0, st.shm_name(), ["l0"], [], []) == (True, "")
                assert st.get_state() == 1
                bad = PyLoadState()
                with pytest.raises(RuntimeError, match="missing KV block hash"):
                    client.load("i0", 0, 0, bad.shm_name(), ["l0"], [1], [b"zz%d" % i])
                assert bad.get_state() == -1
        except BaseException as e:  # reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(120)
        assert not t.is_alive()
    client.close()
    if errors:
        raise errors[0]
    assert native.native.served() >= 8 * 60 * 5 + 2


def test_large_requests_span_frames_and_refill_the_window(native):
    """Save requests of 2.6 MB (60,000 ids and hashes; negative ids, so
    nothing is copied), 40 of them: 105 MB through one connection, past the
    64 MiB after which the server gives the connection window back; and a
    2 MB Query through the Python handler."""
    client = EngineRpcClient(f"http://{native.addr}")
    assert _register(client, "l0", layers=1) == (True, "")
    n = 60000
    hashes = [hashlib.sha256(b"%d" % i).digest() for i in range(n)]
    for _ in range(40):
        assert client.save("i0", 0, 0, [("l0", [-1] * n, hashes)]) == (True, "")
    assert client.query("i0", hashes)["hit_blocks"] == 0
    client.close()


def test_compressed_messages_are_refused(native):
    ch = grpc.insecure_channel(native.addr, compression=grpc.Compression.Gzip)
    call = ch.unary_unary("/pegaflow.Engine/Health", request_serializer=lambda b: b,
                          response_deserializer=lambda b: b)
    with pytest.raises(grpc.RpcError) as e:
        call(b"\x00" * 64, timeout=5)
    assert e.value.code() == grpc.StatusCode.UNIMPLEMENTED
    ch.close()


def test_clients_breaking_the_protocol_do_not_disturb_others(native):
    host, port = native.addr.rsplit(":", 1)
    port = int(port)
    # Not HTTP/2: the connection is closed without a reply.
    s = socket.create_connection((host, port))
    s.sendall(b"GET / HTTP/1.1\r\nHost: example\r\n\r\n")
    got, closed = _read_until_closed(s)
    assert closed and got == b""
    s.close()
    # A header block that does not decode (index 62 of an empty table):
    # GOAWAY with COMPRESSION_ERROR, then the connection closes.
    s = socket.create_connection((host, port))
    s.sendall(PREFACE + _frame(4, 0, 0) + _frame(1, 0x4 | 0x1, 1, b"\xbe"))
    got, closed = _read_until_closed(s)
    assert closed
    frames = _frames(got)
    assert frames[0][0] == 4  # the server's SETTINGS first
    goaways = [f for f in frames if f[0] == 7]
    assert goaways and int.from_bytes(goaways[0][3][4:8], "big") == 9
    s.close()
    # A PING is answered with the same payload; a frame cut short ends the
    # connection.
    s = socket.create_connection((host, port))
    s.sendall(PREFACE + _frame(4, 0, 0) + _frame(6, 0, 0, b"12345678") + b"\x00\x00\x10\x00")
    s.shutdown(socket.SHUT_WR)
    got, closed = _read_until_closed(s)
    assert closed
    pings = [f for f in _frames(got) if f[0] == 6]
    assert pings and pings[0][1] == 1 and pings[0][3] == b"12345678"
    s.close()
    # The server still serves, and serves many short-lived clients.
    for _ in range(20):
        with EngineRpcClient(f"http://{native.addr}") as client:
            assert client.health() == (True, "")


def _goaway_code(host, port, frames_after_settings):
    """The error code of the server's GOAWAY after the preface, our SETTINGS
    and the given bytes; the connection must then close."""
    s = socket.create_connection((host, port))
    try:
        s.sendall(PREFACE + _frame(4, 0, 0) + frames_after_settings)
        got, closed = _read_until_closed(s)
        assert closed
        goaways = [f for f in _frames(got) if f[0] == 7]
        assert goaways, "no GOAWAY"
        return int.from_bytes(goaways[0][3][4:8], "big")
    finally:
        s.close()


def test_per_connection_limits(native):
    """A header block over 1 MiB in a single HEADERS frame is refused as one
    spread over CONTINUATION frames is (PROTOCOL_ERROR); a WINDOW_UPDATE that
    takes the connection's window past 2^31-1 is a FLOW_CONTROL_ERROR, and an
    increment of 0 a PROTOCOL_ERROR (RFC 9113 6.9); the server keeps serving
    other clients."""
    host, port = native.addr.rsplit(":", 1)
    port = int(port)
    big = b"\x00" + bytes([0x7f]) + b"\x81\x80\x40" + b"x" * (1 << 20)  # a literal > 1 MiB
    assert _goaway_code(host, port, _frame(1, 0x4 | 0x1, 1, big)) == 1
    assert _goaway_code(host, port, _frame(8, 0, 0, struct.pack(">I", 0x7fffffff))) == 3
    assert _goaway_code(host, port, _frame(8, 0, 0, struct.pack(">I", 0))) == 1
    with EngineRpcClient(f"http://{native.addr}") as client:
        assert client.health() == (True, "")


def _literal(name, value):
    """An HPACK literal header field without indexing, new name (short)."""
    return bytes([0, len(name)]) + name + bytes([len(value)]) + value


def test_stream_window_overflow_resets_only_that_stream(native):
    """A WINDOW_UPDATE taking one open stream's window past 2^31-1 resets
    that stream (RST_STREAM FLOW_CONTROL_ERROR); the connection goes on (a
    PING is still answered)."""
    host, port = native.addr.rsplit(":", 1)
    block = b"".join(_literal(n, v) for n, v in (
        (b":method", b"POST"), (b":scheme", b"http"), (b":path", b"/pegaflow.Engine/Health"),
        (b":authority", b"x"), (b"content-type", b"application/grpc"), (b"te", b"trailers")))
    s = socket.create_connection((host, int(port)))
    try:
        s.sendall(PREFACE + _frame(4, 0, 0) + _frame(1, 0x4, 1, block) +  # headers, no end
                  _frame(8, 0, 1, struct.pack(">I", 0x7fffffff)) + _frame(6, 0, 0, b"pingpong"))
        s.settimeout(5)
        got, t0 = b"", time.monotonic()
        while time.monotonic() - t0 < 5:
            frames = _frames(got)
            if any(f[0] == 6 and f[1] == 1 for f in frames):
                break
            got += s.recv(65536)
        frames = _frames(got)
        rst = [f for f in frames if f[0] == 3 and f[2] == 1]
        assert rst and int.from_bytes(rst[0][3], "big") == 3
        assert any(f[0] == 6 and f[1] == 1 and f[3] == b"pingpong" for f in frames)
        assert not any(f[0] == 7 for f in frames)  # no GOAWAY
    finally:
        s.close()
