"""The `pegaflow.Engine` gRPC path on the GPU: register layer tensors by
handle, save by hash, overwrite the layers, load by hash through LoadState,
and check every byte against the oracle — first with the server in this
process (pointer handles), then with the server in a child process that
maps the layers through HIP IPC, as a vLLM worker and the reference's
pegaflow-server do (pegaflow-server/src/registry.rs:144-175)."""

import hashlib
import os
import select
import subprocess
import sys
import time

import numpy as np
import pytest

import oracle
from pegaflow_amd import _lib, ipc
from pegaflow_amd._lib import PegaFlowError
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.load_state import LayerWords, PyLoadState
from pegaflow_amd.rpc.client import EngineRpcClient
from pegaflow_amd.rpc.server import Server
from pegaflow_amd.runtime import DeviceBuffer, Event, Stream, memcpy_async

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)


def h(i):
    return hashlib.sha256(b"rpc" + int(i).to_bytes(8, "little")).digest()


def wait(st, timeout=60.0):
    t0 = time.monotonic()
    while not st.is_ready():
        assert time.monotonic() - t0 < timeout, "load did not complete"
        time.sleep(0.0005)
    return st.get_state()


class Layers:
    """KV-first layers [2, nb, block] on device 0."""

    def __init__(self, n_layers, nb, bpb, seed):
        self.nb, self.bpb, self.kv, self.size = nb, bpb, nb * bpb, 2 * nb * bpb
        self.names = [f"model.layers.{l}.self_attn" for l in range(n_layers)]
        self.bufs = [DeviceBuffer(self.size) for _ in range(n_layers)]
        self.fill(seed)

    def fill(self, seed):
        for l, b in enumerate(self.bufs):
            b.fill_random(oracle.layer_seed(seed, l))

    def host(self):
        return [b.download() for b in self.bufs]

    def expected(self, saved_from, clobbered, ids, targets):
        """Oracle: blocks `ids` of `saved_from` copied to `targets` of `clobbered`."""
        out = []
        for src, dst in zip(saved_from, clobbered):
            src, dst = src.copy(), dst.copy()
            m = len(ids)
            host = np.zeros(2 * m * self.bpb, np.uint8)
            reg_s = oracle.layout(src.ctypes.data, self.size, self.nb, self.bpb, self.kv, 2)
            k, v, _ = oracle.save_host_layout(reg_s, m, host.ctypes.data,
                                              host.ctypes.data + m * self.bpb)
            oracle.process_save(reg_s, src, ids, k, v)
            reg_d = oracle.layout(dst.ctypes.data, self.size, self.nb, self.bpb, self.kv, 2)
            oracle.process_load(reg_d, dst, targets, k, v)
            out.append(dst)
        return out

    def close(self):
        for b in self.bufs:
            b.close()


def round_trip(client, layers, handles, inst="vllm-0"):
    n = len(layers.names)
    for name, handle in zip(layers.names, handles):
        assert client.register_context(inst, "llama", 0, 1, 0, n, name, handle, layers.nb,
                                       layers.bpb, layers.kv, 2) == (True, "")
    before = layers.host()
    ids = [7, 0, 33, 12, 63, 20, 21]
    hashes = [h(i) for i in ids]
    assert client.save(inst, 0, 0, [(name, ids, hashes) for name in layers.names]) == (True, "")
    q = client.query(inst, hashes + [h(1000)])
    assert q["ok"] and q["hit_blocks"] == len(ids) and q["prefetch_state"] == "ready"
    layers.fill(seed=99)  # what the GPU held is gone
    clobbered = layers.host()
    targets = [1, 2, 3, 62, 61, 40, 41]
    st = PyLoadState(num_layers=n)
    assert client.load(inst, 0, 0, st.shm_name(), layers.names, targets, hashes) == (True, "")
    assert wait(st) == 1 and st.layers_done() == n
    exp = layers.expected(before, clobbered, ids, targets)
    for l, b in enumerate(layers.bufs):
        assert np.array_equal(b.download(), exp[l]), f"layer {l}"
    assert client.unregister_context(inst) == (True, "")


def test_in_process_server_round_trip(gpu):
    say("[gpu] rpc in-process round trip (pointer handles)")
    srv = Server("127.0.0.1:0", engine=PegaEngine(pool_size=128 * MiB)).start()
    layers = Layers(4, 64, 16 * 8 * 128 * 2, seed=5)
    try:
        with EngineRpcClient(f"http://{srv.addr}") as client:
            handles = [ipc.local_tensor(b.ptr, layers.size, 0) for b in layers.bufs]
            round_trip(client, layers, handles)
    finally:
        srv.stop()
        layers.close()


def _start_server(*extra):
    cmd = [sys.executable, "-u", "-m", "pegaflow_amd.rpc.server", "--addr", "127.0.0.1:0",
           "--pool-size", "128mb", "--log-level", "warning", *extra]
    p = subprocess.Popen(cmd, cwd=ROOT, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         env=dict(os.environ), text=True)
    t0 = time.monotonic()
    seen = []
    while time.monotonic() - t0 < 90:
        r, _, _ = select.select([p.stdout], [], [], 1.0)
        if r:
            line = p.stdout.readline()
            if not line:
                break
            seen.append(line)
            if line.startswith("READY "):
                return p, line.split()[1]
        if p.poll() is not None:
            break
    p.kill()
    p.wait(10)
    raise AssertionError("server did not start:\n" + "".join(seen))


def test_two_process_ipc_round_trip(gpu):
    say("[gpu] rpc two-process round trip (HIP IPC handles)")
    layers = Layers(3, 64, 16 * 8 * 128 * 2, seed=11)
    assert layers.size < ipc.MAX_ALLOC_BYTES
    handles = [ipc.export_tensor(b.ptr, layers.size, 0) for b in layers.bufs]
    p, addr = _start_server()
    say(f"[gpu] server pid {p.pid} at {addr}")
    try:
        with EngineRpcClient(f"http://{addr}", connect_timeout_s=10) as client:
            round_trip(client, layers, handles)
            assert client.shutdown() == (True, "")
        assert p.wait(60) == 0
    finally:
        if p.poll() is None:
            p.kill()
            p.wait(10)
        layers.close()


def test_two_process_round_trip_over_grpcio(gpu):
    """The same round trip against a server whose gRPC endpoint is grpcio's
    (--grpc-impl python) instead of the library's own HTTP/2 server."""
    say("[gpu] rpc two-process round trip, grpcio server")
    layers = Layers(3, 64, 16 * 8 * 128 * 2, seed=13)
    handles = [ipc.export_tensor(b.ptr, layers.size, 0) for b in layers.bufs]
    p, addr = _start_server("--grpc-impl", "python")
    say(f"[gpu] server pid {p.pid} at {addr}")
    try:
        with EngineRpcClient(f"http://{addr}", connect_timeout_s=10) as client:
            assert client.health() == (True, "")
            round_trip(client, layers, handles)
            assert client.shutdown() == (True, "")
        assert p.wait(60) == 0
    finally:
        if p.poll() is None:
            p.kill()
            p.wait(10)
        layers.close()


def _ipc_events_supported():
    try:
        probe = Event(interprocess=True)
    except PegaFlowError as err:
        assert err.code == _lib.PF_ERR_UNSUPPORTED, err
        return False
    try:
        probe.ipc_handle()
    finally:
        probe.close()
    return True


def test_interprocess_events_fail_fast(gpu):
    """Where the runtime refuses to export interprocess events, both ways in
    fail up front with PF_ERR_UNSUPPORTED: creating such an event, and
    creating a LoadState that carries event handles (no loader could be
    handed real ones).  Where it exports them, both succeed."""
    say("[gpu] interprocess events: fail fast or work")
    handles = [bytes([1 + i]) * 64 for i in range(2)]
    if _ipc_events_supported():
        PyLoadState(num_layers=2, layer_events=handles)
        return
    with pytest.raises(PegaFlowError, match="cannot export interprocess events") as ei:
        PyLoadState(num_layers=2, layer_events=handles)
    assert ei.value.code == _lib.PF_ERR_UNSUPPORTED
    # Layer words, the cross-process substitute, are unaffected.
    PyLoadState(num_layers=2)


def test_cross_process_layer_events(gpu):
    """Device-side per-layer completion across processes: this process (the
    consumer) hands the server one interprocess event per layer in the
    LoadState; right after the load is queued its own stream waits on each
    layer's event and snapshots that layer.  Every snapshot must hold the
    restored bytes, which it could not if a wait returned before the
    server's copy of its layer had landed (the copies take ~1 ms; the
    snapshots are queued within microseconds)."""
    say("[gpu] rpc two-process layer events (device-side per-layer wait)")
    if not _ipc_events_supported():
        pytest.skip("this runtime cannot export interprocess events "
                    "(pf_event_create_ipc: PF_ERR_UNSUPPORTED)")
    n_layers = 8
    layers = Layers(n_layers, 256, 16 * 8 * 128 * 2, seed=21)
    handles = [ipc.export_tensor(b.ptr, layers.size, 0) for b in layers.bufs]
    events = [Event(interprocess=True) for _ in range(n_layers)]
    stream = Stream()
    snaps = [DeviceBuffer(layers.size) for _ in range(n_layers)]
    p, addr = _start_server()
    say(f"[gpu] server pid {p.pid} at {addr}")
    inst = "vllm-ev"
    try:
        with EngineRpcClient(f"http://{addr}", connect_timeout_s=10) as client:
            for name, handle in zip(layers.names, handles):
                assert client.register_context(inst, "llama", 0, 1, 0, n_layers, name, handle,
                                               layers.nb, layers.bpb, layers.kv, 2)[0]
            before = layers.host()
            ids = list(range(0, 256, 2))
            hashes = [h(1000 + i) for i in ids]
            assert client.save(inst, 0, 0, [(n, ids, hashes) for n in layers.names])[0]
            layers.fill(seed=77)
            clobbered = layers.host()
            targets = list(range(1, 256, 2))
            st = PyLoadState(num_layers=n_layers,
                             layer_events=[e.ipc_handle() for e in events])
            assert client.load(inst, 0, 0, st.shm_name(), layers.names, targets, hashes)[0]
            for l in range(n_layers):
                assert st.wait_for_layer_on_device(l, lambda i: stream.wait_event(events[i]),
                                                   timeout_s=30)
                memcpy_async(snaps[l].ptr, layers.bufs[l].ptr, layers.size, stream)
            stream.synchronize()
            assert wait(st) == 1 and st.layers_done() == n_layers
            exp = layers.expected(before, clobbered, ids, targets)
            for l in range(n_layers):
                assert np.array_equal(snaps[l].download(), exp[l]), f"layer {l} snapshot"
            assert client.unregister_context(inst)[0]
            assert client.shutdown()[0]
        assert p.wait(60) == 0
    finally:
        if p.poll() is None:
            p.kill()
            p.wait(10)
        for b in snaps:
            b.close()
        for e in events:
            e.close()
        stream.close()
        layers.close()


def test_cross_process_layer_words(gpu):
    """Device-side per-layer completion across processes without interprocess
    events: this process (the consumer) shares a few device words through a
    device-memory IPC handle in the LoadState; the server's copy kernel sets
    word l when layer l lands, and this process's stream waits on each word
    and snapshots that layer.  Every snapshot must hold the restored bytes.
    The same words serve a second load, and a failed load still writes them."""
    say("[gpu] rpc two-process layer words (device-side per-layer wait)")
    n_layers = 8
    layers = Layers(n_layers, 256, 16 * 8 * 128 * 2, seed=23)
    handles = [ipc.export_tensor(b.ptr, layers.size, 0) for b in layers.bufs]
    words = LayerWords(n_layers)
    flag = DeviceBuffer(4 * n_layers)
    stream = Stream()
    snaps = [DeviceBuffer(layers.size) for _ in range(n_layers)]
    p, addr = _start_server()
    say(f"[gpu] server pid {p.pid} at {addr}")
    inst = "vllm-words"
    try:
        with EngineRpcClient(f"http://{addr}", connect_timeout_s=10) as client:
            for name, handle in zip(layers.names, handles):
                assert client.register_context(inst, "llama", 0, 1, 0, n_layers, name, handle,
                                               layers.nb, layers.bpb, layers.kv, 2)[0]
            before = layers.host()
            ids = list(range(0, 256, 2))
            hashes = [h(2000 + i) for i in ids]
            assert client.save(inst, 0, 0, [(n, ids, hashes) for n in layers.names])[0]
            layers.fill(seed=78)
            clobbered = layers.host()
            targets = list(range(1, 256, 2))
            exp = layers.expected(before, clobbered, ids, targets)
            for rnd in range(2):
                layers.fill(seed=78)
                flag.memset(0)
                st = PyLoadState(layer_words=words)
                assert client.load(inst, 0, 0, st.shm_name(), layers.names, targets, hashes)[0]
                for l in range(n_layers):
                    assert st.wait_for_layer_on_device(
                        l, lambda i: words.wait_on_device(stream, i, 30_000_000, flag.ptr + 4 * i))
                    memcpy_async(snaps[l].ptr, layers.bufs[l].ptr, layers.size, stream)
                stream.synchronize()
                assert wait(st) == 1 and st.layers_done() == n_layers
                assert not flag.download().any(), f"round {rnd}: a device wait timed out"
                for l in range(n_layers):
                    assert np.array_equal(snaps[l].download(), exp[l]), f"round {rnd} layer {l}"
            # A load naming an unknown hash fails; its words are still written.
            st = PyLoadState(layer_words=words)
            with pytest.raises(RuntimeError, match="missing KV block hash"):
                client.load(inst, 0, 0, st.shm_name(), layers.names, [1], [h(10**6)])
            assert st.get_state() == -1
            t0 = time.monotonic()
            while (words.buf.download().view(np.uint64) != words.value).any():
                assert time.monotonic() - t0 < 10, "failed load left its words unset"
                time.sleep(0.001)
            assert client.unregister_context(inst)[0]
            assert client.shutdown()[0]
        assert p.wait(60) == 0
    finally:
        if p.poll() is None:
            p.kill()
            p.wait(10)
        for b in snaps:
            b.close()
        flag.close()
        words.close()
        stream.close()
