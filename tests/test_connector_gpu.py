"""The worker-side connector on the GPU, as vLLM drives it: register the KV
caches, save per layer for two requests, report them saved, overwrite the
caches, load the saved blocks by hash into other blocks, wait for each
layer, report the load finished — through an engine in this process and
through the gRPC server — with every byte checked against the oracle."""

import hashlib
import sys
import time

import numpy as np
import pytest

import oracle
from pegaflow_amd import ipc, runtime
from pegaflow_amd.connector import (ConnectorContext, ConnectorMetadata, LoadIntent, SaveIntent,
                                    WorkerConnector)
from pegaflow_amd.engine import PegaEngine
from pegaflow_amd.frontend import LocalEngineClient
from pegaflow_amd.rpc.client import EngineRpcClient
from pegaflow_amd.rpc.server import Server
from pegaflow_amd.runtime import DeviceBuffer

pytestmark = pytest.mark.gpu
MiB = 1 << 20


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class DeviceTensor:
    """A KV-first bf16 layer [2, nb, 16, 8, 128] in a device buffer, with the
    tensor methods the connector reads."""

    def __init__(self, nb, seed):
        self.nb = nb
        self.shape = (2, nb, 16, 8, 128)
        self._stride = (nb * 16 * 8 * 128, 16 * 8 * 128, 8 * 128, 128, 1)
        self.nbytes = 2 * nb * 16 * 8 * 128 * 2
        self.buf = DeviceBuffer(self.nbytes)
        self.fill(seed)

    def fill(self, seed):
        self.buf.fill_random(seed)

    def stride(self):
        return self._stride

    def element_size(self):
        return 2

    def storage_offset(self):
        return 0

    def data_ptr(self):
        return self.buf.ptr


def h(i):
    return hashlib.sha256(b"conn" + int(i).to_bytes(8, "little")).digest()


def expected(before, clobbered, nb, ids, targets):
    bpb = 16 * 8 * 128 * 2
    src, dst = before.copy(), clobbered.copy()
    m = len(ids)
    host = np.zeros(2 * m * bpb, np.uint8)
    reg_s = oracle.layout(src.ctypes.data, src.nbytes, nb, bpb, nb * bpb, 2)
    k, v, _ = oracle.save_host_layout(reg_s, m, host.ctypes.data, host.ctypes.data + m * bpb)
    oracle.process_save(reg_s, src, ids, k, v)
    reg_d = oracle.layout(dst.ctypes.data, dst.nbytes, nb, bpb, nb * bpb, 2)
    oracle.process_load(reg_d, dst, targets, k, v)
    return dst


@pytest.mark.parametrize("transport", ["in_process", "grpc"])
def test_connector_save_load_round_trip(gpu, transport):
    say(f"[gpu] connector round trip over {transport}")
    n_layers, nb = 4, 128
    caches = {f"model.layers.{l}.self_attn": DeviceTensor(nb, oracle.layer_seed(31, l))
              for l in range(n_layers)}
    engine = PegaEngine(pool_size=128 * MiB)
    srv = None
    if transport == "grpc":
        srv = Server("127.0.0.1:0", engine=engine).start()
        client = EngineRpcClient(f"http://{srv.addr}")
    else:
        client = LocalEngineClient(engine)
    ctx = ConnectorContext("vllm-w0", "llama", 16, n_layers, 1, 0, 0, client)
    w = WorkerConnector(ctx, producer_sync=runtime.synchronize,
                        tensor_handle=lambda t: ipc.local_tensor(t.data_ptr(), t.nbytes, 0))
    try:
        w.register_kv_caches(caches)
        before = {n: t.buf.download() for n, t in caches.items()}
        r1 = SaveIntent((3, 5, 7), tuple(h(i) for i in (3, 5, 7)))
        r2 = SaveIntent((10, 11), tuple(h(i) for i in (10, 11)))
        step = ConnectorMetadata(save_intents={"r1": r1, "r2": r2})
        w.start_load_kv(step)  # no loads this step; records the save intents
        for name in caches:
            w.save_kv_layer(step, name)
        w.drain_saves()
        w.wait_for_save()
        assert w.get_finished({"r1", "r2"}) == ({"r1", "r2"}, None)

        for l, t in enumerate(caches.values()):
            t.fill(oracle.layer_seed(99, l))
        clobbered = {n: t.buf.download() for n, t in caches.items()}
        ids = list(r1.block_ids + r2.block_ids)
        targets = [60, 61, 62, 100, 101]
        load = ConnectorMetadata(load_intents={
            "r3": LoadIntent(tuple(targets), r1.block_hashes + r2.block_hashes)})
        assert w.start_load_kv(load) is not None
        for name in caches:
            assert w.wait_for_layer_load(name, timeout_s=30)
        deadline = time.monotonic() + 30
        recving = None
        while recving is None and time.monotonic() < deadline:
            _, recving = w.get_finished(set())
            time.sleep(0.001)
        assert recving == {"r3"}
        for n, t in caches.items():
            assert np.array_equal(t.buf.download(),
                                  expected(before[n], clobbered[n], nb, ids, targets)), n
        w.shutdown()
    finally:
        if srv is not None:
            client.close()
            srv.stop()
        else:
            engine.close()
        for t in caches.values():
            t.buf.close()
