"""The worker-side connector (python/pegaflow/connector/worker.py:33-465) on
the CPU, against a recording client: registration and layout derivation,
batched saves with the producer sync before each, save completion and the
graph-replay skip, failed saves that still complete, asynchronous loads and
their completion, and per-layer waits that block until the layer is in
place (the reference's wait is a no-op)."""

import threading
import time

import pytest

from pegaflow_amd.connector import (ConnectorContext, ConnectorMetadata, LoadIntent, SaveIntent,
                                    WorkerConnector)
from pegaflow_amd.load_state import LoadState


class FakeTensor:
    def __init__(self, shape, stride, esize=2, offset=0, ptr=0x1000):
        self.shape, self._stride, self._esize, self._off, self._ptr = shape, stride, esize, offset, ptr

    def stride(self):
        return self._stride

    def element_size(self):
        return self._esize

    def storage_offset(self):
        return self._off

    def data_ptr(self):
        return self._ptr


class RecordingClient:
    def __init__(self, fail_saves=False):
        self.calls = []
        self.fail_saves = fail_saves
        self.lock = threading.Lock()

    def _rec(self, *a):
        with self.lock:
            self.calls.append(a)

    def register_context(self, *a):
        self._rec("register", *a)
        return True, ""

    def save(self, instance_id, tp_rank, device_id, saves):
        self._rec("save", instance_id, tp_rank, device_id, saves)
        if self.fail_saves:
            raise RuntimeError("save RPC failed: boom")
        return True, ""

    def load(self, *a):
        self._rec("load", *a)
        return True, ""

    def unregister_context(self, instance_id):
        self._rec("unregister", instance_id)
        return True, ""

    def of(self, kind):
        with self.lock:
            return [c for c in self.calls if c[0] == kind]


def make(client, num_layers=3, syncs=None):
    ctx = ConnectorContext("inst", "ns", 16, num_layers, 1, 0, 0, client)
    sync = (lambda: syncs.append(time.monotonic())) if syncs is not None else (lambda: None)
    return WorkerConnector(ctx, producer_sync=sync, tensor_handle=lambda t: b"h%d" % t.data_ptr())


def kv_first(ptr):
    # [2, 100 blocks, 16, 8, 128] bf16, contiguous
    return FakeTensor((2, 100, 16, 8, 128), (100 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128, 128, 1),
                      ptr=ptr)


def test_register_derives_layouts_like_the_reference():
    c = RecordingClient()
    w = make(c, num_layers=2)
    w.register_kv_caches({"l0": kv_first(0x1000),
                          "l1": FakeTensor((64, 16, 576), (16 * 576, 576, 1), esize=1, ptr=0x2000)})
    regs = c.of("register")
    assert regs[0][1:] == ("inst", "ns", 0, 1, 0, 2, "l0", b"h4096", 100, 32768, 3276800, 2)
    assert regs[1][1:] == ("inst", "ns", 0, 1, 0, 2, "l1", b"h8192", 64, 9216, 0, 1)
    with pytest.raises(ValueError, match="zero storage offset"):
        w.register_kv_caches({"bad": FakeTensor((2, 4, 8), (32, 8, 1), offset=8)})
    w.shutdown()
    assert c.of("unregister") == [("unregister", "inst")]


def test_saves_batch_and_complete_after_every_layer():
    c = RecordingClient()
    syncs = []
    w = make(c, syncs=syncs)
    w.register_kv_caches({f"l{i}": kv_first(0x1000 * (i + 1)) for i in range(3)})
    meta = ConnectorMetadata(save_intents={
        "r1": SaveIntent((1, 2), (b"a", b"b")), "r2": SaveIntent((5,), (b"c",))})
    w.start_load_kv(meta)
    for name in ("l0", "l1"):
        w.save_kv_layer(meta, name)
    w.drain_saves()
    assert w.get_finished(set()) == (None, None)  # one layer still to come
    w.save_kv_layer(meta, "l2")
    w.drain_saves()
    w.wait_for_save()
    # Only requests the caller reports finished are returned (worker.py:154-166).
    sending, recving = w.get_finished({"r1"})
    assert sending == {"r1"} and recving is None
    assert w.get_finished({"r2"}) == ({"r2"}, None)
    saved = [(name, ids, hashes) for call in c.of("save") for name, ids, hashes in call[4]]
    assert sorted(n for n, _, _ in saved) == ["l0", "l1", "l2"]
    for _, ids, hashes in saved:
        assert ids == [1, 2, 5] and hashes == [b"a", b"b", b"c"]
    assert len(syncs) == len(c.of("save"))  # the producer sync precedes every save
    w.shutdown()


def test_graph_replay_skip_and_failed_saves_still_complete():
    c = RecordingClient(fail_saves=True)
    w = make(c)
    w.register_kv_caches({f"l{i}": kv_first(0x1000 * (i + 1)) for i in range(3)})
    skipped = ConnectorMetadata(save_intents={"g": SaveIntent((3,), (b"x",))})
    w.start_load_kv(skipped)
    w.wait_for_save()  # no layer hook ran for "g"
    assert w.get_finished({"g"})[0] == {"g"}
    meta = ConnectorMetadata(save_intents={"f": SaveIntent((3,), (b"x",))})
    for name in ("l0", "l1", "l2"):
        w.save_kv_layer(meta, name)
    w.drain_saves()
    assert w.get_finished({"f"})[0] == {"f"}  # continuing without save (worker.py:409-424)
    assert c.of("save")
    w.shutdown()


def test_loads_complete_and_layers_can_be_awaited():
    c = RecordingClient()
    w = make(c)
    w.register_kv_caches({f"l{i}": kv_first(0x1000 * (i + 1)) for i in range(3)})
    meta = ConnectorMetadata(load_intents={
        "r1": LoadIntent((7, 8), (b"a", b"b")), "r2": LoadIntent((9,), (b"c",))})
    shm = w.start_load_kv(meta)
    call = c.of("load")[0]
    assert call[1:] == ("inst", 0, 0, shm, ["l0", "l1", "l2"], [7, 8, 9], [b"a", b"b", b"c"])
    server = LoadState.attach(shm)
    assert server.num_layers() == 3
    done = []

    def waiter():
        done.append(w.wait_for_layer_load("l1", timeout_s=10))

    t = threading.Thread(target=waiter)
    t.start()
    server.set_layers_done(1)
    time.sleep(0.05)
    assert not done  # layer 1 is not in place yet
    server.set_layers_done(2)
    t.join(5)
    assert done == [True]
    assert w.get_finished(set()) == (None, None)
    server.set_completed()
    assert w.get_finished(set()) == (None, {"r1", "r2"})
    assert w.wait_for_layer_load("l2")  # nothing in flight any more
    # A failed load is reported finished too (and waits on it return False).
    shm = w.start_load_kv(ConnectorMetadata(load_intents={"r3": LoadIntent((1,), (b"z",))}))
    LoadState.attach(shm).set_error()
    assert not w.wait_for_layer_load("l0", timeout_s=1)
    assert w.get_finished(set()) == (None, {"r3"})
    assert w.start_load_kv(ConnectorMetadata()) is None
    w.shutdown()


def test_request_reopened_by_later_saves_waits_for_them():
    """A request whose first step's saves completed, then saves again in a
    later step, is sent only once those later saves are processed, also when
    the scheduler reports it finished in between."""
    c = RecordingClient()
    w = make(c, num_layers=2)
    w.register_kv_caches({f"l{i}": kv_first(0x1000 * (i + 1)) for i in range(2)})
    meta = ConnectorMetadata(save_intents={"r": SaveIntent((1,), (b"a",))})
    for name in ("l0", "l1"):
        w.save_kv_layer(meta, name)
    w.drain_saves()
    meta2 = ConnectorMetadata(save_intents={"r": SaveIntent((2,), (b"b",))})
    w.save_kv_layer(meta2, "l0")
    w.drain_saves()
    assert w.get_finished({"r"}) == (None, None)  # layer l1 of the second step pending
    w.save_kv_layer(meta2, "l1")
    w.drain_saves()
    assert w.get_finished(set()) == ({"r"}, None)  # finished earlier, now saved
    assert w.get_finished({"r"}) == (None, None)  # reported once
    w.shutdown()
