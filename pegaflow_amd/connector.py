"""Worker side of the vLLM KV connector, without a vLLM dependency.

Mirrors ``WorkerConnector`` (python/pegaflow/connector/worker.py:33-465) and
the records it consumes (``ConnectorContext``, ``LoadIntent``, ``SaveIntent``:
connector/common.py:22-52, 100-106): registering a worker's KV caches, saving
per layer through a batching save thread, starting asynchronous multi-layer
loads with a LoadState, and reporting finished requests.  It talks to any
client with the ``EngineRpcClient`` surface: the gRPC client
(``rpc.client.EngineRpcClient``) or an engine in the same process
(``frontend.LocalEngineClient``).

One behaviour is new: ``wait_for_layer_load`` really waits for the layer
(the reference's is a no-op, worker.py:288-289).  Loads use a layered
LoadState, so layer l can be used as soon as its bytes are in place.
"""

from __future__ import annotations

import logging
import queue
import threading
from dataclasses import dataclass, field
from typing import Any, Callable, Iterable

from .load_state import PyLoadState
from .transfer import derive_layout

log = logging.getLogger("pegaflow.connector")


@dataclass(frozen=True)
class ConnectorContext:
    """connector/common.py:22-33."""

    instance_id: str
    namespace: str
    block_size: int
    num_layers: int
    tp_size: int
    tp_rank: int | None
    device_id: int | None
    engine_client: Any


@dataclass(frozen=True)
class LoadIntent:
    """connector/common.py:46-52."""

    block_ids: tuple[int, ...]
    block_hashes: tuple[bytes, ...]
    num_tokens: int = 0


@dataclass(frozen=True)
class SaveIntent:
    """connector/common.py:100-106."""

    block_ids: tuple[int, ...]
    block_hashes: tuple[bytes, ...]


@dataclass
class ConnectorMetadata:
    """The per-step intents the scheduler side hands the worker
    (PegaConnectorMetadata, connector/common.py:230-240)."""

    load_intents: dict[str, LoadIntent] = field(default_factory=dict)
    save_intents: dict[str, SaveIntent] = field(default_factory=dict)


@dataclass
class _SaveTask:
    layer_name: str
    metadata: ConnectorMetadata
    request_ids: list[str]
    has_block_table: bool


def _torch_sync() -> None:
    import torch

    torch.cuda.synchronize()


def _torch_handle(tensor) -> bytes:
    from .ipc import export_torch_tensor

    return export_torch_tensor(tensor)


class WorkerConnector:
    """worker.py:33-465.

    ``producer_sync`` runs before each save batch so that the kernels that
    wrote the KV caches have finished (the reference calls
    ``torch.cuda.synchronize()``, worker.py:392-395).  ``tensor_handle``
    turns a KV-cache tensor into ``RegisterContextRequest.wrapper_bytes``
    (default: ``ipc.export_torch_tensor``)."""

    def __init__(self, context: ConnectorContext,
                 producer_sync: Callable[[], None] | None = None,
                 tensor_handle: Callable[[Any], bytes] | None = None):
        self._ctx = context
        self._producer_sync = producer_sync or _torch_sync
        self._tensor_handle = tensor_handle or _torch_handle
        self._save_queue: queue.Queue = queue.Queue()
        self._save_thread = threading.Thread(target=self._save_worker, daemon=True,
                                             name="PegaSaveWorker")
        self._save_thread.start()
        self._req_pending_layers: dict[str, int] = {}
        self._completed_saves: set[str] = set()
        self._save_completion_lock = threading.Lock()
        self._current_save_intents: set[str] = set()
        # shm name -> (state, layer names in load order, request ids)
        self._pending: dict[str, tuple[PyLoadState, list[str], set[str]]] = {}
        self._load_completion_lock = threading.Lock()
        self._registered_layers: list[str] = []
        self._finished_requests: set[str] = set()

    # -- lifecycle ---------------------------------------------------------
    def shutdown(self) -> None:
        """worker.py:60-63."""
        self.unregister_context()
        self._save_queue.put(None)
        self._save_thread.join()

    def unregister_context(self) -> None:
        """worker.py:65-78: rank 0 unregisters the instance."""
        if not self._registered_layers:
            return
        if self._ctx.tp_rank == 0:
            ok, message = self._ctx.engine_client.unregister_context(self._ctx.instance_id)
            if not ok:
                log.warning("unregister context failed: %s", message)
        self._registered_layers.clear()

    # -- registration ------------------------------------------------------
    def register_kv_caches(self, kv_caches: dict[str, Any]) -> None:
        """worker.py:80-146: one RegisterContext per layer, with the layout
        derived from shape and stride (worker.py:104-115)."""
        if self._ctx.device_id is None:
            raise RuntimeError("device id is unknown; cannot register KV caches")
        self._registered_layers = list(kv_caches)
        for layer_name, kv in kv_caches.items():
            if kv.storage_offset() != 0:
                raise ValueError(f"KV cache for {layer_name} must have zero storage offset")
            num_blocks, bytes_per_block, kv_stride_bytes, segments = derive_layout(
                tuple(kv.shape), tuple(kv.stride()), kv.element_size())
            ok, message = self._ctx.engine_client.register_context(
                self._ctx.instance_id, self._ctx.namespace, self._ctx.tp_rank, self._ctx.tp_size,
                self._ctx.device_id, self._ctx.num_layers, layer_name, self._tensor_handle(kv),
                num_blocks, bytes_per_block, kv_stride_bytes, segments)
            if not ok:
                raise RuntimeError(f"Register context failed for {layer_name}: {message}")
        log.info("registered %d KV cache layers for instance %s", len(kv_caches),
                 self._ctx.instance_id)

    # -- completion ----------------------------------------------------------
    def get_finished(self, finished_req_ids: set[str]
                     ) -> tuple[set[str] | None, set[str] | None]:
        """worker.py:148-214: (finished_sending, finished_recving)."""
        finished_sending = finished_recving = None
        with self._save_completion_lock:
            self._finished_requests.update(finished_req_ids & self._req_pending_layers.keys())
            done = self._completed_saves & self._finished_requests
            done |= self._completed_saves & finished_req_ids
            if done:
                self._completed_saves -= done
                self._finished_requests -= done
                finished_sending = done
        with self._load_completion_lock:
            completed: set[str] = set()
            for shm, (st, _layers, reqs) in list(self._pending.items()):
                if st.is_ready():
                    if st.get_state() < 0:
                        log.error("async load failed with state=%d for reqs=%s", st.get_state(),
                                  reqs)
                    completed |= reqs
                    del self._pending[shm]
            if completed:
                finished_recving = completed
        return finished_sending, finished_recving

    # -- loads ---------------------------------------------------------------
    def start_load_kv(self, metadata: ConnectorMetadata,
                      target_layers: Iterable[str] | None = None) -> str | None:
        """worker.py:217-286: one asynchronous multi-layer load for every load
        intent of this step.  ``target_layers`` defaults to the registered
        layers (the reference takes the forward context's attention layers).
        Returns the LoadState's shm name, or None when there is nothing to
        load."""
        self._current_save_intents = set(metadata.save_intents)
        if not metadata.load_intents:
            return None
        ids: list[int] = []
        hashes: list[bytes] = []
        reqs: list[str] = []
        for req_id, intent in metadata.load_intents.items():
            ids.extend(intent.block_ids)
            hashes.extend(intent.block_hashes)
            reqs.append(req_id)
        layers = list(target_layers) if target_layers is not None else list(self._registered_layers)
        if not ids or not layers:
            return None
        st = PyLoadState(num_layers=len(layers))
        ok, message = self._ctx.engine_client.load(self._ctx.instance_id, self._ctx.tp_rank,
                                                   self._ctx.device_id, st.shm_name(), layers,
                                                   ids, hashes)
        if not ok:
            raise RuntimeError(f"Load request failed: {message}")
        with self._load_completion_lock:
            self._pending[st.shm_name()] = (st, layers, set(reqs))
        return st.shm_name()

    def wait_for_layer_load(self, layer_name: str, timeout_s: float = 60.0) -> bool:
        """Blocks until ``layer_name`` is in place for every load in flight
        that covers it; False if one of them failed or timed out."""
        with self._load_completion_lock:
            waits = [(st, layers.index(layer_name)) for st, layers, _ in self._pending.values()
                     if layer_name in layers]
        ok = True
        for st, idx in waits:
            ok = st.wait_for_layer(idx, timeout_s) and ok
        return ok

    # -- saves ---------------------------------------------------------------
    def save_kv_layer(self, metadata: ConnectorMetadata, layer_name: str,
                      has_block_table: bool = True) -> None:
        """worker.py:291-315: queues the layer's save for every save intent."""
        request_ids = list(metadata.save_intents)
        if not request_ids:
            return
        with self._save_completion_lock:
            for req_id in request_ids:
                self._req_pending_layers.setdefault(req_id, len(self._registered_layers))
        self._save_queue.put(_SaveTask(layer_name, metadata, request_ids, has_block_table))

    def wait_for_save(self) -> None:
        """worker.py:317-342: intents whose layers never came (a step replayed
        from a graph calls no save hooks) count as saved."""
        with self._save_completion_lock:
            skipped = self._current_save_intents - set(self._req_pending_layers)
            self._completed_saves |= skipped
            self._current_save_intents = set()
        if skipped:
            log.debug("%d saves skipped (no layer hooks ran): %s", len(skipped), skipped)

    def drain_saves(self) -> None:
        """Returns when every queued layer save has been processed (no
        counterpart in the reference; for orderly shutdown and tests)."""
        self._save_queue.join()

    def _save_worker(self) -> None:
        """worker.py:344-370: batch whatever is queued, one save RPC per batch."""
        while True:
            task = self._save_queue.get()
            if task is None:
                self._save_queue.task_done()
                return
            batch = [task]
            stop = False
            while True:
                try:
                    t = self._save_queue.get_nowait()
                except queue.Empty:
                    break
                if t is None:
                    stop = True
                    break
                batch.append(t)
            self._process_save_batch(batch)
            for _ in batch:
                self._save_queue.task_done()
            if stop:
                self._save_queue.task_done()
                return

    def _process_save_batch(self, batch: list[_SaveTask]) -> None:
        """worker.py:372-427: failures are logged and the requests still
        complete ("continuing without save")."""
        by_layer: dict[str, tuple[list[int], list[bytes]]] = {}
        all_reqs: list[str] = []
        for task in batch:
            all_reqs.extend(task.request_ids)
            if not task.has_block_table:
                continue
            for intent in task.metadata.save_intents.values():
                if not intent.block_ids:
                    continue
                ids, hashes = by_layer.setdefault(task.layer_name, ([], []))
                ids.extend(intent.block_ids)
                hashes.extend(intent.block_hashes)
        if by_layer:
            try:
                self._producer_sync()
                ok, message = self._ctx.engine_client.save(
                    self._ctx.instance_id, self._ctx.tp_rank, self._ctx.device_id,
                    [(name, ids, hashes) for name, (ids, hashes) in by_layer.items()])
                if not ok:
                    log.error("save batch failed: %s (continuing without save)", message)
            except Exception as e:  # noqa: BLE001 - the reference swallows save errors too
                log.error("save failed: %s (continuing without save)", e)
        self._decrement_layer_counter(all_reqs)

    def _decrement_layer_counter(self, request_ids: list[str]) -> None:
        with self._save_completion_lock:
            for req_id in request_ids:
                if req_id not in self._req_pending_layers:
                    continue
                self._req_pending_layers[req_id] -= 1
                if self._req_pending_layers[req_id] < 0:
                    raise AssertionError(f"layer count mismatch for request {req_id}")
                if self._req_pending_layers[req_id] == 0:
                    self._completed_saves.add(req_id)
                    del self._req_pending_layers[req_id]


__all__ = ["ConnectorContext", "LoadIntent", "SaveIntent", "ConnectorMetadata",
           "WorkerConnector"]
