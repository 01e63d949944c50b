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
class _LayerSave:
    """One save_kv_layer call: a layer and the save intents of its step."""

    layer_name: str
    intents: dict[str, SaveIntent]
    has_block_table: bool


@dataclass
class _SaveProgress:
    """What the worker knows about one request's saves.

    ``outstanding`` counts layer saves queued for the request and not yet
    processed: it is set to the number of registered layers when a step's
    first layer save arrives and counts down as batches are processed.
    ``complete`` says every save queued so far has been processed (or that
    the step ran no save hooks at all).  ``finished`` records that the
    scheduler already reported the request finished while saves were still
    outstanding, so it is handed back as soon as they complete."""

    outstanding: int = 0
    complete: bool = False
    finished: bool = False


@dataclass
class _InflightLoad:
    """One asynchronous multi-layer load: its LoadState, the position of each
    layer in the load, and the requests it restores."""

    state: PyLoadState
    layer_pos: dict[str, int]
    requests: frozenset[str]


def _torch_sync() -> None:
    import torch

    torch.cuda.synchronize()


def _torch_handle(tensor) -> bytes:
    from .ipc import export_torch_tensor

    return export_torch_tensor(tensor)


def _group_by_layer(batch: list[_LayerSave]) -> list[tuple[str, list[int], list[bytes]]]:
    """The save RPC's per-layer lists for a batch: each layer's block ids and
    hashes, concatenated over the batch's save intents in queue order.
    Steps run without a block table (worker.py:383-384) contribute none."""
    lists: dict[str, tuple[list[int], list[bytes]]] = {}
    for item in batch:
        if not item.has_block_table:
            continue
        for intent in item.intents.values():
            if intent.block_ids:
                ids, hashes = lists.setdefault(item.layer_name, ([], []))
                ids += intent.block_ids
                hashes += intent.block_hashes
    return [(name, ids, hashes) for name, (ids, hashes) in lists.items()]


class WorkerConnector:
    """worker.py:33-465.

    ``producer_sync`` runs before each save batch so that the kernels that
    wrote the KV caches have finished (the reference calls
    ``torch.cuda.synchronize()``, worker.py:392-395).  ``tensor_handle``
    turns a KV-cache tensor into ``RegisterContextRequest.wrapper_bytes``
    (default: ``ipc.export_torch_tensor``).

    State: one ``_SaveProgress`` per request with saves in flight or
    completed but not yet reported, one ``_InflightLoad`` per load in
    flight, all under one lock.  A single save thread processes, at each
    wake-up, every layer save queued so far as one batch."""

    def __init__(self, context: ConnectorContext,
                 producer_sync: Callable[[], None] | None = None,
                 tensor_handle: Callable[[Any], bytes] | None = None):
        self._ctx = context
        self._producer_sync = producer_sync or _torch_sync
        self._tensor_handle = tensor_handle or _torch_handle
        self._lock = threading.Lock()
        self._saves: dict[str, _SaveProgress] = {}
        self._loads: list[_InflightLoad] = []
        self._step_save_requests: set[str] = set()
        self._registered_layers: list[str] = []
        # The save queue: layer saves not yet taken, whether the thread is
        # processing a batch, and the stop request.
        self._queue_cv = threading.Condition()
        self._queued: list[_LayerSave] = []
        self._busy = False
        self._stopping = False
        self._save_thread = threading.Thread(target=self._run_saves, daemon=True,
                                             name="pegaflow-connector-save")
        self._save_thread.start()

    # -- lifecycle ---------------------------------------------------------
    def shutdown(self) -> None:
        """worker.py:60-63: unregisters, then lets the save thread finish what
        is queued and stop."""
        self.unregister_context()
        with self._queue_cv:
            self._stopping = True
            self._queue_cv.notify_all()
        self._save_thread.join()

    def unregister_context(self) -> None:
        """worker.py:65-78: rank 0 unregisters the instance."""
        if not self._registered_layers:
            return
        if self._ctx.tp_rank == 0:
            ok, message = self._ctx.engine_client.unregister_context(self._ctx.instance_id)
            if not ok:
                log.warning("unregister of instance %s failed: %s", self._ctx.instance_id,
                            message)
        self._registered_layers = []

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
        log.info("instance %s: %d KV cache layers registered", self._ctx.instance_id,
                 len(kv_caches))

    # -- completion ----------------------------------------------------------
    def get_finished(self, finished_req_ids: set[str]
                     ) -> tuple[set[str] | None, set[str] | None]:
        """worker.py:148-214: (finished_sending, finished_recving).

        A request is sent once the scheduler has reported it finished (in
        this call or an earlier one) and every save queued for it has been
        processed.  A request finished while it has no save activity is not
        tracked.  Unlike the reference, a step's new layer saves reopen a
        request whose earlier saves completed but were not yet reported, so
        it is not handed back while those saves are still queued.  Every
        load whose LoadState is ready, failed or not, reports its requests
        as received."""
        with self._lock:
            for rid in finished_req_ids:
                progress = self._saves.get(rid)
                if progress is not None and progress.outstanding > 0:
                    progress.finished = True
            sent = {rid for rid, progress in self._saves.items()
                    if progress.complete and (progress.finished or rid in finished_req_ids)}
            for rid in sent:
                del self._saves[rid]
            ready = [ld for ld in self._loads if ld.state.is_ready()]
            if ready:
                gone = {id(ld) for ld in ready}
                self._loads = [ld for ld in self._loads if id(ld) not in gone]
        received: set[str] = set()
        for ld in ready:
            if ld.state.get_state() < 0:
                log.error("load for requests %s failed (state %d)", sorted(ld.requests),
                          ld.state.get_state())
            received |= ld.requests
        return sent or None, received or None

    # -- loads ---------------------------------------------------------------
    def start_load_kv(self, metadata: ConnectorMetadata,
                      target_layers: Iterable[str] | None = None) -> str | None:
        """worker.py:217-286: one asynchronous multi-layer load for every load
        intent of this step.  ``target_layers`` defaults to the registered
        layers (the reference takes the forward context's attention layers).
        Returns the LoadState's shm name, or None when there is nothing to
        load."""
        with self._lock:
            self._step_save_requests = set(metadata.save_intents)
        intents = metadata.load_intents
        ids = [b for intent in intents.values() for b in intent.block_ids]
        hashes = [x for intent in intents.values() for x in intent.block_hashes]
        layers = list(target_layers) if target_layers is not None else list(self._registered_layers)
        if not ids or not layers:
            return None
        st = PyLoadState(num_layers=len(layers))
        ok, message = self._ctx.engine_client.load(self._ctx.instance_id, self._ctx.tp_rank,
                                                   self._ctx.device_id, st.shm_name(), layers,
                                                   ids, hashes)
        if not ok:
            raise RuntimeError(f"Load request failed: {message}")
        load = _InflightLoad(st, {name: i for i, name in enumerate(layers)}, frozenset(intents))
        with self._lock:
            self._loads.append(load)
        return st.shm_name()

    def wait_for_layer_load(self, layer_name: str, timeout_s: float = 60.0) -> bool:
        """Blocks until ``layer_name`` is in place for every load in flight
        that covers it; False if one of them failed or timed out."""
        with self._lock:
            waits = [(ld.state, ld.layer_pos[layer_name]) for ld in self._loads
                     if layer_name in ld.layer_pos]
        results = [st.wait_for_layer(pos, timeout_s) for st, pos in waits]
        return all(results)

    # -- saves ---------------------------------------------------------------
    def save_kv_layer(self, metadata: ConnectorMetadata, layer_name: str,
                      has_block_table: bool = True) -> None:
        """worker.py:291-315: queues the layer's save for every save intent.
        A request's first layer save of a step expects one save per
        registered layer."""
        if not metadata.save_intents:
            return
        with self._lock:
            for rid in metadata.save_intents:
                progress = self._saves.setdefault(rid, _SaveProgress())
                if progress.outstanding == 0:
                    progress.outstanding = len(self._registered_layers)
                    progress.complete = False
        with self._queue_cv:
            self._queued.append(_LayerSave(layer_name, dict(metadata.save_intents),
                                           has_block_table))
            self._queue_cv.notify_all()

    def wait_for_save(self) -> None:
        """worker.py:317-342: a request of this step with no layer save in
        flight (a step replayed from a graph runs no save hooks) counts as
        saved."""
        with self._lock:
            step, self._step_save_requests = self._step_save_requests, set()
            skipped = [rid for rid in step
                       if rid not in self._saves or self._saves[rid].outstanding == 0]
            for rid in skipped:
                self._saves.setdefault(rid, _SaveProgress()).complete = True
        if skipped:
            log.debug("no layer saves ran for %d requests; counted as saved", len(skipped))

    def drain_saves(self) -> None:
        """Returns when every queued layer save has been processed (no
        counterpart in the reference; for orderly shutdown and tests)."""
        with self._queue_cv:
            self._queue_cv.wait_for(lambda: not self._queued and not self._busy)

    def _run_saves(self) -> None:
        """The save thread (worker.py:344-370): each wake-up takes everything
        queued so far and saves it with one RPC."""
        while True:
            with self._queue_cv:
                self._queue_cv.wait_for(lambda: self._queued or self._stopping)
                if not self._queued:
                    return  # stopping, nothing left
                batch, self._queued = self._queued, []
                self._busy = True
            try:
                self._save_batch(batch)
            finally:
                with self._queue_cv:
                    self._busy = False
                    self._queue_cv.notify_all()

    def _save_batch(self, batch: list[_LayerSave]) -> None:
        """worker.py:372-427: one save RPC for the batch, after the producer
        sync.  A failed save is logged and its requests still count the
        layer as processed, so they complete without it."""
        saves = _group_by_layer(batch)
        if saves:
            try:
                self._producer_sync()
                ok, message = self._ctx.engine_client.save(
                    self._ctx.instance_id, self._ctx.tp_rank, self._ctx.device_id, saves)
                if not ok:
                    log.error("save of %d layers refused: %s; requests complete unsaved",
                              len(saves), message)
            except Exception as e:  # noqa: BLE001 - a failed save must not stop the worker
                log.error("save of %d layers raised %s; requests complete unsaved",
                          len(saves), e)
        with self._lock:
            for item in batch:
                for rid in item.intents:
                    progress = self._saves.get(rid)
                    if progress is None or progress.outstanding == 0:
                        continue
                    progress.outstanding -= 1
                    if progress.outstanding == 0:
                        progress.complete = True


__all__ = ["ConnectorContext", "LoadIntent", "SaveIntent", "ConnectorMetadata",
           "WorkerConnector"]
