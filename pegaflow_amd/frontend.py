"""The engine's request layer, independent of the transport.

``EngineFrontend`` does what the reference's gRPC service does with each
request (pegaflow-server/src/service.rs:133-405): it opens layer-tensor
handles into a registry keyed per (instance, tp_rank, device)
(registry.rs:41-176) and calls the engine.  The gRPC service
(``rpc.server``) and the in-process client (``LocalEngineClient``) both
wrap it, so a connector runs unchanged against either.
"""

from __future__ import annotations

import logging
import threading

from . import _lib
from .engine import PegaEngine
from .ipc import OpenedTensor, open_tensor

log = logging.getLogger("pegaflow.frontend")

PREFETCH_READY, PREFETCH_LOADING, PREFETCH_PARTIAL_MISS = 0, 1, 2
_STATE_NAMES = {PREFETCH_READY: "ready", PREFETCH_LOADING: "loading",
                PREFETCH_PARTIAL_MISS: "partial_miss"}


class RegisterTensorError(RuntimeError):
    """A layer-tensor handle could not be opened (map_py_error,
    service.rs:90-93)."""


class _Refused(Exception):
    """The engine refused a registration (carries the engine's error)."""

    def __init__(self, cause: BaseException):
        super().__init__(str(cause))
        self.cause = cause


class TensorRegistry:
    """Registered layer tensors per context key "instance:tpR:devD"
    (registry.rs:41-176)."""

    def __init__(self):
        self._lock = threading.Lock()
        self._reg_lock = threading.Lock()  # one registration at a time
        self._contexts: dict[str, tuple[int, dict[str, OpenedTensor]]] = {}

    @staticmethod
    def context_key(instance_id: str, tp_rank: int, device_id: int) -> str:
        return f"{instance_id}:tp{tp_rank}:dev{device_id}"

    def register_layer(self, key: str, layer_name: str, device_id: int,
                       wrapper_bytes: bytes, commit=None, drain=None) -> OpenedTensor:
        """Opens the handle and makes it the layer's tensor.

        ``commit(t)`` (the engine's registration of the new address) runs
        before the registry changes: if it raises, the new handle is closed,
        the old one stays, and the error comes back as ``_Refused``.  A
        replaced handle is closed only after ``drain()``, so transfers queued
        on the old mapping finish before it is unmapped."""
        with self._reg_lock:
            t = open_tensor(wrapper_bytes)
            try:
                with self._lock:
                    dev = self._contexts.get(key, (t.device_id, None))[0]
                if dev != t.device_id:
                    raise ValueError(f"context {key} is pinned to device {dev} but got "
                                     f"{t.device_id}")
                if commit is not None:
                    try:
                        commit(t)
                    except Exception as e:
                        raise _Refused(e) from None
            except BaseException:
                t.close()
                raise
            with self._lock:
                _, tensors = self._contexts.setdefault(key, (t.device_id, {}))
                old = tensors.pop(layer_name, None)
                tensors[layer_name] = t
            if old is not None:
                if drain is not None:
                    drain()
                old.close()
            return t

    def tensor(self, key: str, layer_name: str) -> OpenedTensor | None:
        with self._lock:
            return self._contexts.get(key, (None, {}))[1].get(layer_name)

    def drop_instance(self, instance_id: str) -> int:
        prefix = f"{instance_id}:"
        with self._lock:
            keys = [k for k in self._contexts if k.startswith(prefix)]
            dropped = [self._contexts.pop(k)[1] for k in keys]
        n = 0
        for tensors in dropped:
            for t in tensors.values():
                t.close()
                n += 1
        return n

    def clear(self) -> None:
        with self._lock:
            dropped = list(self._contexts.values())
            self._contexts.clear()
        for _, tensors in dropped:
            for t in tensors.values():
                t.close()


class EngineFrontend:
    """Requests against one engine.  Errors: ``RegisterTensorError`` for a
    bad handle, ``PegaFlowError`` (a RuntimeError with the engine's code and
    message) for everything the engine refuses."""

    def __init__(self, engine: PegaEngine, disk: bool = False):
        self.engine = engine
        self.disk = disk  # prefix queries are prefetch-aware with a disk tier
        self.registry = TensorRegistry()

    def register_context(self, instance_id: str, namespace: str, tp_rank: int, tp_size: int,
                         device_id: int, num_layers: int, layer_name: str, wrapper_bytes: bytes,
                         num_blocks: int, bytes_per_block: int, kv_stride_bytes: int,
                         segments: int) -> None:
        """service.rs:140-186.  A layer registered again gets the new
        mapping in the engine before the old mapping is closed, and the old one
        is closed only once the engine's queued loads have drained; a
        registration the engine refuses leaves the old mapping in place."""
        def commit(t):
            self.engine.register_context_layer(instance_id, namespace, t.device_id, layer_name,
                                               t.data_ptr, t.size_bytes, num_blocks,
                                               bytes_per_block, kv_stride_bytes, segments,
                                               tp_rank, tp_size, num_layers)

        try:
            self.registry.register_layer(
                TensorRegistry.context_key(instance_id, tp_rank, device_id), layer_name,
                device_id, bytes(wrapper_bytes), commit=commit, drain=self.engine.wait_idle)
        except _Refused as e:
            raise e.cause from None
        except Exception as e:
            raise RegisterTensorError(f"register tensor failed: {e}") from None

    def save(self, instance_id: str, tp_rank: int, device_id: int, saves) -> None:
        self.engine.batch_save_kv_blocks(instance_id, tp_rank, device_id, saves)

    def serve(self, method: int, request: bytes) -> None:
        """A Load or Save request as its wire bytes, decoded by the engine."""
        self.engine.serve_request(method, request)

    def load(self, instance_id: str, tp_rank: int, device_id: int, load_state_shm: str,
             layer_names, block_ids, block_hashes) -> None:
        self.engine.batch_load_kv_blocks(instance_id, tp_rank, device_id, load_state_shm,
                                         list(layer_names), list(block_ids), list(block_hashes))

    def query(self, instance_id: str, block_hashes) -> dict:
        """service.rs:258-330: {state, hit_blocks, loading_blocks, missing_blocks}."""
        if self.disk:
            q = self.engine.count_prefix_hit_blocks_with_prefetch(instance_id, list(block_hashes))
            return {"state": q["state"], "hit_blocks": q["hit_blocks"],
                    "loading_blocks": q["loading_blocks"], "missing_blocks": q["missing_blocks"]}
        return {"state": PREFETCH_READY,
                "hit_blocks": self.engine.count_prefix_hit_blocks(instance_id, list(block_hashes)),
                "loading_blocks": 0, "missing_blocks": 0}

    def unregister(self, instance_id: str) -> None:
        """The engine first: dropping its instance drains the instance's queued
        loads, so no transfer still reads a mapping when the registry closes
        it."""
        err = None
        try:
            self.engine.unregister_instance(instance_id)
        except Exception as e:
            err = e
        removed = self.registry.drop_instance(instance_id)
        if removed:
            log.info("Dropped %d device tensors for instance %s", removed, instance_id)
        if err is not None:
            raise err

    def close(self) -> None:
        self.engine.wait_idle()
        self.registry.clear()


class LocalEngineClient:
    """The ``EngineRpcClient`` surface (python/src/lib.rs:262-525) over an
    engine in this process: same methods and returns ((ok, message) tuples,
    a dict from ``query``); failures raise RuntimeError."""

    def __init__(self, engine: PegaEngine | None = None, frontend: EngineFrontend | None = None,
                 disk: bool = False):
        if frontend is None:
            if engine is None:
                raise ValueError("an engine or a frontend is required")
            frontend = EngineFrontend(engine, disk=disk)
        self.frontend = frontend

    def endpoint(self) -> str:
        return "in-process"

    def health(self):
        return True, ""

    def register_context(self, instance_id, namespace, tp_rank, tp_size, device_id, num_layers,
                         layer_name, wrapper_bytes, num_blocks, bytes_per_block, kv_stride_bytes,
                         segments):
        self.frontend.register_context(instance_id, namespace, tp_rank, tp_size, device_id,
                                       num_layers, layer_name, wrapper_bytes, num_blocks,
                                       bytes_per_block, kv_stride_bytes, segments)
        return True, ""

    def save(self, instance_id, tp_rank, device_id, saves):
        self.frontend.save(instance_id, tp_rank, device_id, saves)
        return True, ""

    def load(self, instance_id, tp_rank, device_id, load_state_shm, layer_names, block_ids,
             block_hashes):
        self.frontend.load(instance_id, tp_rank, device_id, load_state_shm, layer_names,
                           block_ids, block_hashes)
        return True, ""

    def query(self, instance_id, block_hashes):
        q = self.frontend.query(instance_id, block_hashes)
        return {"ok": True, "message": "", "hit_blocks": q["hit_blocks"],
                "prefetch_state": _STATE_NAMES.get(q["state"], "ready"),
                "loading_blocks": q["loading_blocks"], "missing_blocks": q["missing_blocks"]}

    def unregister_context(self, instance_id):
        self.frontend.unregister(instance_id)
        return True, ""

    def shutdown(self):
        return True, ""

    def close(self) -> None:
        pass


__all__ = ["EngineFrontend", "LocalEngineClient", "TensorRegistry", "RegisterTensorError",
           "PREFETCH_READY", "PREFETCH_LOADING", "PREFETCH_PARTIAL_MISS", "_lib"]
