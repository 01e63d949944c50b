"""PegaEngine: the in-process engine over libpegaflow_hip.so.

Mirrors the reference's Python class (python/src/lib.rs:122-261) — same
method names, argument order and error behaviour (``RuntimeError`` carrying
the engine's message, e.g. "instance foo not found") — plus the save entry
point the reference exposes only through its gRPC service
(``batch_save_kv_blocks``, lib.rs:497-520) and the pool allocator
(``ScaledOffsetAllocator``, allocator.rs:66-171).
"""

from __future__ import annotations

import ctypes
from typing import Iterable, Sequence

import numpy as np

from . import _lib
from ._lib import EngineStats, PegaFlowError, SaveLayer

DEFAULT_PINNED_POOL_BYTES = 30 * 1024 * 1024 * 1024  # lib.rs:56


def lib():
    return _lib.load()


def _raise(rc: int) -> None:
    if rc != _lib.PF_OK:
        raise PegaFlowError(rc, _lib.last_error())


def _hashes(block_hashes: Sequence[bytes]):
    hs = [bytes(h) for h in block_hashes]
    offs = np.zeros(len(hs) + 1, np.uint64)
    if hs:
        offs[1:] = np.cumsum([len(h) for h in hs])
    data = np.frombuffer(b"".join(hs) or b"\0", np.uint8).copy()
    return data, offs


class ScaledOffsetAllocator:
    """Byte allocator in 32-bit units (allocator.rs:66-171)."""

    def __init__(self, total_bytes: int, unit_size: int | None = None):
        h = ctypes.c_void_p()
        if unit_size is None:
            _raise(lib().pf_allocator_create_auto(total_bytes, ctypes.byref(h)))
        else:
            _raise(lib().pf_allocator_create(total_bytes, unit_size, ctypes.byref(h)))
        self._h = h.value

    def allocate(self, size_bytes: int):
        """(offset, size) or None when no region fits."""
        found, off, size = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64()
        _raise(lib().pf_allocator_allocate(self._h, size_bytes, ctypes.byref(found),
                                           ctypes.byref(off), ctypes.byref(size)))
        return (off.value, size.value) if found.value else None

    def free(self, offset: int) -> None:
        _raise(lib().pf_allocator_free(self._h, offset))

    def storage_report(self):
        """(total_free_bytes, largest_free_allocation_bytes)."""
        t, f, l, u = (ctypes.c_uint64() for _ in range(4))
        _raise(lib().pf_allocator_report(self._h, ctypes.byref(t), ctypes.byref(f),
                                         ctypes.byref(l), ctypes.byref(u)))
        return f.value, l.value

    @property
    def unit_size(self) -> int:
        u = ctypes.c_uint64()
        _raise(lib().pf_allocator_report(self._h, None, None, None, ctypes.byref(u)))
        return u.value

    @property
    def total_bytes(self) -> int:
        t = ctypes.c_uint64()
        _raise(lib().pf_allocator_report(self._h, ctypes.byref(t), None, None, None))
        return t.value

    def __del__(self):
        try:
            if self._h:
                lib().pf_allocator_destroy(self._h)
        except Exception:
            pass


class PegaEngine:
    """python/src/lib.rs:89-261.

    ``pool_size`` bytes of pinned host memory back the block store (default
    30 GiB, lib.rs:56).  ``host_pool=True`` backs it with plain host memory
    instead: registration and lookups work, transfers are refused.
    """

    def __init__(self, pool_size: int = DEFAULT_PINNED_POOL_BYTES, host_pool: bool = False,
                 pinned_flags: int = _lib.PINNED_DEFAULT, unit_size_hint: int = 0):
        h = ctypes.c_void_p()
        kind = 1 if host_pool else 0
        _raise(lib().pf_engine_create(pool_size, kind, pinned_flags, unit_size_hint,
                                      ctypes.byref(h)))
        self._h = h.value

    def set_transfer_modes(self, save_mode: int = _lib.MODE_KERNEL,
                           load_mode: int = _lib.MODE_KERNEL) -> None:
        _raise(lib().pf_engine_set_modes(self._h, save_mode, load_mode))

    def register_context_layer(self, instance_id: str, namespace: str, device_id: int,
                               layer_name: str, data_ptr: int, size_bytes: int,
                               num_blocks: int, bytes_per_block: int, kv_stride_bytes: int,
                               segments: int, tp_rank: int, tp_size: int,
                               num_layers: int) -> None:
        _raise(lib().pf_engine_register_context_layer(
            self._h, instance_id.encode(), namespace.encode(), device_id, layer_name.encode(),
            data_ptr, size_bytes, num_blocks, bytes_per_block, kv_stride_bytes, segments,
            tp_rank, tp_size, num_layers))

    def unregister_instance(self, instance_id: str) -> None:
        _raise(lib().pf_engine_unregister_instance(self._h, instance_id.encode()))

    def count_prefix_hit_blocks(self, instance_id: str, block_hashes: Sequence[bytes]) -> int:
        data, offs = _hashes(block_hashes)
        out = ctypes.c_uint64()
        _raise(lib().pf_engine_count_prefix_hit_blocks(
            self._h, instance_id.encode(), data.ctypes.data, offs.ctypes.data, len(offs) - 1,
            ctypes.byref(out)))
        return out.value

    def batch_save_kv_blocks(self, instance_id: str, tp_rank: int, device_id: int,
                             saves: Iterable[tuple[str, Sequence[int], Sequence[bytes]]]) -> None:
        """Blocking save of (layer_name, block_ids, block_hashes) per layer."""
        keep, arr = [], []
        for layer_name, block_ids, block_hashes in saves:
            ids = np.ascontiguousarray(block_ids, dtype=np.int32)
            if len(ids) != len(block_hashes):
                raise PegaFlowError(_lib.PF_ERR_INVALID_ARGUMENT,
                                    f"invalid argument: block_ids length {len(ids)} does not "
                                    f"match block_hashes {len(block_hashes)}")
            data, offs = _hashes(block_hashes)
            name = layer_name.encode()
            keep += [ids, data, offs, name]
            arr.append(SaveLayer(name, ids.ctypes.data, len(ids), data.ctypes.data,
                                 offs.ctypes.data))
        c_arr = (SaveLayer * max(len(arr), 1))(*arr)
        _raise(lib().pf_engine_batch_save(self._h, instance_id.encode(), tp_rank, device_id,
                                          c_arr, len(arr)))
        del keep

    def batch_load_kv_blocks(self, instance_id: str, tp_rank: int, device_id: int,
                             load_state_shm: str, layer_names: Sequence[str],
                             block_ids: Sequence[int], block_hashes: Sequence[bytes]) -> None:
        """Queues a multi-layer load; completion is published in the LoadState."""
        ids = np.ascontiguousarray(block_ids, dtype=np.int32)
        data, offs = _hashes(block_hashes)
        names = [n.encode() for n in layer_names]
        c_names = (ctypes.c_char_p * max(len(names), 1))(*names)
        _raise(lib().pf_engine_batch_load(
            self._h, instance_id.encode(), tp_rank, device_id, load_state_shm.encode(), c_names,
            len(names), ids.ctypes.data, data.ctypes.data, offs.ctypes.data, len(ids)))

    def stats(self) -> dict:
        s = EngineStats()
        _raise(lib().pf_engine_stats_get(self._h, ctypes.byref(s)))
        return {name: getattr(s, name) for name, _ in EngineStats._fields_}

    def wait_idle(self) -> None:
        _raise(lib().pf_engine_wait_idle(self._h))

    def close(self) -> None:
        if self._h:
            lib().pf_engine_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
