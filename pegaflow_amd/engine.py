"""PegaEngine: the in-process engine over libpegaflow_hip.so.

Mirrors the reference's Python class (python/src/lib.rs:122-261) — same
method names, argument order and error behaviour (``RuntimeError`` carrying
the engine's message, e.g. "instance foo not found") — plus the save entry
point the reference exposes only through its gRPC service
(``batch_save_kv_blocks``, lib.rs:497-520) and the pool allocator
(``ScaledOffsetAllocator``, allocator.rs:66-171).
"""

from __future__ import annotations

import array
import ctypes
from typing import Iterable, Sequence

import numpy as np

from . import _lib
from ._lib import DiskStats, EngineStats, PegaFlowError, PrefetchStatus

DEFAULT_PINNED_POOL_BYTES = 30 * 1024 * 1024 * 1024  # lib.rs:56
DEFAULT_DISK_QUOTA_BYTES = 50 * 1024 * 1024 * 1024  # pegaflow-server/src/lib.rs:106-108
PREFETCH_STATE_NAMES = {0: "ready", 1: "loading", 2: "partial_miss"}


def lib():
    return _lib.load()


def _raise(rc: int) -> None:
    if rc != _lib.PF_OK:
        raise PegaFlowError(rc, _lib.last_error())


def _hashes(block_hashes: Sequence[bytes]):
    """(bytes, offsets): hash i is data[offs[i]:offs[i+1]]."""
    n = len(block_hashes)
    data = np.frombuffer(b"".join(block_hashes) or b"\0", np.uint8)
    lengths = set(map(len, block_hashes))
    if len(lengths) == 1 and (step := lengths.pop()) > 0:  # the usual case: one length
        return data, np.arange(0, (n + 1) * step, step, dtype=np.uint64)
    offs = np.zeros(n + 1, np.uint64)
    if n:
        np.cumsum(np.fromiter(map(len, block_hashes), np.uint64, n), out=offs[1:])
    return data, offs


def _block_ids(block_ids: Sequence[int]):
    """(keep-alive object, address, count) of block_ids as int32."""
    if isinstance(block_ids, np.ndarray):
        ids = np.ascontiguousarray(block_ids, dtype=np.int32)
        return ids, ids.ctypes.data, len(ids)
    ids = array.array("i", block_ids)  # C int: 32 bits on this platform
    return ids, ids.buffer_info()[0], len(ids)


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
        self._name_arrays = {}  # tuple of layer names -> C array of their bytes
        self._save_names = {}   # layer name -> (its bytes, their address)

    def set_storage_policy(self, lfu_admission: bool = False, value_size_hint: int = 0,
                           pre_evict: bool = False, pre_evict_threshold: int = 5 << 30,
                           pre_evict_target: int = 8 << 30,
                           pre_evict_interval_ms: int = 100) -> None:
        """The reference's StorageConfig (storage.rs:43-111;
        pf_engine_set_storage_policy): TinyLFU admission of new blocks, its
        sketch sized for pool / value_size_hint entries (0: 128 MiB per
        value), and the pre-eviction monitor (evict least-recently-used
        blocks while fewer than pre_evict_threshold bytes are free, until
        pre_evict_target are).  Both off by default here."""
        _raise(lib().pf_engine_set_storage_policy(
            self._h, int(bool(lfu_admission)), value_size_hint, int(bool(pre_evict)),
            pre_evict_threshold, pre_evict_target, pre_evict_interval_ms))

    def set_transfer_modes(self, save_mode: int = _lib.MODE_AUTO,
                           load_mode: int = _lib.MODE_AUTO) -> None:
        """Transfer modes of saves and loads (pf_engine_set_modes); the
        defaults (AUTO both ways) run a save batch, and a load of blocks
        saved together, staged on the copy engines, and a load of a few
        scattered blocks by the zero-copy kernel."""
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
        """Blocking save of (layer_name, block_ids, block_hashes) per layer.
        Lists shared by several layers (the usual case) are packed once."""
        keep, words = [], []
        # Each list packed once, with its address (numpy's ctypes.data costs
        # microseconds per access: 96 of them were 0.2 ms of a 32-layer save).
        # The pf_save_layer array is built as its 64-bit words (name, ids,
        # count, hash bytes, hash offsets): one ctypes structure per layer
        # cost more than the rest of a 32-layer save's marshalling.
        packed_ids, packed_hashes = {}, {}
        names = self._save_names
        n_layers = 0
        for layer_name, block_ids, block_hashes in saves:
            pi = packed_ids.get(id(block_ids))
            if pi is None:
                pi = packed_ids[id(block_ids)] = _block_ids(block_ids)
                keep += [block_ids, pi[0]]  # keeps id() unique for the whole call
            _, ids_ptr, n_ids = pi
            if n_ids != len(block_hashes):
                raise PegaFlowError(_lib.PF_ERR_INVALID_ARGUMENT,
                                    f"invalid argument: block_ids length {n_ids} does not "
                                    f"match block_hashes {len(block_hashes)}")
            hp = packed_hashes.get(id(block_hashes))
            if hp is None:
                data, offs = _hashes(block_hashes)
                hp = packed_hashes[id(block_hashes)] = (data.ctypes.data, offs.ctypes.data)
                keep += [block_hashes, data, offs]
            name = names.get(layer_name)
            if name is None:
                if len(names) >= 4096:
                    names.clear()
                b = layer_name.encode()
                name = names[layer_name] = (b, ctypes.cast(ctypes.c_char_p(b),
                                                           ctypes.c_void_p).value)
            keep.append(name[0])
            words += (name[1], ids_ptr, n_ids, hp[0], hp[1])
            n_layers += 1
        c_arr = array.array("Q", words or [0] * 5)
        _raise(lib().pf_engine_batch_save(self._h, instance_id.encode(), tp_rank, device_id,
                                          c_arr.buffer_info()[0], n_layers))
        del keep

    def batch_load_kv_blocks(self, instance_id: str, tp_rank: int, device_id: int,
                             load_state_shm: str, layer_names: Sequence[str],
                             block_ids: Sequence[int], block_hashes: Sequence[bytes]) -> None:
        """Queues a multi-layer load; completion is published in the LoadState.
        As in the reference (lib.rs:1008-1043), every hash is looked up and
        ids pair with hashes up to the shorter list: extra hashes get id -1
        (skipped), extra ids are dropped."""
        count = len(block_hashes)
        if len(block_ids) != count:
            block_ids = list(block_ids)[:count] + [-1] * max(0, count - len(block_ids))
        ids, ids_ptr, _ = _block_ids(block_ids)
        data, offs = _hashes(block_hashes)
        # A connector names the same layers on every load: their C array is
        # built once (the bytes objects it points into are kept with it).
        key = tuple(layer_names)
        c_names = self._name_arrays.get(key)
        if c_names is None:
            names = [n.encode() for n in key]
            c_names = (ctypes.c_char_p * max(len(names), 1))(*names)
            c_names._keep = names
            if len(self._name_arrays) >= 64:
                self._name_arrays.clear()
            self._name_arrays[key] = c_names
        _raise(lib().pf_engine_batch_load(
            self._h, instance_id.encode(), tp_rank, device_id, load_state_shm.encode(), c_names,
            len(key), ids_ptr, data.ctypes.data, offs.ctypes.data, count))
        del ids

    # -- disk tier (seal_offload.rs) -------------------------------------
    def enable_disk(self, root: str, quota_bytes: int = DEFAULT_DISK_QUOTA_BYTES,
                    max_pack_blocks: int = 64, max_prefetch_tasks: int = 16,
                    io_threads: int = 4) -> None:
        """Write every block sealed from now on to packed files under
        ``root`` (and index the files already there).  Call before saving."""
        _raise(lib().pf_engine_enable_disk(self._h, str(root).encode(), quota_bytes,
                                           max_pack_blocks, max_prefetch_tasks, io_threads))

    def count_prefix_hit_blocks_with_prefetch(self, instance_id: str,
                                              block_hashes: Sequence[bytes]) -> dict:
        """count_prefix_hit_blocks_async (lib.rs:855-941): {prefetch_state,
        hit_blocks, loading_blocks, missing_blocks}; a miss that is on disk
        starts reading the rest of the prefix into the pinned pool."""
        data, offs = _hashes(block_hashes)
        out = PrefetchStatus()
        _raise(lib().pf_engine_query_prefetch(self._h, instance_id.encode(), data.ctypes.data,
                                              offs.ctypes.data, len(offs) - 1, ctypes.byref(out)))
        return {"prefetch_state": PREFETCH_STATE_NAMES[out.state], "state": out.state,
                "hit_blocks": out.hit_blocks, "loading_blocks": out.loading_blocks,
                "missing_blocks": out.missing_blocks}

    def flush_disk(self) -> None:
        """Returns when every block queued for the disk is written."""
        _raise(lib().pf_engine_disk_flush(self._h))

    def wait_prefetch(self) -> None:
        """Returns when no disk read is in flight."""
        _raise(lib().pf_engine_disk_wait_prefetch(self._h))

    def disk_stats(self) -> dict:
        s = DiskStats()
        _raise(lib().pf_engine_disk_stats(self._h, ctypes.byref(s)))
        return {name: getattr(s, name) for name, _ in DiskStats._fields_}

    def read_block_slot(self, namespace: str, block_hash: bytes, slot: int) -> tuple[bytes, bytes]:
        """(K bytes, V bytes) of one slot of a cached block (V empty when the
        slot is contiguous)."""
        h = bytes(block_hash)
        k, v = ctypes.c_uint64(), ctypes.c_uint64()
        _raise(lib().pf_engine_read_block_slot(self._h, namespace.encode(), h, len(h), slot,
                                               None, 0, ctypes.byref(k), ctypes.byref(v)))
        buf = ctypes.create_string_buffer(k.value + v.value or 1)
        _raise(lib().pf_engine_read_block_slot(self._h, namespace.encode(), h, len(h), slot, buf,
                                               len(buf), ctypes.byref(k), ctypes.byref(v)))
        raw = buf.raw
        return raw[:k.value], raw[k.value:k.value + v.value]

    def stats(self) -> dict:
        s = EngineStats()
        _raise(lib().pf_engine_stats_get(self._h, ctypes.byref(s)))
        return {name: getattr(s, name) for name, _ in EngineStats._fields_}

    def wait_idle(self) -> None:
        _raise(lib().pf_engine_wait_idle(self._h))

    def serve_request(self, method: int, request: bytes) -> None:
        """One Load or Save request (method REQUEST_LOAD / REQUEST_SAVE) in
        engine.proto's encoding, decoded and served natively on this thread,
        as the native gRPC server serves one (pf_engine_serve_request)."""
        _raise(lib().pf_engine_serve_request(self._h, method, request, len(request)))

    def close(self) -> None:
        if self._h:
            lib().pf_engine_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
