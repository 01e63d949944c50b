"""ctypes binding of libpegaflow_hip.so (the C ABI in include/pegaflow_hip.h).

The library is loaded from this package directory.  There is no fallback: if
the library is missing, every entry point raises ``PegaFlowLibraryMissing``
so the product path can never silently run anything but the HIP code.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpegaflow_hip.so")

# Status codes (include/pegaflow_hip.h).
PF_OK = 0
PF_ERR_INVALID_ARGUMENT = 1
PF_ERR_HIP = 2
PF_ERR_STORAGE = 3
PF_ERR_INSTANCE_MISSING = 4
PF_ERR_WORKER_MISSING = 5
PF_ERR_TOPOLOGY_MISMATCH = 6
PF_ERR_INIT = 7
PF_ERR_LOAD_STATE = 8
PF_ERR_ZERO_SIZE = 9
PF_ERR_UNSUPPORTED = 10
PF_ERR_MALFORMED = 11

ERROR_NAMES = {
    PF_ERR_INVALID_ARGUMENT: "invalid argument",
    PF_ERR_HIP: "HIP error",
    PF_ERR_STORAGE: "storage error",
    PF_ERR_INSTANCE_MISSING: "instance missing",
    PF_ERR_WORKER_MISSING: "worker missing",
    PF_ERR_TOPOLOGY_MISMATCH: "topology mismatch",
    PF_ERR_INIT: "failed to initialize",
    PF_ERR_LOAD_STATE: "LoadState error",
    PF_ERR_ZERO_SIZE: "zero size",
    PF_ERR_UNSUPPORTED: "unsupported",
    PF_ERR_MALFORMED: "malformed request",
}

# Transfer modes.
MODE_DMA_REFERENCE = 0
MODE_DMA_BATCHED = 1
MODE_KERNEL = 2
MODE_STAGED = 3
MODE_AUTO = 4

# First layer of a layer-by-layer staged load (pf_xfer_set_staged_head).
STAGED_HEAD_KERNEL = 0
STAGED_HEAD_ENGINE = 1
MODE_NAMES = {
    "dma_reference": MODE_DMA_REFERENCE,
    "dma_batched": MODE_DMA_BATCHED,
    "kernel": MODE_KERNEL,
    "staged": MODE_STAGED,
    "auto": MODE_AUTO,
}

# Layout kinds.
LAYOUT_SPLIT, LAYOUT_CONTIGUOUS, LAYOUT_STRIDED = 0, 1, 2

# Request methods of pf_engine_serve_request (PF_REQUEST_*).
REQUEST_LOAD, REQUEST_SAVE, REQUEST_HEALTH = 1, 2, 3
REQUEST_MAX_BYTES = 256 << 20
# Chunks one pf_load_layers_noalloc call may plan (its static scratch).
NOALLOC_MAX_CHUNKS = 65536

# Pinned allocation flags.
PINNED_DEFAULT = 0
PINNED_COHERENT = 1
PINNED_NONCOHERENT = 2
PINNED_NUMA_USER = 4
PINNED_WRITE_COMBINED = 8

KERNEL_NT_LOADS = 0x100
KERNEL_NT_STORES = 0x200
KERNEL_NONTEMPORAL = KERNEL_NT_LOADS | KERNEL_NT_STORES
KERNEL_XCD_MAJOR = 0x400
# Scatter route only: time two candidate shapes, keep the faster.
KERNEL_AUTO = 0x800
SAVE_DEFAULT_SHAPE = (512, 1 | KERNEL_NONTEMPORAL)
LOAD_DEFAULT_SHAPE = (512, 2 | KERNEL_NONTEMPORAL | KERNEL_XCD_MAJOR | KERNEL_AUTO)
SAVE_HOST_DEFAULT_SHAPE = (512, 2 | KERNEL_NT_LOADS)
LOAD_HOST_DEFAULT_SHAPE = (512, 2 | KERNEL_NONTEMPORAL | KERNEL_XCD_MAJOR)
# Launch-shape routes (PF_ROUTE_*): direction x where the far side lives.
ROUTE_SAVE_DEVICE, ROUTE_LOAD_DEVICE, ROUTE_SAVE_HOST, ROUTE_LOAD_HOST = 0, 1, 2, 3
SAVE_HOST_DEFAULT_GRID, LOAD_HOST_DEFAULT_GRID = 32, 64
DEFAULT_GRIDS = {ROUTE_SAVE_DEVICE: 0, ROUTE_LOAD_DEVICE: 0,
                 ROUTE_SAVE_HOST: SAVE_HOST_DEFAULT_GRID, ROUTE_LOAD_HOST: LOAD_HOST_DEFAULT_GRID}
DEFAULT_SHAPES = {ROUTE_SAVE_DEVICE: SAVE_DEFAULT_SHAPE, ROUTE_LOAD_DEVICE: LOAD_DEFAULT_SHAPE,
                  ROUTE_SAVE_HOST: SAVE_HOST_DEFAULT_SHAPE, ROUTE_LOAD_HOST: LOAD_HOST_DEFAULT_SHAPE}

LOAD_PENDING, LOAD_SUCCESS, LOAD_ERROR = 0, 1, -1


class PegaFlowError(RuntimeError):
    """A failed C-ABI call: ``code`` is the PF_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class PegaFlowLibraryMissing(ImportError):
    pass


class KVLayout(ctypes.Structure):
    """pf_kv_layout — KVCacheRegistration (lib.rs:100-112)."""

    _fields_ = [
        ("data_ptr", ctypes.c_uint64),
        ("size_bytes", ctypes.c_uint64),
        ("num_blocks", ctypes.c_uint64),
        ("bytes_per_block", ctypes.c_uint64),
        ("block_size_bytes", ctypes.c_uint64),
        ("kv_stride_bytes", ctypes.c_uint64),
        ("segments", ctypes.c_uint64),
    ]


class BlockXfer(ctypes.Structure):
    """pf_block_xfer — SaveBlock / LoadBlock (gpu_worker.rs:25-49)."""

    _fields_ = [
        ("block_idx", ctypes.c_int64),
        ("k_host", ctypes.c_uint64),
        ("v_host", ctypes.c_uint64),
    ]


class LayerXfer(ctypes.Structure):
    """pf_layer_xfer — LayerLoadData (gpu_worker.rs:19-23)."""

    _fields_ = [
        ("layout", KVLayout),
        ("blocks", ctypes.c_void_p),
        ("num_blocks", ctypes.c_uint64),
    ]


class LayerSignal(ctypes.Structure):
    """pf_layer_signal — one target of a marked load's per-layer completion words."""

    _fields_ = [
        ("words", ctypes.c_uint64),
        ("value", ctypes.c_uint64),
        ("host_memory", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


MAX_LAYER_SIGNALS = 4
LAYER_WORDS_IPC, LAYER_WORDS_LOCAL = 0, 1


class LayerWords(ctypes.Structure):
    """pf_layer_words — a consumer's per-layer device words in a LoadState."""

    _fields_ = [
        ("kind", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("value", ctypes.c_uint64),
        ("address", ctypes.c_uint64),
        ("alloc_size", ctypes.c_uint64),
        ("offset", ctypes.c_uint64),
        ("handle", ctypes.c_uint8 * 64),
    ]


class SaveLayer(ctypes.Structure):
    """pf_save_layer — one (layer_name, block_ids, block_hashes) of a save batch."""

    _fields_ = [
        ("layer_name", ctypes.c_char_p),
        ("block_ids", ctypes.c_void_p),
        ("num_blocks", ctypes.c_uint64),
        ("hash_data", ctypes.c_void_p),
        ("hash_offsets", ctypes.c_void_p),
    ]


class EngineStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "pool_used_bytes", "pool_total_bytes", "sealed_blocks", "inflight_blocks",
        "evicted_blocks", "saved_bytes", "loaded_bytes", "load_failures",
        "admission_rejections", "pre_evicted_blocks")]


class PrefetchStatus(ctypes.Structure):
    _fields_ = [("state", ctypes.c_int32), ("reserved", ctypes.c_uint32),
                ("hit_blocks", ctypes.c_uint64), ("loading_blocks", ctypes.c_uint64),
                ("missing_blocks", ctypes.c_uint64)]


class DiskStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "files", "bytes", "indexed_blocks", "offloaded_blocks", "written_bytes",
        "prefetched_blocks", "read_bytes", "pending_blocks", "evicted_files", "failures")]


u64 = ctypes.c_uint64
i64 = ctypes.c_int64
u32 = ctypes.c_uint32
i32 = ctypes.c_int
vp = ctypes.c_void_p
pu64 = ctypes.POINTER(ctypes.c_uint64)
pi32 = ctypes.POINTER(ctypes.c_int)
pvp = ctypes.POINTER(ctypes.c_void_p)
pl = ctypes.POINTER(KVLayout)
cs = ctypes.c_char_p
# pf_grpc_handler: (ctx, call, method, request bytes, size).
GRPC_HANDLER = ctypes.CFUNCTYPE(None, vp, vp, cs, ctypes.POINTER(ctypes.c_uint8), u64)

# name -> (restype, argtypes).  Every symbol declared in the header.
SIGNATURES = {
    "pf_last_error": (cs, []),
    "pf_version": (cs, []),
    "pf_layout_init": (i32, [u64, u64, u64, u64, u64, u64, pl]),
    "pf_segment_offset": (i32, [pl, u64, u64, pu64]),
    "pf_is_contiguous_layout": (i32, [pl]),
    "pf_layout_kind": (i32, [pl]),
    "pf_get_device_count": (i32, [pi32]),
    "pf_init": (i32, [i32]),
    "pf_set_device": (i32, [i32]),
    "pf_get_device": (i32, [pi32]),
    "pf_device_synchronize": (i32, []),
    "pf_stream_create": (i32, [pvp]),
    "pf_stream_destroy": (i32, [vp]),
    "pf_stream_synchronize": (i32, [vp]),
    "pf_stream_wait_event": (i32, [vp, vp]),
    "pf_event_create": (i32, [pvp]),
    "pf_event_destroy": (i32, [vp]),
    "pf_event_record": (i32, [vp, vp]),
    "pf_event_synchronize": (i32, [vp]),
    "pf_event_query": (i32, [vp, pi32]),
    "pf_event_elapsed_ms": (i32, [vp, vp, ctypes.POINTER(ctypes.c_float)]),
    "pf_event_create_ipc": (i32, [pvp]),
    "pf_ipc_event_export": (i32, [vp, vp]),
    "pf_ipc_event_open": (i32, [vp, pvp]),
    "pf_device_malloc": (i32, [u64, pu64]),
    "pf_device_free": (i32, [u64]),
    "pf_memcpy_h2d": (i32, [u64, vp, u64]),
    "pf_memcpy_d2h": (i32, [vp, u64, u64]),
    "pf_memcpy_d2d": (i32, [u64, u64, u64]),
    "pf_memset_d8": (i32, [u64, ctypes.c_uint8, u64]),
    "pf_memcpy_async": (i32, [u64, u64, u64, vp]),
    "pf_device_pci_bus_id": (i32, [i32, ctypes.c_char_p, i32]),
    "pf_mem_get_info": (i32, [pu64, pu64]),
    "pf_pinned_allocate": (i32, [u64, u32, pvp, pu64]),
    "pf_pinned_free": (i32, [vp]),
    "pf_host_device_pointer": (i32, [vp, pu64]),
    "pf_huge_page_size": (u64, []),
    "pf_ipc_export": (i32, [u64, vp, pu64, pu64]),
    "pf_ipc_open": (i32, [vp, u64, pu64]),
    "pf_ipc_close": (i32, [u64]),
    "pf_copy_gpu_to_cpu": (i32, [u64, u64, vp, u64, u64]),
    "pf_copy_cpu_to_gpu_async": (i32, [u64, u64, vp, u64, u64, vp]),
    "pf_batch_copy_segments_to_gpu": (i32, [pu64, pu64, u64, u64, pl, vp, pu64]),
    "pf_count_merged_runs": (u64, [pu64, pu64, u64, u64]),
    "pf_copy_block_gpu_to_cpu": (i32, [pl, u64, vp]),
    "pf_xfer_create": (i32, [i32, u64, pvp]),
    "pf_xfer_destroy": (i32, [vp]),
    "pf_xfer_stream": (vp, [vp]),
    "pf_xfer_synchronize": (i32, [vp]),
    "pf_xfer_set_kernel_shape": (i32, [vp, u32, u32]),
    "pf_xfer_last_stats": (i32, [vp, pu64, pu64]),
    "pf_xfer_set_max_grid": (i32, [vp, u32]),
    "pf_xfer_set_staged_slices": (i32, [vp, u64, u64]),
    "pf_copy_engines": (i32, [i32, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)]),
    "pf_set_copy_engines": (i32, [i32, u32, u32]),
    "pf_xfer_set_kernel_shape_dir": (i32, [vp, u32, u32, u32]),
    "pf_xfer_route_shape": (i32, [vp, u32, ctypes.POINTER(u32), ctypes.POINTER(u32),
                                  ctypes.POINTER(i32)]),
    "pf_xfer_set_route_grid": (i32, [vp, u32, u32]),
    "pf_xfer_set_staged_head": (i32, [vp, u32]),
    "pf_xfer_set_cu_mask": (i32, [vp, ctypes.POINTER(ctypes.c_uint32), u32]),
    "pf_cu_mask_per_xcd": (i32, [i32, u32, ctypes.POINTER(ctypes.c_uint32), u32]),
    "pf_xfer_set_timing": (i32, [vp, i32]),
    "pf_xfer_last_kernel_ms": (i32, [vp, ctypes.POINTER(ctypes.c_float), pu64]),
    "pf_save_layers": (i32, [vp, ctypes.POINTER(LayerXfer), u32, u32]),
    "pf_load_layers": (i32, [vp, ctypes.POINTER(LayerXfer), u32, u32, pvp]),
    "pf_load_layers_noalloc": (i32, [vp, ctypes.POINTER(LayerXfer), u32]),
    "pf_load_layers_marked": (i32, [vp, ctypes.POINTER(LayerXfer), u32, u32,
                                    ctypes.POINTER(LayerSignal), u32]),
    "pf_stream_wait_word": (i32, [vp, u64, u64, u32, u64]),
    "pf_host_wait_word": (i32, [vp, u64, u64, pi32]),
    "pf_fill_random": (i32, [u64, u64, u64, u64, vp]),
    "pf_verify_random": (i32, [u64, u64, u64, u64, pu64]),
    "pf_verify_random_chunks": (i32, [pu64, pu64, u64, u64, u64, pu64]),
    "pf_compare": (i32, [u64, u64, u64, pu64]),
    "pf_spin": (i32, [vp, u32]),
    "pf_load_state_create": (i32, [pvp]),
    "pf_load_state_create_layered": (i32, [u32, pvp]),
    "pf_load_state_attach": (i32, [cs, pvp]),
    "pf_load_state_close": (i32, [vp]),
    "pf_load_state_name": (cs, [vp]),
    "pf_load_state_get": (i64, [vp]),
    "pf_load_state_set_completed": (None, [vp]),
    "pf_load_state_set_error": (None, [vp]),
    "pf_load_state_num_layers": (u32, [vp]),
    "pf_load_state_layers_done": (i64, [vp]),
    "pf_load_state_set_layers_done": (None, [vp, i64]),
    "pf_load_state_create_layered_events": (i32, [u32, vp, pvp]),
    "pf_load_state_event_handles": (vp, [vp, ctypes.POINTER(ctypes.c_uint32)]),
    "pf_load_state_create_layered_local_events": (i32, [u32, ctypes.POINTER(vp), vp]),
    "pf_load_state_events_local": (i32, [vp]),
    "pf_load_state_events_recorded": (i64, [vp]),
    "pf_load_state_set_events_recorded": (None, [vp, i64]),
    "pf_load_state_create_layered_words": (i32, [u32, ctypes.POINTER(LayerWords), pvp]),
    "pf_load_state_layer_words": (i32, [vp, ctypes.POINTER(LayerWords),
                                        ctypes.POINTER(ctypes.c_uint32)]),
    "pf_allocator_create": (i32, [u64, u64, pvp]),
    "pf_allocator_create_auto": (i32, [u64, pvp]),
    "pf_allocator_destroy": (i32, [vp]),
    "pf_allocator_allocate": (i32, [vp, u64, pi32, pu64, pu64]),
    "pf_allocator_free": (i32, [vp, u64]),
    "pf_allocator_report": (i32, [vp, pu64, pu64, pu64, pu64]),
    "pf_engine_create": (i32, [u64, u32, u32, u64, pvp]),
    "pf_engine_destroy": (i32, [vp]),
    "pf_engine_set_modes": (i32, [vp, u32, u32]),
    "pf_engine_set_storage_policy": (i32, [vp, i32, u64, i32, u64, u64, u32]),
    "pf_engine_register_context_layer": (i32, [vp, cs, cs, i32, cs, u64, u64, u64, u64, u64,
                                               u64, u64, u64, u64]),
    "pf_engine_unregister_instance": (i32, [vp, cs]),
    "pf_engine_count_prefix_hit_blocks": (i32, [vp, cs, vp, vp, u64, pu64]),
    # The layers: the address of a pf_save_layer array (SaveLayer's layout).
    "pf_engine_batch_save": (i32, [vp, cs, u64, i32, vp, u32]),
    "pf_engine_batch_load": (i32, [vp, cs, u64, i32, cs, ctypes.POINTER(cs), u32, vp, vp, vp,
                                   u64]),
    "pf_engine_serve_request": (i32, [vp, u32, ctypes.c_char_p, u64]),
    "pf_grpc_start": (i32, [vp, cs, GRPC_HANDLER, vp, pvp]),
    "pf_grpc_port": (i32, [vp]),
    "pf_grpc_served": (u64, [vp]),
    "pf_grpc_reply": (i32, [vp, u32, cs, cs, u64]),
    "pf_grpc_stop": (i32, [vp]),
    "pf_engine_stats_get": (i32, [vp, ctypes.POINTER(EngineStats)]),
    "pf_engine_wait_idle": (i32, [vp]),
    "pf_engine_enable_disk": (i32, [vp, cs, u64, u32, u32, u32]),
    "pf_engine_query_prefetch": (i32, [vp, cs, vp, vp, u64, ctypes.POINTER(PrefetchStatus)]),
    "pf_engine_disk_flush": (i32, [vp]),
    "pf_engine_disk_wait_prefetch": (i32, [vp]),
    "pf_engine_disk_stats": (i32, [vp, ctypes.POINTER(DiskStats)]),
    "pf_engine_read_block_slot": (i32, [vp, cs, vp, u64, u64, vp, u64, pu64, pu64]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load and bind the library (once)."""
    global _lib
    if _lib is not None:  # bound already: no lock on the per-call path
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise PegaFlowLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m pegaflow_amd.build`"
            )
        L = ctypes.CDLL(LIB_PATH, mode=os.RTLD_LOCAL | os.RTLD_NOW)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
        return _lib


def last_error() -> str:
    return load().pf_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    if rc != PF_OK:
        msg = last_error()
        prefix = ERROR_NAMES.get(rc, f"error {rc}")
        raise PegaFlowError(rc, f"{what + ': ' if what else ''}{prefix}: {msg}")
