"""Transfer module: layouts, the reference's transfer primitives, and the
batched gather/scatter transfer context (HIP kernels, staged DMA, DMA batches).

Mirrors pegaflow-core/src/transfer.rs and the copy loops of
pegaflow-core/src/gpu_worker.rs:205-390, over libpegaflow_hip.so.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Iterable, Sequence

import numpy as np

from . import _lib
from ._lib import BlockXfer, KVLayout, LayerXfer, check
from .runtime import Event, Stream

BLOCK_DTYPE = np.dtype([("block_idx", "<i8"), ("k_host", "<u8"), ("v_host", "<u8")])
assert BLOCK_DTYPE.itemsize == ctypes.sizeof(BlockXfer)


def lib():
    return _lib.load()


@dataclass(frozen=True)
class KVCacheRegistration:
    """Layout of one registered layer tensor (lib.rs:100-112)."""

    data_ptr: int
    size_bytes: int
    num_blocks: int
    bytes_per_block: int
    block_size_bytes: int
    kv_stride_bytes: int
    segments: int

    @classmethod
    def create(cls, data_ptr: int, size_bytes: int, num_blocks: int, bytes_per_block: int,
               kv_stride_bytes: int, segments: int) -> "KVCacheRegistration":
        """Validated as register_context_layer does (lib.rs:389-449)."""
        out = KVLayout()
        check(lib().pf_layout_init(data_ptr, size_bytes, num_blocks, bytes_per_block,
                                   kv_stride_bytes, segments, ctypes.byref(out)),
              "register layout")
        return cls.from_c(out)

    @classmethod
    def from_c(cls, c: KVLayout) -> "KVCacheRegistration":
        return cls(c.data_ptr, c.size_bytes, c.num_blocks, c.bytes_per_block,
                   c.block_size_bytes, c.kv_stride_bytes, c.segments)

    def to_c(self) -> KVLayout:
        return KVLayout(self.data_ptr, self.size_bytes, self.num_blocks,
                        self.bytes_per_block, self.block_size_bytes,
                        self.kv_stride_bytes, self.segments)

    @property
    def kind(self) -> int:
        return lib().pf_layout_kind(ctypes.byref(self.to_c()))

    @property
    def is_split(self) -> bool:
        return self.segments == 2 and self.kv_stride_bytes > self.bytes_per_block


def derive_layout(shape: Sequence[int], stride: Sequence[int], element_size: int):
    """(num_blocks, bytes_per_block, kv_stride_bytes, segments) of a KV tensor.

    worker.py:104-115: a leading dimension of 2 is the KV-first layout
    [2, num_blocks, ...] (two segments, K then V); otherwise the tensor is
    blocks-first [num_blocks, ...] with one segment per block.
    """
    shape = tuple(int(s) for s in shape)
    stride = tuple(int(s) for s in stride)
    if len(shape) >= 2 and shape[0] == 2:
        num_blocks = shape[1]
        bytes_per_block = stride[1] * element_size
        kv_stride_bytes = stride[0] * element_size
        segments = 2
    else:
        num_blocks = shape[0]
        bytes_per_block = stride[0] * element_size
        kv_stride_bytes = 0
        segments = 1
    if bytes_per_block == 0:
        raise ValueError(f"Invalid bytes_per_block: stride={stride}")
    return num_blocks, bytes_per_block, kv_stride_bytes, segments


def segment_offset(reg: KVCacheRegistration, block_idx: int, segment_idx: int) -> int:
    """transfer.rs:18-47."""
    out = ctypes.c_uint64()
    check(lib().pf_segment_offset(ctypes.byref(reg.to_c()), block_idx, segment_idx,
                                  ctypes.byref(out)), "segment_offset")
    return out.value


def is_contiguous_layout(reg: KVCacheRegistration) -> bool:
    """transfer.rs:50-52."""
    return bool(lib().pf_is_contiguous_layout(ctypes.byref(reg.to_c())))


def copy_gpu_to_cpu(gpu_base: int, offset: int, cpu_buffer: np.ndarray, size: int) -> None:
    """Synchronous device -> host copy (transfer.rs:56-76)."""
    check(lib().pf_copy_gpu_to_cpu(gpu_base, offset, cpu_buffer.ctypes.data,
                                   cpu_buffer.nbytes, size), "copy_gpu_to_cpu")


def copy_cpu_to_gpu_async(gpu_base: int, offset: int, cpu_buffer: np.ndarray, size: int,
                          stream: Stream) -> None:
    """Asynchronous host -> device copy (transfer.rs:80-113)."""
    check(lib().pf_copy_cpu_to_gpu_async(gpu_base, offset, cpu_buffer.ctypes.data,
                                         cpu_buffer.nbytes, size, stream.handle),
          "copy_cpu_to_gpu_async")


def _u64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def batch_copy_segments_to_gpu(transfers_gpu_offsets, transfers_cpu_ptrs, segment_size: int,
                               reg: KVCacheRegistration, stream: Stream) -> int:
    """Merged-run async H2D copies (transfer.rs:116-198); returns copies issued."""
    g, c = _u64(transfers_gpu_offsets), _u64(transfers_cpu_ptrs)
    assert len(g) == len(c)
    out = ctypes.c_uint64()
    pu = ctypes.POINTER(ctypes.c_uint64)
    check(lib().pf_batch_copy_segments_to_gpu(g.ctypes.data_as(pu), c.ctypes.data_as(pu),
                                              len(g), segment_size, ctypes.byref(reg.to_c()),
                                              stream.handle, ctypes.byref(out)),
          "batch_copy_segments_to_gpu")
    return out.value


def count_merged_runs(gpu_offsets, cpu_ptrs, segment_size: int) -> int:
    g, c = _u64(gpu_offsets), _u64(cpu_ptrs)
    pu = ctypes.POINTER(ctypes.c_uint64)
    return int(lib().pf_count_merged_runs(g.ctypes.data_as(pu), c.ctypes.data_as(pu),
                                          len(g), segment_size))


def copy_block_gpu_to_cpu(reg: KVCacheRegistration, block_idx: int, dst: np.ndarray) -> None:
    """transfer.rs:201-239."""
    assert dst.nbytes >= reg.block_size_bytes
    check(lib().pf_copy_block_gpu_to_cpu(ctypes.byref(reg.to_c()), block_idx,
                                         dst.ctypes.data), "copy_block_gpu_to_cpu")


def block_array(block_idx, k_host, v_host=None) -> np.ndarray:
    """Structured array of pf_block_xfer records."""
    b = np.asarray(block_idx, dtype=np.int64)
    out = np.zeros(len(b), BLOCK_DTYPE)
    out["block_idx"] = b
    out["k_host"] = np.asarray(k_host, dtype=np.uint64)
    if v_host is not None:
        out["v_host"] = np.asarray(v_host, dtype=np.uint64)
    return out


@dataclass
class LayerTransfer:
    """Blocks of one layer: registration + block_idx / k_host / v_host."""

    registration: KVCacheRegistration
    blocks: np.ndarray  # BLOCK_DTYPE

    def __getstate__(self):  # the cached C struct points into this process
        state = dict(self.__dict__)
        state.pop("_c", None)
        return state


def _layer_c(lt: LayerTransfer):
    """The layer's pf_layer_xfer and the block array it points into, made
    once per (registration, blocks array) pair and kept on the object: a
    caller that passes the same layers each step (a worker's registered
    layers) pays the marshalling once.  The array is held with the struct,
    so the pointer stays valid; its contents may change between calls."""
    c = lt.__dict__.get("_c")
    if c is not None and c[0] is lt.blocks and c[1] is lt.registration:
        return c[2], c[3]
    b = np.ascontiguousarray(lt.blocks, dtype=BLOCK_DTYPE)
    x = LayerXfer()
    x.layout = lt.registration.to_c()
    x.blocks = b.ctypes.data if len(b) else None
    x.num_blocks = len(b)
    lt.__dict__["_c"] = (lt.blocks, lt.registration, x, b)
    return x, b


def _layer_array(layers: Sequence[LayerTransfer]):
    arr = (LayerXfer * max(len(layers), 1))()
    keep = []
    for i, lt in enumerate(layers):
        x, b = _layer_c(lt)
        arr[i] = x
        keep.append(b)
    return arr, keep


def load_layers_noalloc(layers: Sequence[LayerTransfer], stream: Stream | None = None) -> None:
    """pf_load_layers_noalloc: the kernel-mode load of ``layers`` on ``stream``
    (the current device's null stream when None) with no device allocation;
    asynchronous.  At most ``_lib.NOALLOC_MAX_CHUNKS`` chunks per call."""
    arr, keep = _layer_array(layers)
    check(lib().pf_load_layers_noalloc(stream.handle if stream is not None else None, arr,
                                       len(layers)), "load_layers_noalloc")
    del keep


def cu_mask_per_xcd(cus_per_xcd: int, device: int = 0, words: int = 8):
    """A CU mask with `cus_per_xcd` compute units on each XCD of `device`
    (pf_cu_mask_per_xcd), as a list of 32-bit words."""
    arr = (ctypes.c_uint32 * words)()
    check(lib().pf_cu_mask_per_xcd(device, cus_per_xcd, arr, words), "pf_cu_mask_per_xcd")
    return list(arr)


class TransferContext:
    """A pf_xfer: per-worker streams, descriptor buffers and staging slots."""

    def __init__(self, device: int = 0, staging_bytes: int = 0):
        h = ctypes.c_void_p()
        check(lib().pf_xfer_create(device, staging_bytes, ctypes.byref(h)), "pf_xfer_create")
        self.handle = h.value
        self.device = device
        self.stream = Stream(lib().pf_xfer_stream(self.handle), owned=False)

    def set_kernel_shape(self, threads: int = 0, unroll: int = 0) -> None:
        check(lib().pf_xfer_set_kernel_shape(self.handle, threads, unroll),
              "pf_xfer_set_kernel_shape")

    def synchronize(self) -> None:
        check(lib().pf_xfer_synchronize(self.handle), "pf_xfer_synchronize")

    def last_stats(self):
        k, d = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().pf_xfer_last_stats(self.handle, ctypes.byref(k), ctypes.byref(d)),
              "pf_xfer_last_stats")
        return k.value, d.value

    def set_kernel_shape_dir(self, direction: int, threads: int = 0, unroll: int = 0) -> None:
        """Shape of one route (``_lib.ROUTE_*``): 0 = saves into device memory
        (gather), 1 = loads from device memory (scatter), 2 = saves into
        pinned host memory, 3 = loads from pinned host memory."""
        check(lib().pf_xfer_set_kernel_shape_dir(self.handle, direction, threads, unroll),
              "pf_xfer_set_kernel_shape_dir")

    def set_route_grid(self, route: int, workgroups: int) -> None:
        """Persistent workgroups pulling tiles from a queue on this route (0:
        one workgroup per tile)."""
        check(lib().pf_xfer_set_route_grid(self.handle, route, workgroups),
              "pf_xfer_set_route_grid")

    def route_shape(self, route: int):
        """(threads, unroll, decided): the shape the route's next fixed-map
        launch uses (for an automatic scatter route, the chosen candidate once
        decided)."""
        t, u, d = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_int()
        check(lib().pf_xfer_route_shape(self.handle, route, ctypes.byref(t), ctypes.byref(u),
                                        ctypes.byref(d)), "pf_xfer_route_shape")
        return t.value, u.value, bool(d.value)

    def reset_kernel_shape(self) -> None:
        """Back to the per-route defaults (shapes and work distribution)."""
        for route, shape in _lib.DEFAULT_SHAPES.items():
            self.set_kernel_shape_dir(route, *shape)
        for route, grid in _lib.DEFAULT_GRIDS.items():
            self.set_route_grid(route, grid)

    def set_staged_slices(self, save_bytes: int = 0, load_bytes: int = 0) -> None:
        """Largest staged slice per direction (0 keeps the current value;
        pf_xfer_set_staged_slices).  A load's slices start at a quarter of
        its largest and double."""
        check(lib().pf_xfer_set_staged_slices(self.handle, save_bytes, load_bytes),
              "pf_xfer_set_staged_slices")

    def set_staged_head(self, route: int) -> None:
        """How a staged load waited for layer by layer copies its first layer:
        _lib.STAGED_HEAD_ENGINE (copy engines, the default) or
        _lib.STAGED_HEAD_KERNEL (zero-copy kernel; pf_xfer_set_staged_head)."""
        check(lib().pf_xfer_set_staged_head(self.handle, route), "pf_xfer_set_staged_head")

    def set_cu_mask(self, mask=None) -> None:
        """Compute units this context's kernels run on (pf_xfer_set_cu_mask):
        a sequence of 32-bit words, bit b enabling CU b (on XCD b mod the
        XCD count), or None for unmasked streams.  Waits for the context's
        work and replaces its streams, `self.stream` included."""
        words = list(mask or [])
        arr = (ctypes.c_uint32 * max(1, len(words)))(*words)
        check(lib().pf_xfer_set_cu_mask(self.handle, arr, len(words)), "pf_xfer_set_cu_mask")
        self.stream = Stream(lib().pf_xfer_stream(self.handle), owned=False)

    def set_max_grid(self, max_workgroups: int) -> None:
        check(lib().pf_xfer_set_max_grid(self.handle, max_workgroups), "pf_xfer_set_max_grid")

    def set_timing(self, enable: bool) -> None:
        check(lib().pf_xfer_set_timing(self.handle, int(enable)), "pf_xfer_set_timing")

    def last_kernel_ms(self):
        """(summed kernel ms, launches) of the last call, with timing enabled."""
        ms, n = ctypes.c_float(), ctypes.c_uint64()
        check(lib().pf_xfer_last_kernel_ms(self.handle, ctypes.byref(ms), ctypes.byref(n)),
              "pf_xfer_last_kernel_ms")
        return float(ms.value), n.value

    def save_layers(self, layers: Sequence[LayerTransfer], mode: int = _lib.MODE_KERNEL) -> None:
        """Device -> host for every layer; returns when bytes are in place."""
        arr, keep = _layer_array(layers)
        check(lib().pf_save_layers(self.handle, arr, len(layers), mode), "save_layers")
        del keep

    def load_layers(self, layers: Sequence[LayerTransfer], mode: int = _lib.MODE_KERNEL,
                    layer_events: Iterable[Event] | None = None) -> None:
        """Host -> device for every layer; asynchronous on the context's streams."""
        arr, keep = _layer_array(layers)
        evs = None
        if layer_events is not None:
            ev_list = list(layer_events)
            assert len(ev_list) == len(layers)
            evs = (ctypes.c_void_p * max(len(ev_list), 1))(*[e.handle for e in ev_list])
        check(lib().pf_load_layers(self.handle, arr, len(layers), mode, evs), "load_layers")
        del keep

    def load_layers_marked(self, layers: Sequence[LayerTransfer], signals,
                           mode: int = _lib.MODE_KERNEL) -> None:
        """Host -> device for every layer, asynchronous; ``signals`` is a list of
        ``(words_addr, value, host_memory)``: once layer l's bytes are in place,
        the 8-byte word at ``words_addr + 8*l`` of each target holds ``value``."""
        arr, keep = _layer_array(layers)
        sig = (_lib.LayerSignal * max(len(signals), 1))()
        for i, (words, value, host_memory) in enumerate(signals):
            sig[i].words = words
            sig[i].value = value
            sig[i].host_memory = int(bool(host_memory))
        check(lib().pf_load_layers_marked(self.handle, arr, len(layers), mode, sig,
                                          len(signals)), "load_layers_marked")
        del keep

    def close(self) -> None:
        if self.handle:
            lib().pf_xfer_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
