"""Layer-tensor handles passed in RegisterContextRequest.wrapper_bytes.

The reference pickles a torch ``CudaIPCWrapper`` (ipc_wrapper.py:101-156) and
the server unpickles it and opens the CUDA-IPC handle through torch
(registry.rs:144-175).  Here the bytes are a fixed little-endian record that
never executes anything when read:

    offset  size  field
    0       8     magic  b"PFIPC1\\0\\0" (HIP IPC handle) | b"PFPTR1\\0\\0" (address
                  valid only inside the server's own process)
    8       4     device_id (i32)
    12      4     reserved (0)
    16      8     allocation size in bytes (u64)
    24      8     byte offset of the tensor inside the allocation (u64)
    32      8     tensor size in bytes (u64)
    40      64    hipIpcMemHandle_t (PFIPC1) | u64 address + zeros (PFPTR1)

Allocations of 2 GiB or more cannot be shared across processes here.
"""

from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass

from . import _lib
from ._lib import check

MAGIC_IPC = b"PFIPC1\0\0"
MAGIC_PTR = b"PFPTR1\0\0"
_HEAD = struct.Struct("<8siIQQQ")
RECORD_BYTES = _HEAD.size + 64
MAX_ALLOC_BYTES = 1 << 31


def lib():
    return _lib.load()


def export_tensor(data_ptr: int, nbytes: int, device_id: int) -> bytes:
    """Handle of a device tensor for another process (hipIpcGetMemHandle on
    the allocation that contains it)."""
    h = (ctypes.c_uint8 * 64)()
    base, size = ctypes.c_uint64(), ctypes.c_uint64()
    check(lib().pf_ipc_export(data_ptr, h, ctypes.byref(base), ctypes.byref(size)),
          "pf_ipc_export")
    offset = data_ptr - base.value
    if offset + nbytes > size.value:
        raise ValueError("tensor extends past its allocation")
    return _HEAD.pack(MAGIC_IPC, device_id, 0, size.value, offset, nbytes) + bytes(h)


def export_torch_tensor(tensor) -> bytes:
    """Handle of a torch tensor, from torch's own IPC export, without loading
    this library into the torch process.  The tensor must start at storage
    offset 0, as the reference requires (worker.py:93-95)."""
    if tensor.storage_offset() != 0:
        raise ValueError("KV cache tensor must have zero storage offset")
    storage = tensor.untyped_storage()
    shared = storage._share_cuda_()
    device, handle, size_bytes, offset_bytes = shared[0], shared[1], shared[2], shared[3]
    handle = bytes(handle)
    if len(handle) < 64:
        raise ValueError(f"unexpected IPC handle of {len(handle)} bytes")
    alloc = offset_bytes + size_bytes
    return _HEAD.pack(MAGIC_IPC, int(device), 0, alloc, offset_bytes,
                      tensor.numel() * tensor.element_size()) + handle[:64]


def local_tensor(data_ptr: int, nbytes: int, device_id: int) -> bytes:
    """Handle of a device tensor for a server running in this same process."""
    return (_HEAD.pack(MAGIC_PTR, device_id, 0, nbytes, 0, nbytes)
            + struct.pack("<Q", data_ptr) + bytes(56))


@dataclass
class OpenedTensor:
    """A registered layer tensor on the server side (TensorMetadata,
    registry.rs:6-11) plus the mapping that keeps it alive."""

    data_ptr: int
    size_bytes: int
    device_id: int
    mapped_base: int = 0  # non-zero when opened through IPC

    def close(self) -> None:
        if self.mapped_base:
            lib().pf_ipc_close(self.mapped_base)
            self.mapped_base = 0


def parse(wrapper_bytes: bytes):
    """(magic, device_id, alloc_size, offset, nbytes, payload) of a record."""
    if len(wrapper_bytes) != RECORD_BYTES:
        raise ValueError(f"tensor handle must be {RECORD_BYTES} bytes, got {len(wrapper_bytes)}")
    magic, device, _, alloc, offset, nbytes = _HEAD.unpack_from(wrapper_bytes)
    if magic not in (MAGIC_IPC, MAGIC_PTR):
        raise ValueError("not a pegaflow tensor handle")
    if offset + nbytes > alloc:
        raise ValueError("tensor extends past its allocation")
    return magic, device, alloc, offset, nbytes, wrapper_bytes[_HEAD.size:]


def open_tensor(wrapper_bytes: bytes) -> OpenedTensor:
    magic, device, alloc, offset, nbytes, payload = parse(wrapper_bytes)
    if magic == MAGIC_PTR:
        (ptr,) = struct.unpack_from("<Q", payload)
        return OpenedTensor(ptr + offset, nbytes, device)
    if alloc >= MAX_ALLOC_BYTES:
        raise ValueError(f"shared allocation of {alloc} bytes exceeds the 2 GiB limit")
    check(lib().pf_set_device(device), "pf_set_device")
    h = (ctypes.c_uint8 * 64).from_buffer_copy(payload)
    base = ctypes.c_uint64()
    check(lib().pf_ipc_open(h, alloc, ctypes.byref(base)), "pf_ipc_open")
    return OpenedTensor(base.value + offset, nbytes, device, mapped_base=base.value)
