"""Device runtime objects over the C ABI: streams, events, device buffers and
pinned host buffers, plus the synthetic-data and verification kernels.

These are thin owners of HIP resources created by libpegaflow_hip.so; no
framework tensors are involved.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check


def lib():
    return _lib.load()


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib().pf_get_device_count(ctypes.byref(n)), "pf_get_device_count")
    return n.value


def init(device: int = 0) -> None:
    check(lib().pf_init(device), "pf_init")


def synchronize() -> None:
    check(lib().pf_device_synchronize(), "pf_device_synchronize")


def pci_bus_id(device: int = 0) -> str:
    """The device's PCI address, "dddd:bb:dd.f"."""
    buf = ctypes.create_string_buffer(64)
    check(lib().pf_device_pci_bus_id(device, buf, len(buf)), "pf_device_pci_bus_id")
    return buf.value.decode()


def copy_engines(device: int = 0):
    """(d2h, h2d): the copy-engine id bits the staged mode's copies use on
    the device (0, 0 when unknown)."""
    d, h = ctypes.c_uint32(), ctypes.c_uint32()
    check(lib().pf_copy_engines(device, ctypes.byref(d), ctypes.byref(h)), "pf_copy_engines")
    return d.value, h.value


def set_copy_engines(device: int = 0, d2h: int = 0, h2d: int = 0) -> None:
    """Chooses the staged mode's copy engines on the device: per direction a
    mask of one or two engine id bits (0 keeps that direction's choice)."""
    check(lib().pf_set_copy_engines(device, d2h, h2d), "pf_set_copy_engines")


def mem_get_info():
    f, t = ctypes.c_uint64(), ctypes.c_uint64()
    check(lib().pf_mem_get_info(ctypes.byref(f), ctypes.byref(t)), "pf_mem_get_info")
    return f.value, t.value


class Stream:
    """A non-blocking HIP stream at the default priority."""

    def __init__(self, handle=None, owned: bool = True):
        if handle is None:
            h = ctypes.c_void_p()
            check(lib().pf_stream_create(ctypes.byref(h)), "pf_stream_create")
            handle = h.value
        self.handle = handle
        self._owned = owned and handle is not None

    def synchronize(self) -> None:
        check(lib().pf_stream_synchronize(self.handle), "pf_stream_synchronize")

    def wait_event(self, ev: "Event") -> None:
        check(lib().pf_stream_wait_event(self.handle, ev.handle), "pf_stream_wait_event")

    def close(self) -> None:
        if self._owned and self.handle:
            lib().pf_stream_destroy(self.handle)
        self.handle = None
        self._owned = False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    """A timing-capable HIP event, or with ``interprocess=True`` one without
    timing whose handle another process can open (``ipc_handle`` /
    ``Event.from_ipc_handle``)."""

    def __init__(self, interprocess: bool = False, _handle=None):
        if _handle is not None:
            self.handle = _handle
            return
        h = ctypes.c_void_p()
        if interprocess:
            check(lib().pf_event_create_ipc(ctypes.byref(h)), "pf_event_create_ipc")
        else:
            check(lib().pf_event_create(ctypes.byref(h)), "pf_event_create")
        self.handle = h.value

    def ipc_handle(self) -> bytes:
        buf = (ctypes.c_uint8 * 64)()
        check(lib().pf_ipc_event_export(self.handle, buf), "pf_ipc_event_export")
        return bytes(buf)

    @classmethod
    def from_ipc_handle(cls, handle: bytes) -> "Event":
        """Opens an event exported by another process."""
        if len(handle) != 64:
            raise ValueError("an event handle is 64 bytes")
        buf = (ctypes.c_uint8 * 64).from_buffer_copy(handle)
        h = ctypes.c_void_p()
        check(lib().pf_ipc_event_open(buf, ctypes.byref(h)), "pf_ipc_event_open")
        return cls(_handle=h.value)

    def record(self, stream: Stream | None = None) -> None:
        check(lib().pf_event_record(self.handle, stream.handle if stream else None),
              "pf_event_record")

    def synchronize(self) -> None:
        check(lib().pf_event_synchronize(self.handle), "pf_event_synchronize")

    def query(self) -> bool:
        d = ctypes.c_int(0)
        check(lib().pf_event_query(self.handle, ctypes.byref(d)), "pf_event_query")
        return bool(d.value)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().pf_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)),
              "pf_event_elapsed_ms")
        return float(ms.value)

    def close(self) -> None:
        if self.handle:
            lib().pf_event_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """Device memory from hipMalloc."""

    def __init__(self, nbytes: int):
        p = ctypes.c_uint64()
        check(lib().pf_device_malloc(nbytes, ctypes.byref(p)), "pf_device_malloc")
        self.ptr = p.value
        self.nbytes = nbytes

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().pf_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes),
              "pf_memcpy_h2d")

    def download(self, nbytes: int | None = None, offset: int = 0) -> np.ndarray:
        n = self.nbytes - offset if nbytes is None else nbytes
        assert offset + n <= self.nbytes
        out = np.empty(n, np.uint8)
        check(lib().pf_memcpy_d2h(out.ctypes.data, self.ptr + offset, n), "pf_memcpy_d2h")
        return out

    def fill_random(self, seed: int, word_offset: int = 0, stream: Stream | None = None,
                    nbytes: int | None = None, offset: int = 0) -> None:
        """Fill with splitmix64 words.  Without a stream the fill runs on the
        null stream and is waited for: the transfer contexts' streams are
        non-blocking and would not order after it."""
        n = self.nbytes - offset if nbytes is None else nbytes
        check(lib().pf_fill_random(self.ptr + offset, n, seed % 2**64, word_offset,
                                   stream.handle if stream else None), "pf_fill_random")
        if stream is None:
            synchronize()

    def memset(self, value: int) -> None:
        check(lib().pf_memset_d8(self.ptr, value, self.nbytes), "pf_memset_d8")
        synchronize()

    def close(self) -> None:
        if self.ptr:
            lib().pf_device_free(self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PinnedBuffer:
    """Pinned host memory from hipHostMalloc, mapped for device access.

    ``array`` is a uint8 numpy view of the allocation; ``ptr`` is both its
    host address and the address kernels use for zero-copy access.
    """

    def __init__(self, nbytes: int, flags: int = _lib.PINNED_DEFAULT):
        h = ctypes.c_void_p()
        d = ctypes.c_uint64()
        check(lib().pf_pinned_allocate(nbytes, flags, ctypes.byref(h), ctypes.byref(d)),
              "pf_pinned_allocate")
        self.ptr = h.value
        self.dev_ptr = d.value
        self.nbytes = nbytes
        self.array = np.ctypeslib.as_array(
            ctypes.cast(self.ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(nbytes,))

    def close(self) -> None:
        if self.ptr:
            self.array = None
            lib().pf_pinned_free(self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fill_random(addr: int, nbytes: int, seed: int, word_offset: int = 0,
                stream: Stream | None = None) -> None:
    """As DeviceBuffer.fill_random: waited for when no stream is given."""
    check(lib().pf_fill_random(addr, nbytes, seed % 2**64, word_offset,
                               stream.handle if stream else None), "pf_fill_random")
    if stream is None:
        synchronize()


def verify_random(addr: int, nbytes: int, seed: int, word_offset: int = 0) -> int:
    """Count of 8-byte words at addr that differ from the fill formula."""
    out = ctypes.c_uint64()
    check(lib().pf_verify_random(addr, nbytes, seed % 2**64, word_offset, ctypes.byref(out)),
          "pf_verify_random")
    return out.value


def verify_random_chunks(addrs, word_offsets, chunk_bytes: int, seed: int) -> int:
    """Batched verify: chunk i at addrs[i] must hold words word_offsets[i]..."""
    a = np.ascontiguousarray(addrs, dtype=np.uint64)
    w = np.ascontiguousarray(word_offsets, dtype=np.uint64)
    assert a.shape == w.shape
    out = ctypes.c_uint64()
    pu = ctypes.POINTER(ctypes.c_uint64)
    check(lib().pf_verify_random_chunks(a.ctypes.data_as(pu), w.ctypes.data_as(pu), len(a),
                                        chunk_bytes, seed % 2**64, ctypes.byref(out)),
          "pf_verify_random_chunks")
    return out.value


def compare(a: int, b: int, nbytes: int) -> int:
    """Count of differing bytes between two device-visible buffers."""
    out = ctypes.c_uint64()
    check(lib().pf_compare(a, b, nbytes, ctypes.byref(out)), "pf_compare")
    return out.value


def memcpy_async(dst: int, src: int, nbytes: int, stream: Stream) -> None:
    """hipMemcpyAsync (direction inferred) on stream."""
    check(lib().pf_memcpy_async(dst, src, nbytes, stream.handle), "pf_memcpy_async")


def stream_wait_word(stream: Stream, word: int, value: int, timeout_us: int = 10_000_000,
                     timed_out: int = 0) -> None:
    """Work queued on ``stream`` afterwards waits until the 8-byte word at
    ``word`` is >= value, or ``timeout_us`` passes (the 4-byte word at
    ``timed_out``, if given, is then set to 1)."""
    check(lib().pf_stream_wait_word(stream.handle, word, value, timeout_us, timed_out),
          "pf_stream_wait_word")


def host_wait_word(word: int, value: int, timeout_us: int = 10_000_000) -> bool:
    """Wait on the host until the pinned 8-byte word at ``word`` is >= value;
    False on timeout."""
    reached = ctypes.c_int()
    check(lib().pf_host_wait_word(word, value, timeout_us, ctypes.byref(reached)),
          "pf_host_wait_word")
    return bool(reached.value)


def spin(stream: Stream, microseconds: int) -> None:
    check(lib().pf_spin(stream.handle, microseconds), "pf_spin")


def huge_page_size() -> int:
    return int(lib().pf_huge_page_size())
