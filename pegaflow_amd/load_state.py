"""LoadState: the shared-memory completion word of an asynchronous load.

``PyLoadState`` mirrors the reference's Python class (python/src/lib.rs:539-574:
``shm_name``, ``get_state``, ``is_ready``); ``LoadState`` is the attach side
used by the engine (sync_state.rs:145-177).  ``PyLoadState(num_layers=L)``
adds the per-layer completion counter (``layers_done``, ``wait_for_layer``).
"""

from __future__ import annotations

import ctypes
import time

from . import _lib
from ._lib import check

LOAD_STATE_PENDING = 0
LOAD_STATE_SUCCESS = 1
LOAD_STATE_ERROR = -1


def lib():
    return _lib.load()


class LoadState:
    """Handle on a LoadState mapping (creator or attacher)."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def new(cls, num_layers: int | None = None, event_handles=None) -> "LoadState":
        h = ctypes.c_void_p()
        if event_handles is not None:
            handles = b"".join(bytes(e) for e in event_handles)
            if num_layers is None or len(event_handles) != num_layers or \
                    len(handles) != 64 * num_layers:
                raise ValueError("one 64-byte event handle per layer is required")
            buf = (ctypes.c_uint8 * len(handles)).from_buffer_copy(handles)
            check(lib().pf_load_state_create_layered_events(num_layers, buf, ctypes.byref(h)),
                  "failed to create LoadState")
        elif num_layers is None:
            check(lib().pf_load_state_create(ctypes.byref(h)), "failed to create LoadState")
        else:
            check(lib().pf_load_state_create_layered(num_layers, ctypes.byref(h)),
                  "failed to create LoadState")
        return cls(h.value)

    @classmethod
    def attach(cls, shm_name: str) -> "LoadState":
        h = ctypes.c_void_p()
        check(lib().pf_load_state_attach(shm_name.encode(), ctypes.byref(h)), "LoadState")
        return cls(h.value)

    @property
    def handle(self):
        return self._h

    def shm_name(self) -> str:
        return lib().pf_load_state_name(self._h).decode()

    def get(self) -> int:
        return int(lib().pf_load_state_get(self._h))

    def set_completed(self) -> None:
        lib().pf_load_state_set_completed(self._h)

    def set_error(self) -> None:
        lib().pf_load_state_set_error(self._h)

    def num_layers(self) -> int:
        return int(lib().pf_load_state_num_layers(self._h))

    def layers_done(self) -> int:
        return int(lib().pf_load_state_layers_done(self._h))

    def set_layers_done(self, n: int) -> None:
        lib().pf_load_state_set_layers_done(self._h, n)

    def event_handles(self) -> list[bytes]:
        n = ctypes.c_uint32(0)
        p = lib().pf_load_state_event_handles(self._h, ctypes.byref(n))
        if not p:
            return []
        raw = ctypes.string_at(p, 64 * n.value)
        return [raw[64 * i:64 * (i + 1)] for i in range(n.value)]

    def events_recorded(self) -> int:
        return int(lib().pf_load_state_events_recorded(self._h))

    def set_events_recorded(self, n: int) -> None:
        lib().pf_load_state_set_events_recorded(self._h, n)

    def close(self) -> None:
        if self._h:
            lib().pf_load_state_close(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PyLoadState:
    """python/src/lib.rs:539-574.  State: 0 pending, 1 success, <0 error.

    ``num_layers`` adds the per-layer counter; ``layer_events`` (one 64-byte
    interprocess event handle per layer, e.g. ``torch.cuda.Event(
    interprocess=True).ipc_handle()``) lets the loader mark each layer on the
    device, so a consumer stream can wait for layer l without the CPU
    (``wait_for_layer_on_device``)."""

    def __init__(self, num_layers: int | None = None, layer_events=None):
        self._inner = LoadState.new(num_layers, layer_events)

    def shm_name(self) -> str:
        return self._inner.shm_name()

    def get_state(self) -> int:
        return self._inner.get()

    def is_ready(self) -> bool:
        return self._inner.get() != 0

    # Per-layer completion (absent from the reference, whose
    # wait_for_layer_load is a no-op: worker.py:288-289).
    def layers_done(self) -> int:
        return self._inner.layers_done()

    def wait_for_layer(self, layer_index: int, timeout_s: float = 60.0) -> bool:
        """Block until layer ``layer_index`` (0-based) is in place or the load
        failed; returns False on error or timeout."""
        deadline = time.monotonic() + timeout_s
        spins = 0
        while True:
            st = self._inner.get()
            if st < 0:
                return False
            if self._inner.layers_done() > layer_index or st == LOAD_STATE_SUCCESS:
                return True
            if time.monotonic() > deadline:
                return False
            spins += 1
            if spins > 1000:
                time.sleep(20e-6)

    def events_recorded(self) -> bool:
        """True once the loader has put every layer's event on its stream."""
        n = len(self._inner.event_handles())
        return n > 0 and self._inner.events_recorded() >= n

    def wait_for_layer_on_device(self, layer_index: int, stream_wait, timeout_s: float = 60.0
                                 ) -> bool:
        """Makes a consumer stream wait for layer ``layer_index`` on the
        device.  ``stream_wait(layer_index)`` enqueues the wait on the
        consumer's event for that layer (for torch: ``lambda l:
        torch.cuda.current_stream().wait_event(events[l])``).  It is called
        only after the loader has recorded the events, since a wait before
        the record would not wait at all.  Returns False on a failed load or
        timeout; True without a device wait when the load completed without
        recording (nothing to load)."""
        deadline = time.monotonic() + timeout_s
        spins = 0
        while not self.events_recorded():
            st = self._inner.get()
            if st < 0:
                return False
            if st == LOAD_STATE_SUCCESS:
                if self.events_recorded():
                    break
                return True
            if time.monotonic() > deadline:
                return False
            spins += 1
            if spins > 1000:
                time.sleep(20e-6)
        stream_wait(layer_index)
        return True

    @property
    def inner(self) -> LoadState:
        return self._inner
