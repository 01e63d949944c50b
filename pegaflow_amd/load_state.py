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
    def new(cls, num_layers: int | None = None) -> "LoadState":
        h = ctypes.c_void_p()
        if num_layers is None:
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
    """python/src/lib.rs:539-574.  State: 0 pending, 1 success, <0 error."""

    def __init__(self, num_layers: int | None = None):
        self._inner = LoadState.new(num_layers)

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

    @property
    def inner(self) -> LoadState:
        return self._inner
