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
    def new(cls, num_layers: int | None = None, event_handles=None,
            layer_words: "_lib.LayerWords | None" = None) -> "LoadState":
        h = ctypes.c_void_p()
        if layer_words is not None:
            if event_handles is not None or num_layers is None:
                raise ValueError("layer words need num_layers and exclude layer events")
            check(lib().pf_load_state_create_layered_words(num_layers, ctypes.byref(layer_words),
                                                           ctypes.byref(h)),
                  "failed to create LoadState")
        elif event_handles is not None and all(hasattr(e, "handle") for e in event_handles):
            # In-process events (runtime.Event): their addresses, for an
            # engine in this process.
            if num_layers is None or len(event_handles) != num_layers:
                raise ValueError("one event per layer is required")
            arr = (ctypes.c_void_p * num_layers)(*[e.handle for e in event_handles])
            check(lib().pf_load_state_create_layered_local_events(num_layers, arr,
                                                                  ctypes.byref(h)),
                  "failed to create LoadState")
        elif event_handles is not None:
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

    def events_local(self) -> bool:
        """True when the event block holds in-process event addresses."""
        return bool(lib().pf_load_state_events_local(self._h))

    def layer_words(self):
        """(pf_layer_words, layer count) of the words block, or (None, 0)."""
        w = _lib.LayerWords()
        n = ctypes.c_uint32(0)
        check(lib().pf_load_state_layer_words(self._h, ctypes.byref(w), ctypes.byref(n)),
              "pf_load_state_layer_words")
        return (w, n.value) if n.value else (None, 0)

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


class LayerWords:
    """Device words a consumer gates its streams on: one 8-byte word per
    layer, which the loader sets to the load's value once that layer's bytes
    are in place.  This is device-side per-layer completion for platforms
    that cannot share interprocess events (the reference has none:
    worker.py:288-289).

    ``local=False`` shares the words with a loader in another process through
    a device-memory IPC handle; ``local=True`` hands over their address, for
    an engine in this process.  ``next_load()`` gives the record for the next
    load (each load writes a larger value); ``wait_on_device(stream, l)``
    queues a bounded wait for layer l of the current load on ``stream``."""

    def __init__(self, num_layers: int, local: bool = False):
        from .runtime import DeviceBuffer

        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        self.num_layers = num_layers
        self.local = local
        self.buf = DeviceBuffer(8 * num_layers)
        self.buf.memset(0)
        self.value = 0
        self._handle = None
        if not local:
            h = (ctypes.c_uint8 * 64)()
            base, size = ctypes.c_uint64(), ctypes.c_uint64()
            check(lib().pf_ipc_export(self.buf.ptr, h, ctypes.byref(base), ctypes.byref(size)),
                  "pf_ipc_export")
            self._handle = (bytes(h), size.value, self.buf.ptr - base.value)

    def next_load(self) -> "_lib.LayerWords":
        self.value += 1
        w = _lib.LayerWords()
        w.value = self.value
        if self.local:
            w.kind = _lib.LAYER_WORDS_LOCAL
            w.address = self.buf.ptr
        else:
            handle, size, offset = self._handle
            w.kind = _lib.LAYER_WORDS_IPC
            w.alloc_size = size
            w.offset = offset
            ctypes.memmove(w.handle, handle, 64)
        return w

    def word(self, layer: int) -> int:
        if not 0 <= layer < self.num_layers:
            raise IndexError(layer)
        return self.buf.ptr + 8 * layer

    def wait_on_device(self, stream, layer: int, timeout_us: int = 10_000_000,
                       timed_out: int = 0) -> None:
        from .runtime import stream_wait_word

        stream_wait_word(stream, self.word(layer), self.value, timeout_us, timed_out)

    def close(self) -> None:
        if self.buf is not None:
            self.buf.close()
        self.buf = None


class PyLoadState:
    """python/src/lib.rs:539-574.  State: 0 pending, 1 success, <0 error.

    ``num_layers`` adds the per-layer counter.  Two ways let a consumer
    stream wait for layer l on the device, without the CPU
    (``wait_for_layer_on_device``):
      * ``layer_events``: one 64-byte interprocess event handle per layer
        (e.g. ``torch.cuda.Event(interprocess=True).ipc_handle()``), recorded
        by the loader after each layer; or, for an engine in this process,
        one ``runtime.Event`` per layer, recorded as they are;
      * ``layer_words``: a ``LayerWords`` whose words the loader's copy kernel
        sets per layer (for runtimes that cannot share events)."""

    def __init__(self, num_layers: int | None = None, layer_events=None,
                 layer_words: LayerWords | None = None):
        self._words = layer_words
        record = None
        if layer_words is not None:
            if num_layers is not None and num_layers != layer_words.num_layers:
                raise ValueError("num_layers differs from the layer words")
            num_layers = layer_words.num_layers
            record = layer_words.next_load()
        self._inner = LoadState.new(num_layers, layer_events, record)

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
        device.  ``stream_wait(layer_index)`` enqueues the wait.
          * With layer events, it waits on the consumer's event for that
            layer (for torch: ``lambda l: torch.cuda.current_stream()
            .wait_event(events[l])``), and it is called only after the loader
            has recorded the events, since a wait before the record would not
            wait at all.  Returns False on a failed load or timeout; True
            without a device wait when the load completed without recording
            (nothing to load).
          * With layer words, it is called at once (for this library's
            streams: ``lambda l: words.wait_on_device(stream, l)``): the loader
            writes every word, also for a failed or empty load.  Returns False
            without a wait when the load has already failed."""
        if self._words is not None:
            # The loader sets every word, also when the load fails or has
            # nothing to copy, so the wait can be queued right away.
            if self._inner.get() < 0:
                return False
            stream_wait(layer_index)
            return True
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
