"""pegaflow_amd — MI355X-native KV-block transfer path of PegaFlow.

Layers (reference roles in parentheses):
  * ``transfer``   — layouts, transfer primitives and the batched
                     gather/scatter context (pegaflow-core/src/transfer.rs,
                     the copy loops of gpu_worker.rs);
  * ``runtime``    — streams, events, device and pinned buffers
                     (cudarc contexts/streams, pinned_mem.rs);
  * ``load_state`` — the shared-memory completion word (sync_state.rs,
                     PyLoadState);
  * ``engine``     — PegaEngine: instances, registrations, the pinned block
                     store and the per-device save/load workers
                     (pegaflow-core/src/lib.rs, gpu_worker.rs, storage.rs).

All data movement runs in libpegaflow_hip.so (HIP, gfx950).  Importing this
package does not touch the GPU; the library is loaded on first use and its
absence is an error, never a fallback.
"""

from ._lib import (  # noqa: F401
    MODE_DMA_BATCHED,
    MODE_DMA_REFERENCE,
    MODE_KERNEL,
    MODE_NAMES,
    MODE_STAGED,
    PegaFlowError,
    PegaFlowLibraryMissing,
)

__version__ = "0.1.0"


def library_path() -> str:
    from ._lib import LIB_PATH

    return LIB_PATH
