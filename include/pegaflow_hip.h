/*
 * pegaflow_hip.h — C ABI of the MI355X-native KV-block transfer path.
 *
 * This is the seam between an engine/worker layer (the role of
 * pegaflow-core/src/lib.rs and gpu_worker.rs in the reference) and the
 * transfer, pinned-memory and completion primitives (the role of
 * pegaflow-core/src/transfer.rs, pinned_mem.rs and sync_state.rs).  Every
 * declaration below names the reference interface it replaces.
 *
 * Conventions
 *  - Every entry point returns an int status: PF_OK (0) or a PF_ERR_* code.
 *    On failure a human-readable message is kept per thread and returned by
 *    pf_last_error(); messages follow the reference's wording where the
 *    reference has one (e.g. "Block 3 segment 1 exceeds registered memory").
 *  - Device and host-mapped addresses are passed as uint64_t; host pointers as
 *    void*.  No framework types cross this boundary.
 *  - Device pointers passed in (layer tensors) are borrowed; the library owns
 *    only the streams, events, staging buffers and pinned allocations it
 *    creates.
 *  - Entry points are reentrant.  A pf_xfer context serialises its own work on
 *    its own streams; use one context per worker thread (the reference runs one
 *    load thread and one save thread per device, gpu_worker.rs:61-93).
 */
#ifndef PEGAFLOW_HIP_H
#define PEGAFLOW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status codes.  The engine-level codes mirror EngineError (lib.rs:58-85).   */
/* ------------------------------------------------------------------------ */
enum {
  PF_OK = 0,
  PF_ERR_INVALID_ARGUMENT = 1,  /* EngineError::InvalidArgument               */
  PF_ERR_HIP = 2,               /* a HIP runtime call failed                   */
  PF_ERR_STORAGE = 3,           /* EngineError::Storage (transfer/pool errors) */
  PF_ERR_INSTANCE_MISSING = 4,  /* EngineError::InstanceMissing                */
  PF_ERR_WORKER_MISSING = 5,    /* EngineError::WorkerMissing                  */
  PF_ERR_TOPOLOGY_MISMATCH = 6, /* EngineError::TopologyMismatch               */
  PF_ERR_INIT = 7,              /* EngineError::CudaInit                       */
  PF_ERR_LOAD_STATE = 8,        /* LoadStateError (sync_state.rs:46-56)        */
  PF_ERR_ZERO_SIZE = 9,         /* PinnedMemError::ZeroSize (pinned_mem.rs:72) */
  PF_ERR_UNSUPPORTED = 10,
  PF_ERR_MALFORMED = 11         /* a request that does not decode; the gRPC    */
                                /* service answers INTERNAL, as gRPC servers  */
                                /* do for a message that does not parse       */
};

/* Message of the last failed call on the calling thread ("" if none). */
const char* pf_last_error(void);
/* Library version string. */
const char* pf_version(void);

/* ------------------------------------------------------------------------ */
/* Layer layout.                                                              */
/* Replaces KVCacheRegistration (pegaflow-core/src/lib.rs:100-112).           */
/* ------------------------------------------------------------------------ */
typedef struct pf_kv_layout {
  uint64_t data_ptr;         /* device base address of the layer tensor     */
  uint64_t size_bytes;       /* registered bytes starting at data_ptr       */
  uint64_t num_blocks;       /* paged blocks in the layer                   */
  uint64_t bytes_per_block;  /* bytes of one segment of one block           */
  uint64_t block_size_bytes; /* bytes_per_block * segments                  */
  uint64_t kv_stride_bytes;  /* distance between K and V segments (0 if 1)  */
  uint64_t segments;         /* 2 for KV-first, 1 for blocks-first          */
} pf_kv_layout;

/* Fill *out from the register_context_layer arguments, with the reference's
 * validation (lib.rs:389-449): zero sizes, missing stride, checked overflow of
 * the last segment's end, and end > size_bytes are PF_ERR_INVALID_ARGUMENT. */
int pf_layout_init(uint64_t data_ptr, uint64_t size_bytes, uint64_t num_blocks,
                   uint64_t bytes_per_block, uint64_t kv_stride_bytes,
                   uint64_t segments, pf_kv_layout* out);

/* Replaces segment_offset (transfer.rs:18-47): block_idx*bytes_per_block +
 * segment_idx*kv_stride_bytes, checked; error when segment_idx >= segments,
 * on overflow, or when offset + bytes_per_block > size_bytes. */
int pf_segment_offset(const pf_kv_layout* layout, uint64_t block_idx,
                      uint64_t segment_idx, uint64_t* out_offset);

/* Replaces is_contiguous_layout (transfer.rs:50-52): 1 when segments <= 1 or
 * kv_stride_bytes == bytes_per_block, else 0. */
int pf_is_contiguous_layout(const pf_kv_layout* layout);

/* How a layer's blocks are moved, as dispatched in gpu_worker.rs:218-282 and
 * 326-372: SPLIT = per-segment K list then V list (segments == 2 and
 * kv_stride_bytes > bytes_per_block); CONTIGUOUS = one block_size_bytes chunk
 * per block; STRIDED = any other multi-segment layout (save copies each
 * segment to dst + s*bytes_per_block, load copies block_size_bytes from
 * segment_offset(block, 0), exactly as the reference does). */
enum { PF_LAYOUT_SPLIT = 0, PF_LAYOUT_CONTIGUOUS = 1, PF_LAYOUT_STRIDED = 2 };
/* -1 for a null layout. */
int pf_layout_kind(const pf_kv_layout* layout);

/* ------------------------------------------------------------------------ */
/* Device runtime: devices, streams, events, device memory.                   */
/* Replaces CudaContext::new / new_stream / record_event / synchronize        */
/* (gpu_worker.rs:146-150, 286-291; lib.rs:247).                              */
/* ------------------------------------------------------------------------ */
typedef void* pf_stream;
typedef void* pf_event;

int pf_get_device_count(int* count);
/* hipSetDevice + once-per-device library init (wall-clock rate query).      */
int pf_init(int device);
int pf_set_device(int device);
int pf_get_device(int* device);
int pf_device_synchronize(void);

/* Non-blocking stream at the default priority. */
int pf_stream_create(pf_stream* out);
int pf_stream_destroy(pf_stream stream);
int pf_stream_synchronize(pf_stream stream);
int pf_stream_wait_event(pf_stream stream, pf_event event);

/* Timing-capable event. */
int pf_event_create(pf_event* out);
int pf_event_destroy(pf_event event);
int pf_event_record(pf_event event, pf_stream stream);
int pf_event_synchronize(pf_event event);
/* *done = 1 when the event has completed, 0 when still pending. */
int pf_event_query(pf_event event, int* done);
int pf_event_elapsed_ms(pf_event start, pf_event end, float* ms);

int pf_device_malloc(uint64_t size, uint64_t* out_dev_ptr);
int pf_device_free(uint64_t dev_ptr);
int pf_memcpy_h2d(uint64_t dst_dev, const void* src, uint64_t size);
int pf_memcpy_d2h(void* dst, uint64_t src_dev, uint64_t size);
int pf_memcpy_d2d(uint64_t dst_dev, uint64_t src_dev, uint64_t size);
int pf_memset_d8(uint64_t dst_dev, uint8_t value, uint64_t size);
/* hipMemcpyAsync with the direction inferred from the addresses. */
int pf_memcpy_async(uint64_t dst, uint64_t src, uint64_t size, pf_stream stream);
/* Free and total device memory in bytes. */
int pf_mem_get_info(uint64_t* free_bytes, uint64_t* total_bytes);
/* PCI address of the device, "dddd:bb:dd.f" (lower case, NUL-terminated in
 * len bytes), to find its NUMA node under /sys/bus/pci/devices (no
 * counterpart in the reference; the pinned pool's NUMA placement and the
 * benchmark's host-thread count use it). */
int pf_device_pci_bus_id(int device, char* buf, int len);

/* ------------------------------------------------------------------------ */
/* Pinned host memory.                                                        */
/* Replaces PinnedMemory::{allocate, allocate_hugepages} and Drop              */
/* (pinned_mem.rs:128-266).  Backed by hipHostMalloc and always mapped for     */
/* device access, so the transfer kernels can read and write it directly.     */
/* ------------------------------------------------------------------------ */
enum {
  PF_PINNED_DEFAULT = 0,     /* hipHostMallocMapped | Portable             */
  PF_PINNED_COHERENT = 1,    /* + hipHostMallocCoherent (fine-grained)     */
  PF_PINNED_NONCOHERENT = 2, /* + hipHostMallocNonCoherent (coarse-grained)*/
  PF_PINNED_NUMA_USER = 4,   /* + hipHostMallocNumaUser (caller's policy)  */
  PF_PINNED_WRITE_COMBINED = 8 /* + hipHostMallocWriteCombined: the         */
                               /* reference's pool flag (pinned_mem.rs:159)  */
};
/* size == 0 is PF_ERR_ZERO_SIZE (pinned_mem.rs:150-152).  *dev_ptr receives
 * the device-visible address of the allocation (hipHostGetDevicePointer). */
int pf_pinned_allocate(uint64_t size, uint32_t flags, void** host_ptr,
                       uint64_t* dev_ptr);
int pf_pinned_free(void* host_ptr);
/* Device-visible address of a host pointer inside a pinned allocation. */
int pf_host_device_pointer(const void* host_ptr, uint64_t* dev_ptr);
/* Huge page size in bytes parsed from /proc/meminfo ("Hugepagesize: N kB"),
 * 0 when absent (pinned_mem.rs:33-52). */
uint64_t pf_huge_page_size(void);

/* ------------------------------------------------------------------------ */
/* Device-memory IPC.  Replaces the CUDA-IPC sharing of layer tensors between */
/* the inference process and the engine server (torch _share_cuda_ /          */
/* _new_shared_cuda: ipc_wrapper.py:101-156, registry.rs:144-175).           */
/* Allocations of 2 GiB or more are refused on both ends.                     */
/* ------------------------------------------------------------------------ */
#define PF_IPC_HANDLE_BYTES 64
#define PF_IPC_MAX_ALLOC_BYTES (1ull << 31)
/* Handle of the device allocation containing dev_ptr, with its base and size. */
int pf_ipc_export(uint64_t dev_ptr, uint8_t* handle, uint64_t* alloc_base,
                  uint64_t* alloc_size);
/* Maps an exported allocation of alloc_size bytes into this process; *base is
 * the mapped base address.  The range becomes valid for the kernels. */
int pf_ipc_open(const uint8_t* handle, uint64_t alloc_size, uint64_t* base);
int pf_ipc_close(uint64_t base);
/* No counterpart in the reference (its per-layer wait is a no-op,
 * worker.py:288-289): events another process can record and this one wait
 * on, for cross-process per-layer completion on the device.  The event is
 * created with timing disabled and the interprocess flag; its 64-byte handle
 * is opened in the other process with pf_ipc_event_open (not in the same
 * process).  Destroy both with pf_event_destroy.  A runtime that refuses to
 * export interprocess events (probed once per process) makes
 * pf_event_create_ipc fail with PF_ERR_UNSUPPORTED; cross-process waits then
 * use layer words (pf_load_state_create_layered_words). */
int pf_event_create_ipc(pf_event* out);
int pf_ipc_event_export(pf_event event, uint8_t* handle);
int pf_ipc_event_open(const uint8_t* handle, pf_event* out);

/* ------------------------------------------------------------------------ */
/* Reference-equivalent DMA primitives (transfer.rs:56-239).                  */
/* ------------------------------------------------------------------------ */
/* Synchronous device -> host copy of size bytes from gpu_base+offset.
 * cpu_buffer_len < size is "CPU buffer too small: ..." (the reference takes a
 * slice and leaves the check to its callers, which pass size == len).
 * Replaces copy_gpu_to_cpu (transfer.rs:56-76). */
int pf_copy_gpu_to_cpu(uint64_t gpu_base, uint64_t offset, void* cpu_buffer,
                       uint64_t cpu_buffer_len, uint64_t size);
/* Asynchronous host -> device copy on stream; cpu_buffer_len < size is
 * "CPU buffer too small: ..." (transfer.rs:89-95).
 * Replaces copy_cpu_to_gpu_async (transfer.rs:80-113). */
int pf_copy_cpu_to_gpu_async(uint64_t gpu_base, uint64_t offset,
                             const void* cpu_buffer, uint64_t cpu_buffer_len,
                             uint64_t size, pf_stream stream);
/* Greedy run merging + one async H2D copy per run.  Entry j joins the run
 * started at i iff gpu_offsets[j] == gpu_offsets[i] + (j-i)*segment_size and
 * cpu_ptrs[j] == cpu_ptrs[i] + (j-i)*segment_size.  *out_batches receives the
 * number of copies issued (may be NULL).
 * Replaces batch_copy_segments_to_gpu (transfer.rs:116-198). */
int pf_batch_copy_segments_to_gpu(const uint64_t* gpu_offsets,
                                  const uint64_t* cpu_ptrs, uint64_t count,
                                  uint64_t segment_size,
                                  const pf_kv_layout* layout, pf_stream stream,
                                  uint64_t* out_batches);
/* Number of copies pf_batch_copy_segments_to_gpu would issue (no copies). */
uint64_t pf_count_merged_runs(const uint64_t* gpu_offsets,
                              const uint64_t* cpu_ptrs, uint64_t count,
                              uint64_t segment_size);
/* Synchronous copy of one whole block to dst: one chunk of block_size_bytes
 * when contiguous, else each segment s to dst + s*bytes_per_block.  Errors of
 * segment_offset are returned as they are; a contiguous whole block that
 * ends past size_bytes is "Block b exceeds registered memory (offset o,
 * size block_size_bytes, limit size_bytes)" (the reference bounds only the
 * first segment there and would read past the tensor).
 * Replaces copy_block_gpu_to_cpu / copy_gpu_to_cpu_strided
 * (transfer.rs:201-239). */
int pf_copy_block_gpu_to_cpu(const pf_kv_layout* layout, uint64_t block_idx,
                             void* dst);

/* ------------------------------------------------------------------------ */
/* Batched transfer contexts and kernels (the hot path).                      */
/* Replace process_save_task / process_load_task (gpu_worker.rs:205-390).     */
/* ------------------------------------------------------------------------ */
typedef struct pf_xfer pf_xfer;

/* One block of one layer.  Replaces SaveBlock (gpu_worker.rs:38-44) and
 * LoadBlock + LayerBlock::{k_ptr, v_ptr} (gpu_worker.rs:25-28,
 * storage.rs:294-300).  k_host / v_host are host (or host-mapped, or device)
 * addresses; v_host == 0 means k_host + bytes_per_block, as the reference's
 * unwrap_or_else fallbacks do (gpu_worker.rs:233-236, 354-356). */
typedef struct pf_block_xfer {
  int64_t block_idx;
  uint64_t k_host;
  uint64_t v_host;
} pf_block_xfer;

/* Blocks of one layer.  Replaces LayerLoadData (gpu_worker.rs:19-23) and the
 * (registration, blocks) pair of SaveTask (gpu_worker.rs:32-36). */
typedef struct pf_layer_xfer {
  pf_kv_layout layout;
  const pf_block_xfer* blocks;
  uint64_t num_blocks;
} pf_layer_xfer;

/* Transfer strategies.  All produce identical bytes.
 *  DMA_REFERENCE: the reference's calls — save = one synchronous D2H copy per
 *                 segment (gpu_worker.rs:344-371); load = merged runs, one
 *                 async H2D copy per run (transfer.rs:116-198).
 *  DMA_BATCHED:   merged runs, async, in both directions; one sync at the end.
 *  KERNEL:        one gather/scatter kernel per layer moves 16 B per lane
 *                 directly between the paged layer tensor and the (host-mapped
 *                 pinned, or device) addresses.
 *  STAGED:        the kernel runs HBM<->HBM between the paged tensor and
 *                 packed staging slots, and the host link is crossed only by
 *                 DMA copies of host-contiguous runs; the call is cut into
 *                 slices that may span layers.  With the host side in pinned
 *                 memory the copies run on a fast copy engine per
 *                 direction that the runtime's own copies do not use
 *                 (pf_copy_engines), driven from the calling
 *                 thread (a load returns once its copies are done and its
 *                 last kernels are issued); otherwise through HIP, slices
 *                 alternating between the context's two streams.  Unlike
 *                 KERNEL, it leaves kernels running beside it at their
 *                 speed: shader reads and writes of host memory hold up
 *                 every other kernel's memory traffic (a bf16 GEMM in
 *                 another process ran 29x slower beside a KERNEL save of the
 *                 Llama prefix, 1.03x beside a STAGED one).
 *  AUTO:          STAGED when the context has staging and the call's
 *                 host-contiguous runs average at least 1 MiB (long enough
 *                 for DMA copies to run at the link's speed), else KERNEL.
 *                 No counterpart in the reference (its calls are DMA). */
enum {
  PF_MODE_DMA_REFERENCE = 0,
  PF_MODE_DMA_BATCHED = 1,
  PF_MODE_KERNEL = 2,
  PF_MODE_STAGED = 3,
  PF_MODE_AUTO = 4
};

/* Create a transfer context on device: its own two non-blocking streams, a
 * device descriptor buffer, and (if staging_bytes > 0) two staging slots of
 * staging_bytes/2 each for PF_MODE_STAGED, one per stream. */
int pf_xfer_create(int device, uint64_t staging_bytes, pf_xfer** out);
int pf_xfer_destroy(pf_xfer* xfer);
/* The context's first stream: the kernel mode's launches run on it, and every
 * load's work (on both streams in the staged mode) is ordered before what is
 * queued on it afterwards. */
pf_stream pf_xfer_stream(pf_xfer* xfer);
/* Wait for all work issued on the context. */
int pf_xfer_synchronize(pf_xfer* xfer);
/* Select the kernel's launch shape: threads per workgroup (64..1024, multiple
 * of 64) and 16-byte loads in flight per lane (1, 2, 4, 8 or 16), optionally
 * OR-ed with PF_KERNEL_NT_LOADS and/or PF_KERNEL_NT_STORES for non-temporal
 * (streaming) loads and stores.  0 keeps the current value.  Sets the shape
 * of every route; defaults below. */
#define PF_KERNEL_NT_LOADS 0x100u
#define PF_KERNEL_NT_STORES 0x200u
#define PF_KERNEL_NONTEMPORAL (PF_KERNEL_NT_LOADS | PF_KERNEL_NT_STORES)
/* Give each of the 8 XCDs one contiguous range of tiles instead of the
 * hardware's round-robin deal (only with an uncapped grid). */
#define PF_KERNEL_XCD_MAJOR 0x400u
/* Scatters only (PF_ROUTE_LOAD_DEVICE): choose the shape on evidence.  The
 * context times two candidate shapes, 512 threads with 2 loads per lane in
 * XCD-major order and 512 threads with 1 load per lane in round-robin order
 * (both non-temporal), twice each on its first scatters of at least 64 MiB,
 * and keeps the faster.  Which one wins depends on where the destination
 * tensors lie in HBM.  The other bits of the value are then ignored. */
#define PF_KERNEL_AUTO 0x800u
/* Launch shapes are kept per route: the direction, and whether the far side
 * of the copy is device memory (an HBM-bound gather or scatter) or pinned
 * host memory (zero-copy over the host link). */
enum {
  PF_ROUTE_SAVE_DEVICE = 0, /* paged tensor -> device memory (gather)       */
  PF_ROUTE_LOAD_DEVICE = 1, /* device memory -> paged tensor (scatter)      */
  PF_ROUTE_SAVE_HOST = 2,   /* paged tensor -> pinned host memory           */
  PF_ROUTE_LOAD_HOST = 3    /* pinned host memory -> paged tensor           */
};
/* Per-route defaults (the fastest shapes measured on MI355X): HBM gathers
 * move 8 KiB tiles in round-robin order; scatters choose on evidence
 * (PF_KERNEL_AUTO); zero-copy saves 16 KiB tiles with streaming loads and
 * ordinary stores into host memory (2% faster than streaming both). */
#define PF_SAVE_DEFAULT_THREADS 512u
#define PF_SAVE_DEFAULT_UNROLL (1u | PF_KERNEL_NONTEMPORAL)
#define PF_LOAD_DEFAULT_THREADS 512u
#define PF_LOAD_DEFAULT_UNROLL (2u | PF_KERNEL_NONTEMPORAL | PF_KERNEL_XCD_MAJOR | PF_KERNEL_AUTO)
#define PF_SAVE_HOST_DEFAULT_THREADS 512u
#define PF_SAVE_HOST_DEFAULT_UNROLL (2u | PF_KERNEL_NT_LOADS)
#define PF_LOAD_HOST_DEFAULT_THREADS 512u
#define PF_LOAD_HOST_DEFAULT_UNROLL (2u | PF_KERNEL_NONTEMPORAL | PF_KERNEL_XCD_MAJOR)
/* Shape for one route only (PF_ROUTE_*; 0 and 1 are also "saves" and
 * "loads" of device memory).  pf_xfer_set_kernel_shape sets every route.
 * Setting the scatter route's shape restarts its choice when the new value
 * carries PF_KERNEL_AUTO, and ends it otherwise. */
int pf_xfer_set_kernel_shape_dir(pf_xfer* xfer, uint32_t direction,
                                 uint32_t threads, uint32_t unroll);
/* The shape a route's next fixed-map launch uses: the route's setting, or for
 * a scatter route on PF_KERNEL_AUTO the chosen candidate once both have been
 * timed (*decided = 1), else the first candidate (*decided = 0). */
int pf_xfer_route_shape(pf_xfer* xfer, uint32_t route, uint32_t* threads,
                        uint32_t* unroll, int* decided);
/* Work distribution per route.  0: one workgroup per tile, dealt to the XCDs
 * by the hardware (best for HBM-bound copies).  N > 0: N persistent
 * workgroups take tiles from a queue in order (best over the host link,
 * whose bandwidth the XCDs do not share fairly: the queue keeps tiles, and
 * a marked load's layers, finishing in order, and few requests in flight
 * keep the link at its peak).  Marked launches always run queued (at
 * PF_LOAD_HOST_DEFAULT_GRID when their route says 0).  pf_xfer_set_max_grid
 * caps both kinds.  Every route may run queued: the staged mode's two
 * streams each have a queue of their own, and a queued launch leaves its
 * queue empty. */
#define PF_SAVE_HOST_DEFAULT_GRID 32u
#define PF_LOAD_HOST_DEFAULT_GRID 64u
int pf_xfer_set_route_grid(pf_xfer* xfer, uint32_t route, uint32_t workgroups);
int pf_xfer_set_kernel_shape(pf_xfer* xfer, uint32_t threads, uint32_t unroll);
/* Upper bound on workgroups per gather/scatter launch (0 = one workgroup per
 * tile, the default); with a bound, each workgroup loops over tiles. */
int pf_xfer_set_max_grid(pf_xfer* xfer, uint32_t max_workgroups);
/* The copy engines (HSA SDMA engine id bits, from hsa_amd_sdma_engine_id_t)
 * the staged mode's copies run on for `device`: device to host, then host to
 * device; one each, different where the device allows.  By default two of
 * the four fast engines (0-3 on MI355X) that the runtime's own copies do not
 * use (hipMemcpyAsync takes the lowest engine of each preferred set), so a
 * model's small copies beside a staged transfer do not queue behind its
 * slices; the environment variable PEGAFLOW_COPY_ENGINES="<d2h>,<h2d>" or
 * pf_set_copy_engines names others, one or two bits each, slices alternating
 * between two.  Both 0 when they are not known (the staged mode then copies
 * through HIP).  No counterpart in the reference (its copies are cuMemcpy
 * calls); bench_copy_engines measures each engine. */
int pf_copy_engines(int device, uint32_t* d2h_engine, uint32_t* h2d_engine);
/* Chooses the copy engines of the staged mode on `device`, per direction a
 * mask of one or two engine id bits (0 keeps that direction's choice), from
 * those the runtime reports available (else PF_ERR_INVALID_ARGUMENT); copies
 * issued afterwards use them.  PF_ERR_UNSUPPORTED when the device's engines
 * are not known.  No counterpart in the reference. */
int pf_set_copy_engines(int device, uint32_t d2h_engines, uint32_t h2d_engines);
/* Largest staged slice per direction, in bytes (0 keeps the current value);
 * slices are further capped by the staging slot.  A load's slices start at
 * a quarter of its largest slice (at most 16 MiB) and double, each of the
 * first layers ending its last slice meanwhile, so the first layers land
 * early.  Each copy-engine command costs about 10 us besides its bytes:
 * measured on the Llama-3.1-8B prefix (1.25 GiB), a staged save took 23.85,
 * 23.75 and 23.73 ms with 64, 128 and 256 MiB slices, and a staged restore
 * 23.79, 23.67 and 23.60 ms (56.9 GB/s).  A context staging both slots of
 * the defaults holds 512 MiB of HBM. */
#define PF_STAGED_SAVE_SLICE_DEFAULT (256ull << 20)
#define PF_STAGED_LOAD_SLICE_DEFAULT (256ull << 20)
int pf_xfer_set_staged_slices(pf_xfer* xfer, uint64_t save_bytes, uint64_t load_bytes);
/* How a staged load whose caller waits layer by layer (marks or per-layer
 * events) copies its first layer: PF_STAGED_HEAD_ENGINE (the default)
 * through the copy engines as one copy, then one scatter kernel that marks
 * the layer itself; PF_STAGED_HEAD_KERNEL by the zero-copy kernel.  Beside a
 * GEMM whose workgroups fill every CU, each kernel of the load waits for one
 * of the GEMM's kernels to end, so either route lands the layer after one
 * such wait.  Measured on the Llama-3.1-8B prefix beside a bf16 8192^3 GEMM
 * run back to back by another process (bench.py --first-layer-study, four
 * runs): the copy-engine route lands the first layer 1.57-1.65 ms after the
 * call, the load runs at 54.2-55.7 GB/s and the GEMM 1.01-1.04x slower; the
 * kernel route 1.50-1.58 ms, 53.3-53.6 GB/s and 1.04-1.06x (its 0.74 ms of
 * shader traffic over the host link also slows every other kernel's memory
 * traffic).  On an idle device both land it in 0.93-1.02 ms.  The
 * environment variable PEGAFLOW_STAGED_HEAD=kernel (or =engine) sets the
 * route of contexts created afterwards, the engine's included.  Other
 * routes: PF_ERR_INVALID_ARGUMENT.  No counterpart in the reference (its
 * loads are one cuMemcpyHtoDAsync per run). */
#define PF_STAGED_HEAD_KERNEL 0u
#define PF_STAGED_HEAD_ENGINE 1u
int pf_xfer_set_staged_head(pf_xfer* xfer, uint32_t route);
/* Compute units the context's kernels run on.  Bit b of `mask` (word b/32,
 * bit b%32) enables the device's CU b; the runtime deals the bits to the
 * XCDs round-robin, so bit b is on XCD b mod (number of XCDs) — on MI355X
 * bits 0-7 are one CU on each of the 8 XCDs, the next 8 a second CU of
 * each.  `words` = 0 restores unmasked streams.  A mask that leaves an XCD
 * without a CU is refused (PF_ERR_INVALID_ARGUMENT): every launch is split
 * across the XCDs, and that XCD's share would never run.  The call waits for
 * the context's work, then replaces its two streams: a stream handle taken
 * from pf_xfer_stream before the call is no longer valid after it.  Masked
 * streams are ordered with the null stream.  PEGAFLOW_CUS_PER_XCD=<k> masks
 * every context created afterwards (the engine's included) to k CUs per
 * XCD.  No counterpart in the reference (its copies run on DMA engines). */
int pf_xfer_set_cu_mask(pf_xfer* xfer, const uint32_t* mask, uint32_t words);
/* Fills `mask` (`words` words) with k CUs on each XCD of `device`: bits 0
 * to k*(number of XCDs)-1. */
int pf_cu_mask_per_xcd(int device, uint32_t cus_per_xcd, uint32_t* mask, uint32_t words);
/* Number of gather/scatter kernel launches and DMA copies issued by the last
 * save/load call on this context. */
int pf_xfer_last_stats(pf_xfer* xfer, uint64_t* kernel_launches,
                       uint64_t* dma_copies);
/* Kernel timing: when enabled, every gather/scatter launch is bracketed by
 * two events on the context's kernel stream.  pf_xfer_last_kernel_ms waits
 * for the last call's kernels and returns their summed duration and count. */
int pf_xfer_set_timing(pf_xfer* xfer, int enable);
int pf_xfer_last_kernel_ms(pf_xfer* xfer, float* ms, uint64_t* launches);

/* Device -> host: for every layer, copy each block's segments to its
 * k_host/v_host destinations as process_save_task does (gpu_worker.rs:321-390).
 * Every block_idx must be < num_blocks and pass segment_offset's bound.
 * Blocking: returns when the bytes are in place. */
int pf_save_layers(pf_xfer* xfer, const pf_layer_xfer* layers,
                   uint32_t num_layers, uint32_t mode);

/* Host -> device: for every layer, copy each block's segments from
 * k_host/v_host into the paged tensor as process_load_task does
 * (gpu_worker.rs:205-283).  Asynchronous: returns after issuing (a STAGED
 * load on the copy engines: once its copies are done).  If
 * layer_events is non-NULL, layer_events[l] is recorded once layer l's bytes
 * are in place (per-layer completion, which the reference lacks:
 * worker.py:288-289).  Completion of the whole call is pf_xfer_synchronize or
 * the last layer's event.  A save or load that fails returns with none of
 * its copies (or marks) still in flight. */
int pf_load_layers(pf_xfer* xfer, const pf_layer_xfer* layers,
                   uint32_t num_layers, uint32_t mode, pf_event* layer_events);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory: tight serving loops and harnesses that forbid hipMalloc.  Not for
 * HIP graph capture: the scratch below is shared by every call on a device,
 * so a replayed graph would copy the blocks of whichever call ran last; on a
 * stream that is capturing, the call fails with PF_ERR_UNSUPPORTED before
 * anything is issued.  pf_load_layers in PF_MODE_KERNEL without events, with
 * the same bytes, issued on the caller's stream (NULL: the current device's
 * null stream) instead of a transfer context's.  The chunk descriptors and
 * the tile queue live in a static device array of the library (one copy per
 * device, 256 B + PF_NOALLOC_MAX_CHUNKS x 16 B = 1 MiB + 256 B, held until
 * the process ends); nothing is allocated on the device or in pinned memory.
 * A call of more than PF_NOALLOC_MAX_CHUNKS chunks (segments, or whole
 * blocks for single-segment layouts, summed over layers) fails with
 * PF_ERR_INVALID_ARGUMENT before anything is issued.  Asynchronous: returns
 * after issuing; stream order serialises calls on one stream, and the array
 * keeps the last call's descriptors.  Calls on one device that overlap on
 * different streams race on the shared array: the caller orders them.
 * Layers whose copies must run in list order use async DMA copies on the
 * stream, as pf_load_layers does. */
#define PF_NOALLOC_MAX_CHUNKS 65536
int pf_load_layers_noalloc(pf_stream stream, const pf_layer_xfer* layers,
                           uint32_t num_layers);

/* Layer marks: per-layer completion written by the load itself.  No
 * counterpart in the reference (its per-layer wait is a no-op,
 * worker.py:288-289; its load syncs once after all layers,
 * gpu_worker.rs:286-291).  Unlike layer_events, marks do not split a load
 * from pinned host memory into one launch per layer: in PF_MODE_KERNEL one
 * launch covers every such layer (two for a large call, whose first eighth
 * of layers is launched before the rest is planned) and its last workgroup
 * on layer l writes the marks of layer l.  Layers loaded from device memory (an
 * HBM-bound copy) get one launch each, followed by their marks; DMA copies
 * are marked after each layer's copies.  In PF_MODE_STAGED (and AUTO when it
 * stages) each slice's scatter marks the layers it completes, counting a
 * layer's tiles over the slices that hold it, so a layer lands after one
 * kernel; layers in slices that cannot carry them (more than 8 layers,
 * unaligned chunks) are marked by a separate kernel after their last
 * slice. 
 *
 * A signal target is an array of one 8-byte word per layer of the call:
 * words + 8*l is set to `value` once layer l's bytes are in place.  The
 * array may be host-mapped pinned memory (host_memory = 1, the host polls
 * it; an array inside a pf_pinned_allocate allocation is treated so even
 * when the flag is 0), device memory of this process, or device memory of
 * another process mapped with pf_ipc_open (host_memory = 0; a stream waits
 * on it with pf_stream_wait_word).  Every word is written exactly once per call, empty
 * layers included; values must be nonzero, and a caller reusing an array
 * gives each call a larger value than the last, since waiters wait for
 * word >= value. */
#define PF_MAX_LAYER_SIGNALS 4
typedef struct pf_layer_signal {
  uint64_t words;       /* address of num_layers 8-byte words (8-aligned)  */
  uint64_t value;       /* nonzero                                        */
  uint32_t host_memory; /* 1: pinned host memory, 0: device memory        */
  uint32_t reserved;    /* 0                                              */
} pf_layer_signal;
/* pf_load_layers with marks instead of events (1..PF_MAX_LAYER_SIGNALS
 * targets).  Asynchronous like pf_load_layers. */
int pf_load_layers_marked(pf_xfer* xfer, const pf_layer_xfer* layers,
                          uint32_t num_layers, uint32_t mode,
                          const pf_layer_signal* signals, uint32_t num_signals);
/* Bounded device-side wait (no counterpart in the reference): work queued on
 * stream after this call starts once the 8-byte word at `word` (device,
 * IPC-mapped or pinned host memory) is >= value, or after timeout_us
 * microseconds (at most 60 s), whichever comes first; the waiting kernel
 * always ends.  A timeout sets the 4-byte word at timed_out (if nonzero,
 * device or pinned memory) to 1; the caller clears it beforehand. */
int pf_stream_wait_word(pf_stream stream, uint64_t word, uint64_t value,
                        uint32_t timeout_us, uint64_t timed_out);
/* Host-side wait on a word in pinned host memory: *reached = 1 once the word
 * is >= value, 0 if timeout_us passed first. */
int pf_host_wait_word(const uint64_t* word, uint64_t value, uint64_t timeout_us,
                      int* reached);

/* ------------------------------------------------------------------------ */
/* Synthetic data and verification kernels (benchmarks and parity tests).     */
/* ------------------------------------------------------------------------ */
/* Fill size_bytes (multiple of 8) at dst_dev with splitmix64 words:
 * word[i] = mix64(seed + (word_offset + i + 1) * 0x9E3779B97F4A7C15). */
int pf_fill_random(uint64_t dst_dev, uint64_t size_bytes, uint64_t seed,
                   uint64_t word_offset, pf_stream stream);
/* Count 8-byte words at addr that differ from the pf_fill_random formula
 * (words expected: seed, word_offset...).  Synchronous; addr may be
 * host-mapped. */
int pf_verify_random(uint64_t addr, uint64_t size_bytes, uint64_t seed,
                     uint64_t word_offset, uint64_t* mismatches);
/* Batched form of pf_verify_random: chunk i (chunk_bytes at addrs[i]) must
 * hold the words seed, word_offsets[i]... .  Host arrays; synchronous. */
int pf_verify_random_chunks(const uint64_t* addrs, const uint64_t* word_offsets,
                            uint64_t n, uint64_t chunk_bytes, uint64_t seed,
                            uint64_t* mismatches);
/* Count differing bytes between two device-visible buffers (synchronous). */
int pf_compare(uint64_t a, uint64_t b, uint64_t size_bytes,
               uint64_t* mismatches);
/* Busy-wait on the device wall clock for `microseconds` on stream: a
 * stand-in for a layer's attention compute in overlap measurements. */
int pf_spin(pf_stream stream, uint32_t microseconds);

/* ------------------------------------------------------------------------ */
/* LoadState: cross-process completion word in POSIX shared memory.           */
/* Replaces sync_state.rs:19-292.  The first 32 bytes are byte-identical to   */
/* the reference's mapping: a native-endian u64 offset (8) at byte 0, then    */
/* {u32 magic 0x50464C44, u32 version 1, i64 state} at that offset.           */
/* A layered state appends an extension record after byte 32:               */
/* {u32 magic 0x50464C58 ('PFLX'), u32 num_layers, i64 layers_done} so a      */
/* reader that knows only the reference's record still attaches to it.       */
/* ------------------------------------------------------------------------ */
typedef struct pf_load_state pf_load_state;
enum { PF_LOAD_PENDING = 0, PF_LOAD_SUCCESS = 1, PF_LOAD_ERROR = -1 };

/* LoadState::new (sync_state.rs:125-142): shm "pega_load_<32 hex>". */
int pf_load_state_create(pf_load_state** out);
/* Same, with a per-layer completion counter for num_layers layers. */
int pf_load_state_create_layered(uint32_t num_layers, pf_load_state** out);
/* LoadState::attach (sync_state.rs:145-155). */
int pf_load_state_attach(const char* shm_name, pf_load_state** out);
/* Unmaps; the creator also unlinks the shm name. */
int pf_load_state_close(pf_load_state* state);
const char* pf_load_state_name(const pf_load_state* state);
int64_t pf_load_state_get(const pf_load_state* state);
void pf_load_state_set_completed(pf_load_state* state);
void pf_load_state_set_error(pf_load_state* state);
/* Layered extension: number of layers (0 for a plain state), layers whose
 * bytes are in place, and the writer's increment (release ordering). */
uint32_t pf_load_state_num_layers(const pf_load_state* state);
int64_t pf_load_state_layers_done(const pf_load_state* state);
void pf_load_state_set_layers_done(pf_load_state* state, int64_t n);
/* Device-side per-layer completion across processes (no counterpart in the
 * reference).  A layered state created with one interprocess event handle
 * per layer (num_layers x PF_IPC_HANDLE_BYTES) carries, after the layered
 * extension at byte 48, {u32 magic 0x50464C45 ('PFLE'), u32 count,
 * i64 events_recorded} and the handles.  The loader opens the handles,
 * records layer l's event on its stream after layer l's copy, and then
 * publishes events_recorded = count; from then on the consumer may make a
 * stream wait on event l (waiting earlier would see no record).  Where the
 * runtime refuses to export interprocess events (as pf_event_create_ipc
 * reports) this fails with PF_ERR_UNSUPPORTED; with no device present the
 * handles are kept as opaque bytes. */
int pf_load_state_create_layered_events(uint32_t num_layers,
                                        const uint8_t* event_handles,
                                        pf_load_state** out);
/* The in-process variant of the event block (no counterpart in the
 * reference): num_layers events of the loader's own process (pf_event_create
 * or pf_event_create_ipc), whose addresses fill the handle slots (8 bytes,
 * then zeros) under magic 0x50464C4C ('PFLL').  The loader records them as
 * it records opened handles, one launch per layer, then publishes
 * events_recorded.  For an engine in the consumer's process, and for
 * runtimes that cannot export interprocess events. */
int pf_load_state_create_layered_local_events(uint32_t num_layers,
                                              const pf_event* events,
                                              pf_load_state** out);
/* Handles carried by a state (NULL / 0 when none). */
const uint8_t* pf_load_state_event_handles(const pf_load_state* state,
                                           uint32_t* count);
/* 1 when the state's event block holds in-process event addresses. */
int pf_load_state_events_local(const pf_load_state* state);
int64_t pf_load_state_events_recorded(const pf_load_state* state);
void pf_load_state_set_events_recorded(pf_load_state* state, int64_t n);
/* Device-side per-layer completion through layer words (no counterpart in
 * the reference), for platforms without interprocess events.  The consumer
 * owns num_layers 8-byte words of device memory and gives them to the loader
 * in a words block at byte 48 (instead of the event block):
 * {u32 magic 0x50464C57 ('PFLW'), u32 count, u64 value, u32 kind,
 * u32 reserved, u64 address, u64 alloc_size, u64 offset, 64-byte handle}.
 * The loader writes value into word l once layer l's bytes are in place
 * (pf_load_layers_marked), and into every word when the load fails after it
 * mapped them; the consumer gates a stream on word l with
 * pf_stream_wait_word(word_l, value), at any time after the load request.
 * kind PF_LAYER_WORDS_IPC: the words are at offset inside the allocation of
 * alloc_size bytes exported as handle (pf_ipc_export); kind
 * PF_LAYER_WORDS_LOCAL: at address, in the loader's own process. */
enum { PF_LAYER_WORDS_IPC = 0, PF_LAYER_WORDS_LOCAL = 1 };
typedef struct pf_layer_words {
  uint32_t kind;
  uint32_t reserved; /* 0 */
  uint64_t value;    /* nonzero; larger than any earlier load's on the same words */
  uint64_t address;
  uint64_t alloc_size;
  uint64_t offset;
  uint8_t handle[PF_IPC_HANDLE_BYTES];
} pf_layer_words;
int pf_load_state_create_layered_words(uint32_t num_layers,
                                       const pf_layer_words* words,
                                       pf_load_state** out);
/* The words block of a state: *count = its layer count (0 when the state has
 * none, *out untouched). */
int pf_load_state_layer_words(const pf_load_state* state, pf_layer_words* out,
                              uint32_t* count);

/* ------------------------------------------------------------------------ */
/* Pool allocator.  Replaces ScaledOffsetAllocator (allocator.rs:66-171):     */
/* byte requests rounded up to whole units, 32-bit unit counts.               */
/* ------------------------------------------------------------------------ */
typedef struct pf_allocator pf_allocator;
/* unit_size 0 is "unit size must be greater than zero" (allocator.rs:110). */
int pf_allocator_create(uint64_t total_bytes, uint64_t unit_size,
                        pf_allocator** out);
/* Smallest unit that keeps the unit count within 32 bits (allocator.rs:77-86). */
int pf_allocator_create_auto(uint64_t total_bytes, pf_allocator** out);
int pf_allocator_destroy(pf_allocator* a);
/* *found = 0 when no free region fits (or size_bytes == 0); a request whose
 * unit count exceeds 32 bits is PF_ERR_INVALID_ARGUMENT (RequestTooLarge). */
int pf_allocator_allocate(pf_allocator* a, uint64_t size_bytes, int* found,
                          uint64_t* offset, uint64_t* size);
int pf_allocator_free(pf_allocator* a, uint64_t offset);
/* StorageReportBytes plus totals (allocator.rs:157-177). */
int pf_allocator_report(pf_allocator* a, uint64_t* total_bytes,
                        uint64_t* free_bytes, uint64_t* largest_free_bytes,
                        uint64_t* unit_size);

/* ------------------------------------------------------------------------ */
/* Engine.  Replaces PegaEngine (lib.rs:93-1069) with its StorageEngine       */
/* (storage.rs) and GpuWorkerPool (gpu_worker.rs).  Names and argument order  */
/* follow the reference's Python bindings (python/src/lib.rs:122-261).        */
/* Hash lists are passed as one byte buffer and n+1 offsets: hash i is        */
/* hash_data[hash_offsets[i] .. hash_offsets[i+1]).                           */
/* ------------------------------------------------------------------------ */
typedef struct pf_engine pf_engine;
enum {
  PF_POOL_PINNED = 0, /* hipHostMalloc pool, mapped for device access        */
  PF_POOL_HOST = 1    /* plain host memory: bookkeeping only, no transfers   */
};
/* PegaEngine::new_with_pool_size (lib.rs:284-288).  unit_hint 0 = default. */
int pf_engine_create(uint64_t pool_bytes, uint32_t pool_kind,
                     uint32_t pinned_flags, uint64_t unit_hint,
                     pf_engine** out);
int pf_engine_destroy(pf_engine* e);
/* Transfer strategies used by saves and loads.  Defaults: PF_MODE_AUTO both
 * ways: a save batch's host regions, and a load of blocks saved together,
 * are long runs, so they run staged on the copy engines and leave the
 * device's other kernels at their speed; a load of a few scattered blocks
 * takes the kernel.  A load whose LoadState carries per-layer events runs
 * the kernel mode instead of the staged one (its events are recorded at
 * issue).  The workers' contexts have staging for every mode.  An AUTO load
 * is resolved from its first layer's block list. */
int pf_engine_set_modes(pf_engine* e, uint32_t save_mode, uint32_t load_mode);
/* register_context_layer (lib.rs:373-469). */
int pf_engine_register_context_layer(pf_engine* e, const char* instance_id,
                                     const char* namespace_, int device_id,
                                     const char* layer_name, uint64_t data_ptr,
                                     uint64_t size_bytes, uint64_t num_blocks,
                                     uint64_t bytes_per_block,
                                     uint64_t kv_stride_bytes,
                                     uint64_t segments, uint64_t tp_rank,
                                     uint64_t tp_size, uint64_t num_layers);
/* unregister_instance (lib.rs:473-484). */
int pf_engine_unregister_instance(pf_engine* e, const char* instance_id);
/* count_prefix_hit_blocks (lib.rs:803-838). */
int pf_engine_count_prefix_hit_blocks(pf_engine* e, const char* instance_id,
                                      const uint8_t* hash_data,
                                      const uint64_t* hash_offsets, uint64_t n,
                                      uint64_t* hits);
/* One layer of a save batch: (layer_name, block_ids, block_hashes). */
typedef struct pf_save_layer {
  const char* layer_name;
  const int32_t* block_ids;
  uint64_t num_blocks;
  const uint8_t* hash_data;
  const uint64_t* hash_offsets;
} pf_save_layer;
/* batch_save_kv_blocks_from_ipc (lib.rs:497-782): blocking; every layer of
 * the batch is copied by one batched transfer. */
int pf_engine_batch_save(pf_engine* e, const char* instance_id,
                         uint64_t tp_rank, int device_id,
                         const pf_save_layer* layers, uint32_t num_layers);
/* batch_load_kv_blocks_multi_layer (lib.rs:957-1069): returns once the load
 * is queued; completion (and, for a layered LoadState, per-layer progress) is
 * published in the LoadState named load_state_shm. */
int pf_engine_batch_load(pf_engine* e, const char* instance_id,
                         uint64_t tp_rank, int device_id,
                         const char* load_state_shm,
                         const char* const* layer_names, uint32_t num_layers,
                         const int32_t* block_ids, const uint8_t* hash_data,
                         const uint64_t* hash_offsets, uint64_t n);
typedef struct pf_engine_stats {
  uint64_t pool_used_bytes;
  uint64_t pool_total_bytes;
  uint64_t sealed_blocks;
  uint64_t inflight_blocks;
  uint64_t evicted_blocks;
  uint64_t saved_bytes;
  uint64_t loaded_bytes;
  uint64_t load_failures;
  uint64_t admission_rejections; /* new blocks TinyLFU refused (cache.rs:84-92) */
  uint64_t pre_evicted_blocks;   /* blocks the pre-eviction monitor evicted    */
} pf_engine_stats;
int pf_engine_stats_get(pf_engine* e, pf_engine_stats* out);
/* Storage policy (replaces StorageConfig and PreEvictConfig, storage.rs:43-111,
 * and TinyLfuCache's sizing, cache.rs:33-47).
 *  - lfu_admission: TinyLFU admission of newly sealed blocks and of blocks read
 *    back from disk (cache.rs:71-95): each is recorded in a count-min sketch,
 *    and refused when its estimate is below that of the least recently used
 *    block; lookup hits are recorded too.  The sketch is sized for
 *    pool_bytes / value_size_hint entries (value_size_hint 0: 128 MiB, as the
 *    reference's default).  Off by default here; the reference turns it on by
 *    default, where its 128 MiB sizing for KV blocks of a few MiB makes the
 *    sketch's collisions decide (replayed on the host: 9-17% of new 2 MiB
 *    blocks refused under a save/load mix).
 *  - pre_evict: a thread that every interval_ms evicts least-recently-used
 *    blocks while the pool's free bytes are below threshold_bytes, until
 *    target_bytes are free (storage.rs:646-688).  0 stops it.
 * May be called again at any time; admission restarts with an empty sketch. */
int pf_engine_set_storage_policy(pf_engine* e, int lfu_admission, uint64_t value_size_hint,
                                 int pre_evict, uint64_t threshold_bytes,
                                 uint64_t target_bytes, uint32_t interval_ms);
/* Block until every queued load has finished. */
int pf_engine_wait_idle(pf_engine* e);

/* ------------------------------------------------------------------------ */
/* The engine's decoder of the Engine service's request bytes (no           */
/* counterpart in the reference, whose tonic service decodes with prost:    */
/* service.rs:184-250).  Requests mean what the gRPC service's Load and Save */
/* mean.                                                                     */
/* ------------------------------------------------------------------------ */
enum { PF_REQUEST_LOAD = 1, PF_REQUEST_SAVE = 2, PF_REQUEST_HEALTH = 3 };
/* Largest request message the native gRPC server accepts. */
#define PF_REQUEST_MAX_BYTES (256u << 20)
/* One request (method PF_REQUEST_*; the engine.proto LoadRequest or
 * SaveRequest message bytes, none for Health), served on the calling
 * thread, for a server that receives the bytes itself (the native gRPC
 * server's Load and Save).  A request that does not decode fails with
 * PF_ERR_MALFORMED. */
int pf_engine_serve_request(pf_engine* engine, uint32_t method,
                            const uint8_t* request, uint64_t size);

/* ------------------------------------------------------------------------ */
/* Native gRPC server for the Engine service (service.rs:133-405, served by  */
/* the reference from Rust with tonic): engine.proto over HTTP/2 without     */
/* TLS, as an insecure gRPC channel connects.  Load and Health are served on */
/* the connection's thread and Save on a worker thread, by the engine's own  */
/* decoder of the request bytes (pf_engine_serve_request), with engine       */
/* errors mapped to gRPC codes as service.rs:77-88 does.  The other RPCs go  */
/* to the caller's handler.                                                  */
/* ------------------------------------------------------------------------ */
typedef struct pf_grpc_server pf_grpc_server;
typedef struct pf_grpc_call pf_grpc_call;
/* Called on one of the server's threads with the RPC's name within the
 * service ("RegisterContext", "Query", ...) and its request message bytes;
 * answers with pf_grpc_reply before returning (a call left unanswered fails
 * with INTERNAL). */
typedef void (*pf_grpc_handler)(void* ctx, pf_grpc_call* call, const char* method,
                                const uint8_t* request, uint64_t size);
/* Listens on address "host:port" (an IPv6 host in brackets; port 0: a free
 * port, see pf_grpc_port).  handler may be null: the other RPCs then fail
 * with UNIMPLEMENTED. */
int pf_grpc_start(pf_engine* engine, const char* address, pf_grpc_handler handler,
                  void* ctx, pf_grpc_server** out);
int pf_grpc_port(const pf_grpc_server* server);
/* Requests dispatched so far. */
uint64_t pf_grpc_served(const pf_grpc_server* server);
/* The answer to a call handed to the handler, once: gRPC status 0 with the
 * response message bytes, or an error status with its message. */
int pf_grpc_reply(pf_grpc_call* call, uint32_t status, const char* message,
                  const uint8_t* response, uint64_t size);
/* Stops listening, closes every connection and waits for the server's
 * threads; handler calls already running finish first. */
int pf_grpc_stop(pf_grpc_server* server);

/* ------------------------------------------------------------------------ */
/* Disk tier.  Replaces the DFS offload and prefetch of seal_offload.rs and   */
/* the Redis index behind it (BlockMeta, seal_offload.rs:72-97) with packed   */
/* files "<root>/<namespace>/<uuid>.bin" plus a "<uuid>.json" sidecar each.   */
/* ------------------------------------------------------------------------ */
/* spawn_dfs_offload_task (seal_offload.rs:169-191) with DfsOffloadConfig
 * (seal_offload.rs:45-69): every block sealed from now on is written to disk
 * in batches of up to max_pack_blocks; files already under root are indexed.
 * Enable before the first save.  0 picks the default for max_pack_blocks
 * (64), max_prefetch_tasks (16) and io_threads (4). */
int pf_engine_enable_disk(pf_engine* e, const char* root, uint64_t quota_bytes,
                          uint32_t max_pack_blocks, uint32_t max_prefetch_tasks,
                          uint32_t io_threads);
enum {
  PF_PREFETCH_READY = 0,       /* PrefetchState, engine.proto:66-74 */
  PF_PREFETCH_LOADING = 1,
  PF_PREFETCH_PARTIAL_MISS = 2
};
typedef struct pf_prefetch_status {
  int32_t state;
  uint32_t reserved;
  uint64_t hit_blocks;
  uint64_t loading_blocks;
  uint64_t missing_blocks;
} pf_prefetch_status;
/* count_prefix_hit_blocks_async (lib.rs:855-941): cache hits, then blocks
 * being read; when the first other block is on disk, a background read of
 * the rest of the prefix starts and the call reports it as loading.  Without
 * a disk tier: the plain prefix count, state READY. */
int pf_engine_query_prefetch(pf_engine* e, const char* instance_id,
                             const uint8_t* hash_data,
                             const uint64_t* hash_offsets, uint64_t n,
                             pf_prefetch_status* out);
/* No counterpart in the reference (tests, benchmarks, orderly shutdown):
 * block until every queued block is on disk / no disk read is in flight. */
int pf_engine_disk_flush(pf_engine* e);
int pf_engine_disk_wait_prefetch(pf_engine* e);
typedef struct pf_disk_stats {
  uint64_t files;
  uint64_t bytes;
  uint64_t indexed_blocks;
  uint64_t offloaded_blocks;
  uint64_t written_bytes;
  uint64_t prefetched_blocks;
  uint64_t read_bytes;
  uint64_t pending_blocks;
  uint64_t evicted_files;
  uint64_t failures;
} pf_disk_stats;
int pf_engine_disk_stats(pf_engine* e, pf_disk_stats* out);
/* No counterpart in the reference (inspection for tests and tools): copy the
 * host bytes of one slot of a cached block, K half then V half, into dst.
 * *k_bytes / *v_bytes receive the sizes (v 0 for a contiguous slot). */
int pf_engine_read_block_slot(pf_engine* e, const char* namespace_,
                              const uint8_t* hash, uint64_t hash_len,
                              uint64_t slot, uint8_t* dst, uint64_t dst_len,
                              uint64_t* k_bytes, uint64_t* v_bytes);

#ifdef __cplusplus
}
#endif

#endif /* PEGAFLOW_HIP_H */
