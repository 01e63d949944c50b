// pf_common.h — internal helpers shared by the pegaflow_hip sources.
#pragma once

#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdint>
#include <functional>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/pegaflow_hip.h"

namespace pf {

// Thread-local last-error message (pf_last_error).
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
std::string strf(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Per-call phase timings on stderr when PEGAFLOW_TRACE is set (the role of
// the reference's tracing spans and per-task GB/s logs, gpu_worker.rs:293-314);
// absolute times are CLOCK_MONOTONIC microseconds, comparable across the
// processes of one host.
bool tracing();
double mono_us(std::chrono::steady_clock::time_point t);
long thread_minor_faults();  // of the calling thread, for traces

// Returns PF_ERR_HIP with "<what> failed: <hip error string>" on error.
int hip_fail(hipError_t e, const char* what);

#define PF_HIP(call)                                   \
  do {                                                 \
    hipError_t pf_e_ = (call);                         \
    if (pf_e_ != hipSuccess) return ::pf::hip_fail(pf_e_, #call); \
  } while (0)

// One copy unit for the gather/scatter kernels: `chunk_bytes` bytes from
// src to dst (device-visible addresses; chunk size is uniform per launch).
struct ChunkDesc {
  uint64_t src;
  uint64_t dst;
};

// Where a load marks each finished layer: word[layer] of each target is set
// to that target's value.  Bit i of host_mask: target i is host memory.
constexpr uint32_t kMaxSignalTargets = PF_MAX_LAYER_SIGNALS;
struct SignalTargets {
  uint64_t words[kMaxSignalTargets];
  uint64_t value[kMaxSignalTargets];
  uint32_t host_mask;
  uint32_t count;
};

// The layers of one marking launch: chunks [chunk_start[g], chunk_start[g+1])
// of the launch belong to call layer layer[g] (every group non-empty);
// counters[layer] counts finished tiles and is 0 between launches.
struct LayerMarks {
  const uint32_t* chunk_start;  // n + 1 entries, device memory
  const uint32_t* layer;        // n entries, device memory
  uint32_t n;
  uint32_t* counters;
  SignalTargets targets;
};

// The layers of one marked scatter of a staged slice (passed by value, so
// the kernel reads them from its arguments): chunks [chunk_start[g],
// chunk_start[g+1]) of the launch belong to call layer layer[g], for g < n
// (every group non-empty, n <= kSliceMarkLayers).  tiles[g] is the layer's
// tile count over all the launches that copy it (a layer may span slices:
// counters[layer] adds up across them and the launch that reaches the count
// marks the layer), or 0 for a layer marked otherwise (not counted).
constexpr uint32_t kSliceMarkLayers = 8;
struct SliceMarks {
  uint32_t n;
  uint32_t chunk_start[kSliceMarkLayers + 1];
  uint32_t layer[kSliceMarkLayers];
  uint32_t tiles[kSliceMarkLayers];
  uint32_t* counters;
  SignalTargets targets;
};

// Layers marked by mark_layers_kernel (passed by value).
constexpr uint32_t kLayerListMax = 64;
struct LayerList {
  uint32_t n;
  uint32_t ids[kLayerListMax];
};

// Kernel launchers (pf_kernels.hip).
hipError_t launch_copy_chunks(const ChunkDesc* d_descs, uint32_t n_chunks,
                              uint64_t chunk_bytes, bool aligned16,
                              uint32_t threads, uint32_t unroll,
                              uint32_t max_grid, hipStream_t stream);
// The queued copy (16-byte aligned chunks only): `grid` persistent
// workgroups pull tiles from the two-word queue at `queue` (device memory),
// which holds 0, 0 when the launch starts and again when it ends.  Launches
// that may run at the same time need separate queues.  With marks, each
// finished layer is marked.
hipError_t launch_copy_chunks_queue(const ChunkDesc* d_descs, uint32_t n_chunks,
                                    uint64_t chunk_bytes, uint32_t threads, uint32_t unroll,
                                    uint32_t grid, const LayerMarks* marks,
                                    uint32_t* queue, uint32_t* n_tiles, hipStream_t stream);
// A marked copy between device buffers with a fixed workgroup -> tile map
// (16-byte aligned chunks): each finished layer of `marks` is marked.
hipError_t launch_copy_chunks_marked(const ChunkDesc* d_descs, uint32_t n_chunks,
                                     uint64_t chunk_bytes, uint32_t threads, uint32_t unroll,
                                     uint32_t grid, const SliceMarks& marks,
                                     hipStream_t stream);
hipError_t launch_mark_layers(const LayerList& list, const SignalTargets& t,
                              hipStream_t stream);
hipError_t launch_wait_word(uint64_t word, uint64_t value, uint64_t max_ticks,
                            uint64_t timed_out, hipStream_t stream);
hipError_t launch_fill_random(uint64_t dst, uint64_t size_bytes, uint64_t seed,
                              uint64_t word_offset, hipStream_t stream);
hipError_t launch_verify_random(uint64_t addr, uint64_t size_bytes,
                                uint64_t seed, uint64_t word_offset,
                                unsigned long long* d_count,
                                hipStream_t stream);
hipError_t launch_verify_random_chunks(const uint64_t* d_addrs,
                                       const uint64_t* d_word_offsets,
                                       uint64_t n, uint64_t chunk_bytes,
                                       uint64_t seed,
                                       unsigned long long* d_count,
                                       hipStream_t stream);
hipError_t launch_compare(uint64_t a, uint64_t b, uint64_t size_bytes,
                          unsigned long long* d_count, hipStream_t stream);
hipError_t launch_spin(uint64_t ticks, hipStream_t stream);

// Registry of pinned allocations made by pf_pinned_allocate, so that kernels
// are only ever given host ranges that are mapped for device access.
void pinned_register(uint64_t base, uint64_t size);
void pinned_unregister(uint64_t base);
// True when [addr, addr+len) lies inside one registered pinned allocation;
// *base/*end receive that allocation's bounds.
bool pinned_lookup(uint64_t addr, uint64_t len, uint64_t* base, uint64_t* end);

// DMA copies over the host link on chosen copy engines (pf_runtime.cpp).  The
// HIP runtime gives each copy an engine of its own choosing, and the 16
// engines of an MI355X move host data at very different rates (measured,
// 1 GiB each: device to host 57.1 GB/s on engines 0-3, 7-13 GB/s on the
// others; host to device 57.6 down to 28 GB/s), so a process whose copies
// land on a slow engine moves them at a fraction of the link's speed.
// These copies use the runtime's preferred engines for each direction,
// different ones for each direction where it allows.
//
// A signal counts a batch's copies still in flight (0: none).
struct EngineSignal {
  uint64_t handle = 0;
};
// True when the device's engines for both directions are known.
bool engine_copies_available(int device);
// The engine id bits in use for each direction, one or two each (false,
// and 0, when unknown).
bool engine_ids(int device, uint32_t* d2h, uint32_t* h2d);
// Sets the engines of either direction (a mask of one or two engine id
// bits; 0 keeps that direction's); copies issued afterwards use them.
int set_engine_ids(int device, uint32_t d2h, uint32_t h2d);
int engine_signal_create(EngineSignal* s);  // value 0
void engine_signal_destroy(EngineSignal* s);
// Adds n to the count before n copies are submitted against the signal.
void engine_signal_add(EngineSignal* s, int64_t n);
// One copy of `bytes` on one of the device's engines for the direction (d2h:
// device to host; `lane` alternates between the direction's two engines).
// The host side must lie in pinned memory.  On success the signal drops by
// one when the copy is done; on failure it is dropped here.
int engine_copy(int device, bool d2h, uint64_t dst, uint64_t src, uint64_t bytes,
                EngineSignal* s, unsigned lane);
// Waits until the signal reads 0 (an error after kEngineWaitSeconds):
// asleep until the copy's completion interrupt, or, with spin, polling the
// signal (about 25 us sooner, for a core kept busy meanwhile).
constexpr int kEngineWaitSeconds = 60;
int engine_signal_wait(EngineSignal* s, bool spin = false);

// Address validation for kernel access.  A kernel that touches an unmapped
// address faults the GPU, so every range a kernel will touch is checked
// first: it must lie inside one pinned allocation made by pf_pinned_allocate
// or inside one device allocation.  Results are cached for the lifetime of
// the object only (allocations may be freed between calls).
class RangeCache {
 public:
  bool check(uint64_t addr, uint64_t len);

 private:
  bool contains(uint64_t addr, uint64_t len);
  std::vector<std::pair<uint64_t, uint64_t>> ok_;  // [begin, end)
  uint64_t last_b_ = 0, last_e_ = 0;
};

// Whether this process's runtime exports interprocess events: 1 yes, 0 no
// (it refuses hipIpcGetEventHandle; *why then holds its error), -1 no device
// to ask.  Probed once, on the current device, with one throwaway event.
int ipc_events_supported(std::string* why = nullptr);
// PF_ERR_UNSUPPORTED (message set) where ipc_events_supported says 0.
int refuse_ipc_events();

// Layout kind (PF_LAYOUT_*), shared by the transfer paths.
inline int layout_kind(const pf_kv_layout& l) {
  if (l.segments == 2 && l.kv_stride_bytes > l.bytes_per_block)
    return PF_LAYOUT_SPLIT;
  if (l.segments <= 1 || l.kv_stride_bytes == l.bytes_per_block)
    return PF_LAYOUT_CONTIGUOUS;
  return PF_LAYOUT_STRIDED;
}

// segment_offset with the reference's checks; message set on failure.
int segment_offset(const pf_kv_layout& l, uint64_t block, uint64_t seg,
                   uint64_t* out);

// Static device scratch of pf_load_layers_noalloc (one copy per device,
// held until the process ends): the tile queue in the first 256 bytes, then
// up to PF_NOALLOC_MAX_CHUNKS chunk descriptors.
constexpr uint64_t kNoAllocQueueBytes = 256;
constexpr uint64_t kNoAllocScratchBytes =
    kNoAllocQueueBytes + PF_NOALLOC_MAX_CHUNKS * sizeof(ChunkDesc);
struct NoAllocScratch {
  uint64_t base = 0;        // device address of the device's copy of the array
  std::mutex mu;            // host-side bookkeeping of calls on this device
};
// The device's scratch.  The array's address is looked up once per device,
// with that device current (pf_init does it; a first call on a device that
// pf_init never saw does it then).
int noalloc_scratch(int device, NoAllocScratch** out);

// pf_save_layers without its final wait: the copy may still be in flight on
// the context's stream when this returns; pf_xfer_synchronize completes it.
// The staged mode still waits.  For callers that overlap host work with the
// copy and must not use the bytes before the wait.
int save_layers_begin(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                      uint32_t mode);

// Layers [head, num_layers) of a load whose block lists another thread is
// still building.  In kernel mode the call plans and issues layers
// [0, head) first, then calls ready(), which returns PF_OK once every later
// entry of the call's layer array holds its blocks (an error fails the call,
// with the first part drained), and issues the rest; descriptor room for
// the later layers is reserved beforehand from max_blocks, a bound on each
// one's block count.  In the other modes, or with head 0, ready() is called
// before anything is issued.
struct PendingLayers {
  uint32_t head = 0;
  uint64_t max_blocks = 0;
  std::function<int()> ready;
};
// save_layers_begin for a save whose later layers are pending: in the
// kernel and staged modes the first `head` layers' copies start before
// ready() is called; the other modes call it before anything is issued.
int save_layers_pending_begin(pf_xfer* x, pf_layer_xfer* layers, uint32_t num_layers,
                              uint32_t mode, const PendingLayers& pending);
// A load whose later layers are pending: layer_events as pf_load_layers',
// signals as pf_load_layers_marked's (num_signals 0: no marks).
int load_layers_pending(pf_xfer* x, pf_layer_xfer* layers, uint32_t num_layers, uint32_t mode,
                        pf_event* layer_events, const pf_layer_signal* signals,
                        uint32_t num_signals, const PendingLayers& pending);
// The leading layers that a kernel-mode call over the host link of
// num_layers layers and `chunks` chunks in all plans and issues before
// planning the rest (0: the call is planned whole).
uint32_t pipeline_head_layers(uint32_t num_layers, uint64_t chunks);

// The mode a call in `mode` runs in on context x: PF_MODE_AUTO resolved
// against the layers' host-side runs and the context's staging; other modes
// unchanged.
uint32_t resolve_mode(const pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                      uint32_t mode);

// Writes the signal's value into all num_layers words on the context's
// stream and waits: releases consumers of a load that failed before its
// marks were written.
int mark_all_layers(pf_xfer* x, const pf_layer_signal& signal, uint32_t num_layers);

}  // namespace pf
