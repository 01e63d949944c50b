// pf_transfer.cpp — the transfer module: reference-equivalent DMA primitives
// (transfer.rs) and the batched transfer context that replaces the per-call
// copy loops of gpu_worker.rs with gather/scatter kernels.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

#include "pf_common.h"
#include "pf_staged.h"

using namespace pf;

namespace {

// ---------------------------------------------------------------------------
// Chunk planning.  A layer's transfer is a list of equal-size chunks, each
// pairing a device address inside the paged layer tensor with an address on
// the other side (host pinned memory, or any device-visible buffer).
// ---------------------------------------------------------------------------
// Chunks of distinct blocks never overlap in the layer tensor: split layouts
// whose V region starts past the K region, and single-segment layouts.  Other
// registrations (allowed by the reference's validation, never produced by
// vLLM) can make two blocks' chunks overlap, where the reference's in-order
// copies decide which bytes win.
bool device_chunks_disjoint(const pf_kv_layout& l) {
  const int kind = layout_kind(l);
  if (kind == PF_LAYOUT_SPLIT) {
    uint64_t k_end = 0;
    return !__builtin_mul_overflow(l.num_blocks, l.bytes_per_block, &k_end) &&
           l.kv_stride_bytes >= k_end;
  }
  return kind == PF_LAYOUT_CONTIGUOUS && l.segments <= 1;
}

// Host-side chunks are pairwise disjoint (checked in O(n) for the usual
// increasing order, else after sorting a copy).
bool host_chunks_disjoint(const LayerPlan& p) {
  bool increasing = true;
  for (size_t i = 1; i < p.chunks.size() && increasing; ++i)
    increasing = p.chunks[i].host >= p.chunks[i - 1].host + p.chunk_bytes;
  if (increasing) return true;
  std::vector<uint64_t> h(p.chunks.size());
  for (size_t i = 0; i < h.size(); ++i) h[i] = p.chunks[i].host;
  std::sort(h.begin(), h.end());
  for (size_t i = 1; i < h.size(); ++i)
    if (h[i] < h[i - 1] + p.chunk_bytes) return false;
  return true;
}

// segment_offset without its per-call checks for the common case: blocks up
// to max_block have an in-bounds segment `seg` at block*bpb + seg_off; any
// other block goes through segment_offset itself, for its exact error.
struct SegBound {
  bool any = false;  // false: no block is in bounds
  uint64_t seg_off = 0;
  uint64_t max_block = 0;
};

SegBound seg_bound(const pf_kv_layout& l, uint64_t seg, uint64_t bytes) {
  SegBound b;
  uint64_t off = 0, need = 0;
  if (seg >= l.segments || l.bytes_per_block == 0 ||
      __builtin_mul_overflow(seg, l.kv_stride_bytes, &off) ||
      __builtin_add_overflow(off, bytes, &need) || need > l.size_bytes)
    return b;
  b.any = true;
  b.seg_off = off;
  b.max_block = (l.size_bytes - need) / l.bytes_per_block;
  return b;
}

int plan_layer(const pf_layer_xfer& lx, bool is_save, LayerPlan* out) {
  const pf_kv_layout& l = lx.layout;
  if (l.bytes_per_block == 0 || l.segments == 0 || l.num_blocks == 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "invalid KV cache layout");
  if (lx.num_blocks > 0 && !lx.blocks)
    return fail(PF_ERR_INVALID_ARGUMENT, "null block list");
  const uint64_t seg = l.bytes_per_block;
  const int kind = layout_kind(l);
  out->chunks.clear();
  for (uint64_t i = 0; i < lx.num_blocks; ++i) {
    if (lx.blocks[i].block_idx < 0)
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("block index %lld must be >= 0",
                       (long long)lx.blocks[i].block_idx));
    if (lx.blocks[i].k_host == 0)
      return fail(PF_ERR_INVALID_ARGUMENT, "null host address for block");
  }
  uint64_t off = 0;
  // Offset of segment s of a block, with segment_offset's checks: the
  // precomputed bound admits the block, or segment_offset reports why not.
  auto offset_of = [&](const SegBound& sb, uint64_t block, uint64_t s, uint64_t* o) -> int {
    if (sb.any && block <= sb.max_block) {
      *o = block * seg + sb.seg_off;
      return PF_OK;
    }
    return segment_offset(l, block, s, o);
  };
  if (kind == PF_LAYOUT_SPLIT) {
    // gpu_worker.rs:226-240 (load) and 334-360 (save): K list, then V list.
    out->chunk_bytes = seg;
    out->chunks.reserve(lx.num_blocks * 2);
    const SegBound k = seg_bound(l, 0, seg), v = seg_bound(l, 1, seg);
    for (uint64_t i = 0; i < lx.num_blocks; ++i) {
      const pf_block_xfer& b = lx.blocks[i];
      if (int rc = offset_of(k, static_cast<uint64_t>(b.block_idx), 0, &off)) return rc;
      out->chunks.push_back({l.data_ptr + off, b.k_host});
    }
    out->list_break = out->chunks.size();
    for (uint64_t i = 0; i < lx.num_blocks; ++i) {
      const pf_block_xfer& b = lx.blocks[i];
      if (int rc = offset_of(v, static_cast<uint64_t>(b.block_idx), 1, &off)) return rc;
      out->chunks.push_back({l.data_ptr + off, b.v_host ? b.v_host : b.k_host + seg});
    }
    return PF_OK;
  }
  if (kind == PF_LAYOUT_STRIDED && is_save) {
    // copy_gpu_to_cpu_strided (transfer.rs:217-239): segment s of block b to
    // dst + s * bytes_per_block.
    out->chunk_bytes = seg;
    out->chunks.reserve(lx.num_blocks * l.segments);
    for (uint64_t i = 0; i < lx.num_blocks; ++i) {
      const pf_block_xfer& b = lx.blocks[i];
      for (uint64_t s = 0; s < l.segments; ++s) {
        if (int rc = segment_offset(l, static_cast<uint64_t>(b.block_idx), s, &off)) return rc;
        out->chunks.push_back({l.data_ptr + off, b.k_host + s * seg});
      }
    }
    out->list_break = out->chunks.size();
    return PF_OK;
  }
  // Whole block of block_size_bytes at segment_offset(b, 0): the contiguous
  // save (transfer.rs:206-210) and every non-split load (gpu_worker.rs:260-282).
  const uint64_t bs = l.block_size_bytes;
  out->chunk_bytes = bs;
  out->chunks.reserve(lx.num_blocks);
  // Blocks within this bound pass both segment_offset(b, 0) and the
  // whole-block end check below.
  const SegBound whole = seg_bound(l, 0, bs >= seg ? bs : seg);
  for (uint64_t i = 0; i < lx.num_blocks; ++i) {
    const pf_block_xfer& b = lx.blocks[i];
    const uint64_t block = static_cast<uint64_t>(b.block_idx);
    if (whole.any && block <= whole.max_block) {
      out->chunks.push_back({l.data_ptr + block * seg, b.k_host});
      continue;
    }
    if (int rc = segment_offset(l, block, 0, &off)) return rc;
    uint64_t end = 0;
    if (__builtin_add_overflow(off, bs, &end) || end > l.size_bytes)
      return fail(PF_ERR_STORAGE,
                  strf("Block %lld exceeds registered memory (offset %llu, size "
                       "%llu, limit %llu)",
                       (long long)b.block_idx, (unsigned long long)off,
                       (unsigned long long)bs, (unsigned long long)l.size_bytes));
    out->chunks.push_back({l.data_ptr + off, b.k_host});
  }
  out->list_break = out->chunks.size();
  return PF_OK;
}

// Parallel kernels give the reference's bytes only when no two chunks write
// the same byte.  The reference copies in list order, so for a load that
// names a block twice the later copy wins: only the last occurrence is kept.
// Layouts whose blocks can overlap, loads naming a block past num_blocks, and
// kernel saves to overlapping host ranges are copied in list order instead.
// (The staged save writes the host side with in-order copies already.)
void apply_write_policy(const pf_layer_xfer& lx, bool is_save, bool staged, LayerPlan* p) {
  p->ordered = false;
  if (p->chunks.empty()) return;
  if (is_save) {
    p->ordered = !staged && !host_chunks_disjoint(*p);
    return;
  }
  if (!device_chunks_disjoint(lx.layout)) {
    p->ordered = true;
    return;
  }
  const uint64_t nb = lx.layout.num_blocks;
  const size_t n = static_cast<size_t>(lx.num_blocks);
  // Blocks seen in this layer: stamp[b] == epoch (a per-thread array reused
  // across layers and calls instead of a zeroed one per layer).
  thread_local std::vector<uint32_t> stamp;
  thread_local uint32_t epoch = 0;
  for (size_t i = 0; i < n; ++i)
    if (static_cast<uint64_t>(lx.blocks[i].block_idx) >= nb) {
      p->ordered = true;
      return;
    }
  if (stamp.size() < nb) stamp.resize(static_cast<size_t>(nb), 0);
  if (++epoch == 0) {  // wrapped: clear, so no old stamp can match
    std::fill(stamp.begin(), stamp.end(), 0);
    epoch = 1;
  }
  std::vector<uint8_t> keep;
  bool any_dup = false;
  for (size_t i = n; i-- > 0;) {
    const size_t b = static_cast<size_t>(lx.blocks[i].block_idx);
    if (stamp[b] == epoch) {
      if (!any_dup) keep.assign(n, 1);
      keep[i] = 0;
      any_dup = true;
    } else {
      stamp[b] = epoch;
    }
  }
  if (!any_dup) return;
  const size_t per_block = p->chunks.size() / n;  // 2 for split, 1 otherwise
  std::vector<Chunk> kept;
  kept.reserve(p->chunks.size());
  for (size_t part = 0; part < per_block; ++part) {
    for (size_t i = 0; i < n; ++i)
      if (keep[i]) kept.push_back(p->chunks[part * n + i]);
    if (part == 0) p->list_break = kept.size();
  }
  p->chunks.swap(kept);
  if (per_block == 1) p->list_break = p->chunks.size();
}

// The layer tensor must lie inside one device allocation and each host-side
// chunk inside one pinned or device allocation (RangeCache, pf_runtime.cpp).
int check_device_tensor(RangeCache& rc, const pf_kv_layout& l) {
  if (!rc.check(l.data_ptr, l.size_bytes))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("layer tensor [0x%llx, +%llu) is not inside one device "
                     "allocation",
                     (unsigned long long)l.data_ptr, (unsigned long long)l.size_bytes));
  return PF_OK;
}

int check_host_chunks(RangeCache& rc, const LayerPlan& p) {
  if (p.chunks.empty()) return PF_OK;
  // The usual case: every chunk inside one allocation (the pool), checked
  // as the span from the lowest to the end of the highest.
  uint64_t lo = p.chunks[0].host, hi = p.chunks[0].host;
  for (const Chunk& c : p.chunks) {
    lo = c.host < lo ? c.host : lo;
    hi = c.host > hi ? c.host : hi;
  }
  uint64_t end = 0;
  if (!__builtin_add_overflow(hi, p.chunk_bytes, &end) && rc.check(lo, end - lo)) return PF_OK;
  for (const Chunk& c : p.chunks)
    if (!rc.check(c.host, p.chunk_bytes))
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("host range [0x%llx, +%llu) is not device-accessible "
                       "(allocate it with pf_pinned_allocate)",
                       (unsigned long long)c.host, (unsigned long long)p.chunk_bytes));
  return PF_OK;
}

// Greedy run merging of transfer.rs:134-177 over chunks [begin, end): a run
// grows while the device and host addresses both continue chunk_bytes past
// the run's start.  Calls fn(first_chunk_index, n_chunks) per run.
template <class F>
void for_each_run(const LayerPlan& p, size_t begin, size_t end, F fn) {
  size_t i = begin;
  const uint64_t cb = p.chunk_bytes;
  while (i < end) {
    size_t n = 1;
    while (i + n < end && p.chunks[i + n].dev == p.chunks[i].dev + n * cb &&
           p.chunks[i + n].host == p.chunks[i].host + n * cb)
      ++n;
    fn(i, n);
    i += n;
  }
}

bool aligned16(uint64_t v) { return (v & 15u) == 0; }

}  // namespace

// Scatter shapes a context chooses between (route PF_ROUTE_LOAD_DEVICE with
// PF_KERNEL_AUTO).  Which is faster depends on where the destination tensors
// lie in HBM: measured into two sets of the 32 Llama layer tensors in one
// process, the first took 0.417 ms into one set and 0.498 ms into the other,
// the second 0.463 and 0.475 ms; the bytes moved are the same (every write a
// full 64 B request).  So a context times both on its first large scatters
// and keeps the faster.
constexpr uint32_t kScatterShapes[2][2] = {
    {512, 2u | PF_KERNEL_NONTEMPORAL | PF_KERNEL_XCD_MAJOR},
    {512, 1u | PF_KERNEL_NONTEMPORAL}};
constexpr int kScatterTrialsPerShape = 2;
constexpr uint64_t kScatterTrialMinBytes = 64ull << 20;  // time only launches this large

// Staging slots of a staged call on the copy engines, at most.
constexpr int kEngineSlots = 8;
// Largest slice of a staged load that reports each layer's completion.
constexpr uint64_t kLayeredLoadSlice = 64ull << 20;
// Shape of a marked staged load's scatter that marks its slice's layers
// itself (copy_chunks_marked_kernel): 512 threads, up to four non-temporal
// 16-byte loads per lane (a 32 KiB chunk is one tile), 128 workgroups.
// Each workgroup ends each of its layers with a release fence that writes
// its XCD's L2 back, so fewer, busier workgroups win: measured on 40 MiB
// layers of 32 KiB chunks, 24.8 us per layer with 128 workgroups and four
// loads per lane, 25.1 with 256, 32 with 512, 73 with 1,280, 108 with one
// workgroup per 8 KiB tile, 46 with 64.
constexpr uint32_t kMarkedScatterThreads = 512;
constexpr uint32_t kMarkedScatterGrid = 128;
// Loads per lane for chunks of chunk_bytes: the tile covers a chunk of up to
// 32 KiB, or 32 KiB of a larger one.
static uint32_t marked_unroll(uint64_t chunk_bytes) {
  const uint64_t c16 = chunk_bytes / 16;
  return c16 >= 4u * kMarkedScatterThreads ? 4u : c16 >= 2u * kMarkedScatterThreads ? 2u : 1u;
}

struct ScatterTrial {
  hipEvent_t start = nullptr, stop = nullptr;
  uint64_t bytes = 0;       // bytes of the launch being timed
  bool pending = false;     // recorded, not read back yet
  int done = 0;             // timed launches read back
  double best_ns_per_byte = 0;
};

// ---------------------------------------------------------------------------
// Transfer context.
// ---------------------------------------------------------------------------
struct pf_xfer {
  int device = 0;
  hipStream_t stream = nullptr;  // kernels; DMA for the DMA modes
  hipStream_t dma = nullptr;     // link-side copies of the staged mode
  ChunkDesc* d_desc = nullptr;
  size_t d_cap = 0;
  // Host staging of the descriptors for the upload.
  ChunkDesc* h_desc = nullptr;
  size_t h_cap = 0;
  hipEvent_t desc_uploaded = nullptr;
  bool desc_inflight = false;
  // Pipelined calls: recorded on the kernel stream before the call's first
  // part, i.e. once every earlier launch (a reader of the descriptors) ended.
  hipEvent_t parts_ready = nullptr;
  // Small calls: descriptors the kernels read in place from coherent pinned
  // memory (kHostDescMax entries), reused only once the stream has drained.
  ChunkDesc* h_small = nullptr;
  bool small_inflight = false;
  // The upload kernel's own descriptor, read in place: [0] for a call's
  // first part, [1] for a pipelined call's second part.
  ChunkDesc* h_boot = nullptr;
  // Descriptor base the next launches read: d_desc, or h_small.
  const ChunkDesc* desc_base = nullptr;
  // Staging for PF_MODE_STAGED: one slot per lane (stream, then dma), each
  // slot_bytes long, the first at `staging`.
  uint64_t staging = 0;
  uint64_t slot_bytes = 0;
  // Largest staged slice per direction (0: save, 1: load), capped by slot_bytes.
  uint64_t staged_slice[2] = {PF_STAGED_SAVE_SLICE_DEFAULT, PF_STAGED_LOAD_SLICE_DEFAULT};
  // A layer-by-layer staged load's first layer: PF_STAGED_HEAD_ENGINE or _KERNEL.
  uint32_t staged_head = PF_STAGED_HEAD_ENGINE;
  // Recorded on a lane for the other lane to wait on (one per lane).
  hipEvent_t lane_mark[2] = {nullptr, nullptr};
  // Staged copies on the copy engines (when the device's are known): one
  // completion signal and one kernel-done event per staging slot, and the
  // end of the last staged call's kernels on the context's stream.
  bool engine_ok = false;
  EngineSignal eng_sig[kEngineSlots];
  hipEvent_t eng_ev[kEngineSlots] = {};
  hipEvent_t staging_free = nullptr;
  // End of a pipelined staged load's first layer, copied by the kernel.
  hipEvent_t head_done = nullptr;
  // Launch shapes per route (PF_ROUTE_*), the fastest measured on MI355X:
  //   gather into HBM:   512 threads, one non-temporal 16 B load per lane
  //                      (8 KiB tiles), round-robin tile order;
  //   scatter:           512 threads, two non-temporal loads per lane (16 KiB
  //                      tiles), XCD-major tile order;
  //   save to the host:  512 threads, two streaming loads per lane, ordinary
  //                      stores into host memory.
  uint32_t threads[4] = {PF_SAVE_DEFAULT_THREADS, PF_LOAD_DEFAULT_THREADS,
                         PF_SAVE_HOST_DEFAULT_THREADS, PF_LOAD_HOST_DEFAULT_THREADS};
  uint32_t unroll[4] = {PF_SAVE_DEFAULT_UNROLL, PF_LOAD_DEFAULT_UNROLL,
                        PF_SAVE_HOST_DEFAULT_UNROLL, PF_LOAD_HOST_DEFAULT_UNROLL};
  uint32_t max_grid = 0;
  uint64_t last_kernels = 0;
  uint64_t last_dma = 0;
  bool timing = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> timers;  // one pair per launch
  // Per-layer tile counters of marking launches (0 between launches), and
  // after them one tile queue per lane (kernel stream, link-side stream),
  // each in a 256-byte line of its own: queued launches on the two lanes
  // may run at the same time.
  uint32_t* d_counters = nullptr;
  size_t counters_cap = 0;
  uint32_t* d_queue[2] = {nullptr, nullptr};
  // Persistent workgroups of a queued launch per route (0: a fixed
  // workgroup per tile).  Copies over the host link run queued.
  uint32_t grid[4] = {0, 0, PF_SAVE_HOST_DEFAULT_GRID, PF_LOAD_HOST_DEFAULT_GRID};
  // The scatter route's choice between kScatterShapes (-1: still timing).
  ScatterTrial trials[2];
  int scatter_choice = -1;
  // Per-layer plans of the call in progress (under mu), kept with their
  // capacity for the next call: a call plans tens of thousands of chunks,
  // and fresh buffers each time cost page faults before the first launch.
  std::vector<LayerPlan> plans, plans_rest;
  std::mutex mu;
};

namespace {

int ensure_desc_capacity(pf_xfer* x, size_t n) {
  // The host staging of descriptors may still be read by the previous call's
  // upload; wait for it before rewriting.
  if (x->desc_inflight) {
    PF_HIP(hipEventSynchronize(x->desc_uploaded));
    x->desc_inflight = false;
  }
  if (n > x->h_cap) {
    size_t cap = 1;
    while (cap < n) cap <<= 1;
    if (x->h_desc) PF_HIP(hipHostFree(x->h_desc));
    x->h_desc = nullptr;
    x->h_cap = 0;
    // Read in place by the upload kernel: mapped, and uncached on the device
    // (rewritten by the host between calls).
    PF_HIP(hipHostMalloc(reinterpret_cast<void**>(&x->h_desc), cap * sizeof(ChunkDesc),
                         hipHostMallocMapped | hipHostMallocCoherent));
    x->h_cap = cap;
  }
  if (n > x->d_cap) {
    size_t cap = 1;
    while (cap < n) cap <<= 1;
    // Kernels of earlier calls may still read the old buffer.
    PF_HIP(hipStreamSynchronize(x->dma));
    PF_HIP(hipStreamSynchronize(x->stream));
    if (x->d_desc) PF_HIP(hipFree(x->d_desc));
    x->d_desc = nullptr;
    x->d_cap = 0;
    PF_HIP(hipMalloc(reinterpret_cast<void**>(&x->d_desc), cap * sizeof(ChunkDesc)));
    x->d_cap = cap;
  }
  return PF_OK;
}

// Workgroup size of the descriptor upload kernel (4 KiB tiles).
constexpr uint32_t kDescUploadThreads = 256;

// Copies descriptors [off, off + n) of the host staging to the same place in
// device memory; the next launches read from there.  A later part of a
// pipelined call (off > 0) copies on the link-side stream, so the copy runs
// under the earlier part's kernel instead of between the two kernels, and
// the kernel stream waits for it.
int upload_desc(pf_xfer* x, size_t n, size_t off = 0) {
  x->desc_base = x->d_desc + off;
  if (n == 0) return PF_OK;
  hipStream_t s = off ? x->dma : x->stream;
  if (off) {
    // Not before earlier calls' kernels are done with this region, nor
    // before the first part's own upload (desc_uploaded, if it uploaded),
    // which the next call's reuse of the staging waits for through the
    // event recorded below.
    PF_HIP(hipStreamWaitEvent(s, x->parts_ready, 0));
    PF_HIP(hipStreamWaitEvent(s, x->desc_uploaded, 0));
  }
  // Copied by the chunk kernel, which reads the host staging in place (one
  // boot descriptor per part of a call, itself read in place), not by a DMA
  // copy: the process's DMA copies to the device share an engine queue, so a
  // staged restore's 1.25 GiB of copies held a concurrent save's 640 KiB
  // upload, and with it the whole save, for 28 ms.
  ChunkDesc* boot = x->h_boot + (off ? 1 : 0);
  *boot = ChunkDesc{reinterpret_cast<uint64_t>(x->h_desc + off),
                    reinterpret_cast<uint64_t>(x->d_desc + off)};
  (void)hipGetLastError();
  const hipError_t e = launch_copy_chunks(boot, 1, n * sizeof(ChunkDesc), true,
                                          kDescUploadThreads, 1, 0, s);
  if (e != hipSuccess) return hip_fail(e, "descriptor upload kernel launch");
  PF_HIP(hipEventRecord(x->desc_uploaded, s));
  if (off) PF_HIP(hipStreamWaitEvent(x->stream, x->desc_uploaded, 0));
  x->desc_inflight = true;
  return PF_OK;
}

// Small calls: a separate copy of the descriptors costs about 12 us before
// the first kernel can start, more than the kernels of a one-block load
// take.  Up to this many descriptors the kernels read them in place from
// coherent pinned memory (one 16-byte read over the host link per
// workgroup); larger calls upload them, since an HBM-bound launch would feel
// that read in every workgroup.
constexpr size_t kHostDescMax = 512;

// The in-place buffer for a call of n descriptors, or null when the call
// must upload (too many, or the previous in-place call may still be read).
ChunkDesc* small_desc(pf_xfer* x, size_t n) {
  if (n > kHostDescMax || !x->h_small) return nullptr;
  if (x->small_inflight) {
    if (hipStreamQuery(x->stream) != hipSuccess) {
      (void)hipGetLastError();  // still running (or an error the sync reports)
      return nullptr;
    }
    x->small_inflight = false;
  }
  return x->h_small;
}

// One gather/scatter launch of the n chunks at descs on `stream`.  With
// qgrid > 0 (16-byte aligned chunks only) it runs queued: qgrid persistent
// workgroups pull tiles from the queue at `queue`, which no launch that may
// overlap this one uses.  Otherwise one workgroup per tile (at most max_grid
// workgroups, 0 = no cap).
hipError_t issue_copy(hipStream_t stream, const ChunkDesc* descs, size_t n, uint64_t chunk_bytes,
                      bool al16, uint32_t threads, uint32_t unroll, uint32_t qgrid,
                      uint32_t max_grid, const LayerMarks* marks, uint32_t* queue) {
  (void)hipGetLastError();
  if (!(al16 && qgrid > 0))
    return launch_copy_chunks(descs, static_cast<uint32_t>(n), chunk_bytes, al16, threads, unroll,
                              max_grid, stream);
  // Chunks smaller than a tile (e.g. 4 KiB segments of one tensor-parallel
  // rank) get workgroups sized to the chunk, and proportionally more of
  // them, so each pull moves a whole chunk with every lane busy and the
  // bytes in flight stay the same (measured: 4 KiB-segment save 53.9 ->
  // 55.6 GB/s).
  const uint64_t u = unroll & 0xffu;
  const uint64_t want = ((chunk_bytes / 16 + u - 1) / u + 63) / 64 * 64;
  if (u > 0 && want < threads) {
    const uint32_t t2 = static_cast<uint32_t>(want < 64 ? 64 : want);
    const uint64_t g2 = static_cast<uint64_t>(qgrid) * threads / t2;
    qgrid = static_cast<uint32_t>(g2 < (1u << 16) ? g2 : (1u << 16));
    if (max_grid && qgrid > max_grid) qgrid = max_grid;
    threads = t2;
  }
  uint32_t n_tiles = 0;
  return launch_copy_chunks_queue(descs, static_cast<uint32_t>(n), chunk_bytes, threads, unroll,
                                  qgrid, marks, queue, &n_tiles, stream);
}

// Reads back finished scatter trials; once every candidate has been timed
// kScatterTrialsPerShape times, the faster (per byte, best run) is kept.
void scatter_trials_update(pf_xfer* x) {
  if (x->scatter_choice >= 0) return;
  for (ScatterTrial& t : x->trials) {
    if (!t.pending) continue;
    const hipError_t q = hipEventQuery(t.stop);
    if (q == hipErrorNotReady) {
      (void)hipGetLastError();
      continue;
    }
    t.pending = false;
    float ms = 0.f;
    if (q == hipSuccess && hipEventElapsedTime(&ms, t.start, t.stop) == hipSuccess && t.bytes) {
      const double v = ms * 1e6 / static_cast<double>(t.bytes);
      if (t.done == 0 || v < t.best_ns_per_byte) t.best_ns_per_byte = v;
      ++t.done;
    }
    (void)hipGetLastError();
  }
  if (x->trials[0].done >= kScatterTrialsPerShape && x->trials[1].done >= kScatterTrialsPerShape)
    x->scatter_choice = x->trials[0].best_ns_per_byte <= x->trials[1].best_ns_per_byte ? 0 : 1;
}

// The candidate a scatter of `bytes` runs with, and the trial to time it
// under (null: untimed).  Trials alternate between the candidates; launches
// too small to time, and launches while a trial is still running, use the
// first candidate.
int scatter_pick(pf_xfer* x, uint64_t bytes, ScatterTrial** timed) {
  *timed = nullptr;
  scatter_trials_update(x);
  if (x->scatter_choice >= 0) return x->scatter_choice;
  if (bytes < kScatterTrialMinBytes || x->trials[0].pending || x->trials[1].pending) return 0;
  const int i = x->trials[1].done < x->trials[0].done ? 1 : 0;
  ScatterTrial& t = x->trials[i];
  if (!t.start && hipEventCreate(&t.start) != hipSuccess) t.start = nullptr;
  if (t.start && !t.stop && hipEventCreate(&t.stop) != hipSuccess) t.stop = nullptr;
  (void)hipGetLastError();
  if (t.start && t.stop) *timed = &t;
  return i;
}

void scatter_trials_reset(pf_xfer* x) {
  x->scatter_choice = -1;
  for (ScatterTrial& t : x->trials) {
    t.pending = false;
    t.done = 0;
    t.best_ns_per_byte = 0;
  }
}

int check_launch_size(size_t n, uint64_t chunk_bytes) {
  if (n > 0xffffffffull) return fail(PF_ERR_INVALID_ARGUMENT, "too many chunks");
  if (chunk_bytes / 16 >= (1ull << 31)) return fail(PF_ERR_INVALID_ARGUMENT, "chunk too large");
  return PF_OK;
}

int launch(pf_xfer* x, size_t first, size_t n, uint64_t chunk_bytes, bool al16, bool is_save,
           bool host_side = false, const LayerMarks* marks = nullptr,
           hipStream_t stream = nullptr) {
  if (n == 0) return PF_OK;
  if (!stream) stream = x->stream;
  const int dir = (is_save ? PF_ROUTE_SAVE_DEVICE : PF_ROUTE_LOAD_DEVICE) + (host_side ? 2 : 0);
  if (int rc = check_launch_size(n, chunk_bytes)) return rc;
  std::pair<hipEvent_t, hipEvent_t>* tm = nullptr;
  if (x->timing) {
    if (x->last_kernels >= x->timers.size()) {
      std::pair<hipEvent_t, hipEvent_t> p{nullptr, nullptr};
      PF_HIP(hipEventCreate(&p.first));
      PF_HIP(hipEventCreate(&p.second));
      x->timers.push_back(p);
    }
    tm = &x->timers[x->last_kernels];
    PF_HIP(hipEventRecord(tm->first, stream));
  }
  // Queued launches: copies over the host link, and every marking launch
  // (its layers must land in order).  See copy_chunks_queue_kernel.
  uint32_t qgrid = x->grid[dir];
  if (marks && qgrid == 0) qgrid = PF_LOAD_HOST_DEFAULT_GRID;
  if (x->max_grid && qgrid > x->max_grid) qgrid = x->max_grid;
  // Each lane's launches run in its stream's order; the two lanes overlap.
  uint32_t* queue = x->d_queue[stream == x->dma ? 1 : 0];
  if (al16 && qgrid > 0 && !queue)
    return fail(PF_ERR_INVALID_ARGUMENT, "tile queue not allocated");
  if (marks && !(al16 && qgrid > 0))
    return fail(PF_ERR_INVALID_ARGUMENT, "a marking launch needs 16-byte aligned chunks");
  uint32_t threads = x->threads[dir], unroll = x->unroll[dir];
  ScatterTrial* trial = nullptr;
  if ((unroll & PF_KERNEL_AUTO) && dir == PF_ROUTE_LOAD_DEVICE && al16 && qgrid == 0) {
    const int pick = scatter_pick(x, static_cast<uint64_t>(n) * chunk_bytes, &trial);
    threads = kScatterShapes[pick][0];
    unroll = kScatterShapes[pick][1];
    if (trial) PF_HIP(hipEventRecord(trial->start, stream));
  }
  unroll &= ~PF_KERNEL_AUTO;
  const hipError_t e = issue_copy(stream, x->desc_base + first, n, chunk_bytes, al16,
                                  threads, unroll, qgrid, x->max_grid, marks, queue);
  if (e != hipSuccess) return hip_fail(e, "gather/scatter kernel launch");
  if (trial) {
    PF_HIP(hipEventRecord(trial->stop, stream));
    trial->bytes = static_cast<uint64_t>(n) * chunk_bytes;
    trial->pending = true;
  }
  if (tm) PF_HIP(hipEventRecord(tm->second, stream));
  x->last_kernels++;
  return PF_OK;
}

// A marked copy between device buffers (16-byte aligned chunks) on the
// context's stream with a fixed workgroup -> tile map: the staged load's
// scatter of a slice whose layers it marks itself.
int launch_marked_scatter(pf_xfer* x, size_t first, size_t n, uint64_t chunk_bytes,
                          const SliceMarks& m) {
  if (n == 0) return PF_OK;
  if (int rc = check_launch_size(n, chunk_bytes)) return rc;
  std::pair<hipEvent_t, hipEvent_t>* tm = nullptr;
  if (x->timing) {
    if (x->last_kernels >= x->timers.size()) {
      std::pair<hipEvent_t, hipEvent_t> p{nullptr, nullptr};
      PF_HIP(hipEventCreate(&p.first));
      PF_HIP(hipEventCreate(&p.second));
      x->timers.push_back(p);
    }
    tm = &x->timers[x->last_kernels];
    PF_HIP(hipEventRecord(tm->first, x->stream));
  }
  (void)hipGetLastError();
  const hipError_t e = launch_copy_chunks_marked(
      x->desc_base + first, static_cast<uint32_t>(n), chunk_bytes, kMarkedScatterThreads,
      marked_unroll(chunk_bytes) | PF_KERNEL_NT_LOADS, kMarkedScatterGrid, m, x->stream);
  if (e != hipSuccess) return hip_fail(e, "marked scatter kernel launch");
  if (tm) PF_HIP(hipEventRecord(tm->second, x->stream));
  x->last_kernels++;
  return PF_OK;
}

// Counters for marking launches over num_layers layers, zeroed on the
// context's stream before first use.
int ensure_counters(pf_xfer* x, size_t num_layers) {
  if (num_layers <= x->counters_cap) return PF_OK;
  size_t cap = 64;
  while (cap < num_layers) cap <<= 1;
  PF_HIP(hipStreamSynchronize(x->dma));  // earlier launches may still count
  PF_HIP(hipStreamSynchronize(x->stream));
  if (x->d_counters) PF_HIP(hipFree(x->d_counters));
  x->d_counters = nullptr;
  x->d_queue[0] = x->d_queue[1] = nullptr;
  x->counters_cap = 0;
  // cap counters, then one 256-byte line per lane holding its tile queue.
  const size_t words = cap + 128;
  PF_HIP(hipMalloc(reinterpret_cast<void**>(&x->d_counters), words * sizeof(uint32_t)));
  PF_HIP(hipMemsetAsync(x->d_counters, 0, words * sizeof(uint32_t), x->stream));
  PF_HIP(hipStreamSynchronize(x->stream));  // the link-side lane's first launch finds 0 too
  x->d_queue[0] = x->d_counters + cap;
  x->d_queue[1] = x->d_counters + cap + 64;
  x->counters_cap = cap;
  return PF_OK;
}

// Marks the given layers on the context's stream (after the work queued so far).
int mark_layers(pf_xfer* x, const std::vector<uint32_t>& ids, const SignalTargets& t,
                hipStream_t stream = nullptr) {
  if (!stream) stream = x->stream;
  for (size_t i = 0; i < ids.size(); i += kLayerListMax) {
    LayerList list{};
    list.n = static_cast<uint32_t>(std::min<size_t>(kLayerListMax, ids.size() - i));
    for (uint32_t k = 0; k < list.n; ++k) list.ids[k] = ids[i + k];
    (void)hipGetLastError();
    hipError_t e = launch_mark_layers(list, t, stream);
    if (e != hipSuccess) return hip_fail(e, "layer mark kernel launch");
  }
  return PF_OK;
}

int mark_layer(pf_xfer* x, uint32_t li, const SignalTargets* t) {
  if (!t) return PF_OK;
  return mark_layers(x, std::vector<uint32_t>{li}, *t);
}

int plan_all(const pf_layer_xfer* layers, uint32_t n, bool is_save,
             std::vector<LayerPlan>* plans) {
  plans->resize(n);
  for (uint32_t i = 0; i < n; ++i)
    if (int rc = plan_layer(layers[i], is_save, &(*plans)[i])) return rc;
  return PF_OK;
}

int check_all_kernel(const pf_layer_xfer* layers, const std::vector<LayerPlan>& plans,
                     bool host_side) {
  RangeCache rc;
  for (size_t i = 0; i < plans.size(); ++i) {
    if (plans[i].chunks.empty() || plans[i].ordered) continue;
    if (int r = check_device_tensor(rc, layers[i].layout)) return r;
    if (host_side)
      if (int r = check_host_chunks(rc, plans[i])) return r;
  }
  return PF_OK;
}

bool chunks_aligned(const LayerPlan& p) {
  if (!aligned16(p.chunk_bytes)) return false;
  for (const Chunk& c : p.chunks)
    if (!aligned16(c.dev) || !aligned16(c.host)) return false;
  return true;
}

// ---- DMA modes ------------------------------------------------------------
// The copies of one layer as DMA calls on `stream`, in list order; *issued
// counts them.
int dma_copies(hipStream_t stream, const LayerPlan& p, bool is_save, bool per_chunk_sync,
               uint64_t* issued) {
  hipError_t e = hipSuccess;
  auto issue = [&](size_t i, size_t n) {
    if (e != hipSuccess) return;
    const Chunk& c = p.chunks[i];
    const uint64_t bytes = n * p.chunk_bytes;
    if (is_save)
      e = hipMemcpyAsync(reinterpret_cast<void*>(c.host), reinterpret_cast<void*>(c.dev),
                         bytes, hipMemcpyDefault, stream);
    else
      e = hipMemcpyAsync(reinterpret_cast<void*>(c.dev), reinterpret_cast<void*>(c.host),
                         bytes, hipMemcpyDefault, stream);
    if (e == hipSuccess && per_chunk_sync) e = hipStreamSynchronize(stream);
    ++*issued;
  };
  if (per_chunk_sync) {
    // gpu_worker.rs:344-371: one synchronous copy per segment, no merging.
    for (size_t i = 0; i < p.chunks.size(); ++i) issue(i, 1);
  } else {
    for_each_run(p, 0, p.list_break, issue);
    for_each_run(p, p.list_break, p.chunks.size(), issue);
  }
  if (e != hipSuccess)
    return hip_fail(e, is_save ? "hipMemcpyDtoH" : "hipMemcpyHtoDAsync");
  return PF_OK;
}

int dma_layer(pf_xfer* x, const LayerPlan& p, bool is_save, bool per_chunk_sync) {
  return dma_copies(x->stream, p, is_save, per_chunk_sync, &x->last_dma);
}

// ---- staged mode ----------------------------------------------------------
// The host link is crossed only by DMA copies of host-contiguous runs; the
// chunk kernel moves the paged side between the layer tensors and a packed
// staging slot in HBM.  Host-memory traffic issued by shaders (the zero-copy
// kernels) holds up the memory traffic of every other kernel on the device
// while it runs: measured from another process, a bf16 8192^3 GEMM ran 29x
// slower beside a zero-copy save of the Llama prefix and 2.4x slower beside
// a zero-copy restore, against 1.03x beside this mode.
//
// A call's chunks are cut, in layer order, into slices of at most the
// direction's slice size; a slice may span layers, but not an ordered layer
// (copied in place, in list order) or a change of chunk size, and a load's
// layer ends its last slice while slices grow and once it is half full
// (StagedPlanner).  With pinned host memory and known copy engines the
// slices' copies run on the engines (staged_engine).  Otherwise consecutive
// slices alternate between the context's two lanes (its two streams), each
// lane owning one staging slot: a slice's copies and kernel run in order on
// its lane, so the lane's next slice refills the slot only once the kernel
// has read it, with no wait across streams, while the other lane's copies
// keep the link busy.  (On one stream each copy starts about 10 us after the
// previous one ends: 8 MiB copies moved 53.7 GB/s host to device on one
// stream, 57.4 GB/s alternating over two.)
// Plans layers [begin, end) of a staged call into plans[begin, end).
int plan_range(const pf_layer_xfer* layers, uint32_t begin, uint32_t end, bool is_save,
               std::vector<LayerPlan>* plans) {
  for (uint32_t li = begin; li < end; ++li) {
    if (int rc = plan_layer(layers[li], is_save, &(*plans)[li])) return rc;
    apply_write_policy(layers[li], is_save, true, &(*plans)[li]);
  }
  return PF_OK;
}

// The device tensors of layers [begin, end) that the staged kernels touch.
int check_devices(const pf_layer_xfer* layers, const std::vector<LayerPlan>& plans,
                  uint32_t begin, uint32_t end) {
  RangeCache rc;
  for (uint32_t li = begin; li < end; ++li)
    if (!plans[li].chunks.empty() && !plans[li].ordered)
      if (int r = check_device_tensor(rc, layers[li].layout)) return r;
  return PF_OK;
}

// A staged save may copy its slices out on both lanes only when no two of its
// host-side chunks overlap: the reference's in-order copies decide which
// bytes an overlap keeps, and one lane keeps that order.  Checked per layer,
// then across layers by their spans (sorting every chunk only when spans of
// different layers interleave).
bool save_hosts_disjoint(const std::vector<LayerPlan>& plans) {
  std::vector<std::pair<uint64_t, uint64_t>> spans;
  for (const LayerPlan& p : plans) {
    if (p.chunks.empty()) continue;
    if (!host_chunks_disjoint(p)) return false;
    uint64_t lo = p.chunks[0].host, hi = p.chunks[0].host;
    for (const Chunk& c : p.chunks) {
      lo = std::min(lo, c.host);
      hi = std::max(hi, c.host);
    }
    spans.push_back({lo, hi + p.chunk_bytes});
  }
  std::sort(spans.begin(), spans.end());
  bool interleaved = false;
  for (size_t i = 1; i < spans.size() && !interleaved; ++i)
    interleaved = spans[i].first < spans[i - 1].second;
  if (!interleaved) return true;
  std::vector<std::pair<uint64_t, uint64_t>> all;
  for (const LayerPlan& p : plans)
    for (const Chunk& c : p.chunks) all.push_back({c.host, c.host + p.chunk_bytes});
  std::sort(all.begin(), all.end());
  for (size_t i = 1; i < all.size(); ++i)
    if (all[i].first < all[i - 1].second) return false;
  return true;
}

// Calls fn(chunk, k) for the chunks of a staged step in order, k counting
// from 0 (the chunk's place in the slot).
template <class F>
void for_each_step_chunk(const std::vector<LayerPlan>& plans, const StagedPlan& sp,
                         const StagedStep& st, F fn) {
  size_t k = 0;
  for (size_t pi = st.piece_begin; pi < st.piece_end; ++pi) {
    const Piece& pc = sp.pieces[pi];
    const LayerPlan& p = plans[pc.layer];
    for (size_t i = pc.begin; i < pc.end; ++i) fn(p.chunks[i], k++);
  }
}

// PEGAFLOW_TRACE: microseconds from the start of a staged call to each of
// its steps (slices queued and completed, layers completed), printed as one
// line when the call ends.
struct StagedTrace {
  bool on = tracing();
  std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
  std::string line;
  void mark(const char* what, size_t i) {
    if (!on) return;
    const double us =
        std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    line += strf(" %s%zu=%.0f", what, i, us);
  }
  void print(bool is_save) {
    if (on)
      std::fprintf(stderr, "[pegaflow] staged %s at=%.0fus%s\n", is_save ? "save" : "load",
                   mono_us(t0), line.c_str());
  }
};

// Waits for every copy-engine copy the context has in flight.
int engine_drain(pf_xfer* x) {
  if (!x->engine_ok) return PF_OK;
  int rc = PF_OK;
  for (EngineSignal& s : x->eng_sig)
    if (int r = engine_signal_wait(&s)) rc = r;
  return rc;
}

// True when every host-side chunk of the staged layers [begin, end) lies in
// pinned memory (the copy engines read and write it directly); checked per
// layer by its span first.
bool hosts_pinned(const std::vector<LayerPlan>& plans, uint32_t begin, uint32_t end) {
  for (uint32_t li = begin; li < end; ++li) {
    const LayerPlan& p = plans[li];
    if (p.chunks.empty() || p.ordered) continue;
    uint64_t lo = p.chunks[0].host, hi = p.chunks[0].host;
    for (const Chunk& c : p.chunks) {
      lo = std::min(lo, c.host);
      hi = std::max(hi, c.host);
    }
    uint64_t b = 0, e = 0;
    if (hi + p.chunk_bytes >= hi && pinned_lookup(lo, hi + p.chunk_bytes - lo, &b, &e)) continue;
    for (const Chunk& c : p.chunks)
      if (!pinned_lookup(c.host, p.chunk_bytes, &b, &e)) return false;
  }
  return true;
}

// Pinned host memory, by the allocation found last.
struct PinnedCache {
  uint64_t b = 0, e = 0;
  bool covers(uint64_t a, uint64_t n) {
    if (a >= b && a + n >= a && a + n <= e) return true;
    return pinned_lookup(a, n, &b, &e);
  }
};

// The staged mode with its copies on the device's copy engines, driven from
// the calling thread.  An engine runs its copies in submission order, one
// after another, so keeping the next slice's copy queued behind the running
// one keeps the link busy: a save gathers a slice into its slot, waits for
// the gather and queues the slot's copies; a load queues the copies of the
// first slots and, as each slot's copies complete, scatters it and queues
// the copies that refill it once the scatter is done.  Every kernel runs on
// the context's stream.  A load returns once its copies are done and its
// last kernels are issued, with its layer events and marks recorded.
//
// A pipelined load (head < num_layers) has planned and sliced only its
// first `head` layers on entry.  Once their first copies are queued it takes
// the rest of its layers (pending->ready(), when they were still being
// listed), plans and slices them and uploads their descriptors while those
// copies run.  Host runs outside pinned memory are copied through HIP, each
// waited for before the next is queued.
int kernel_direct(pf_xfer* x, const pf_layer_xfer* layers, const std::vector<LayerPlan>& plans,
                  bool is_save, pf_event* layer_events, const SignalTargets* sig,
                  bool wait_save, size_t desc_off, uint32_t layer_base, size_t* used);

int staged_engine(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                  std::vector<LayerPlan>& plans, StagedPlanner& planner, StagedPlan& sp,
                  uint32_t head, bool kernel_head, bool slice_marks, const PendingLayers* pending,
                  bool is_save, pf_event* layer_events, const SignalTargets* sig,
                  bool wait_save, StagedTrace& tr) {
  const bool piped = head < num_layers;
  // Slots: as many as the staging holds of the largest slice (at least one).
  // A pipelined call's later slices are not known yet; each is at most the
  // planner's cap or one chunk (a block or a segment of its layer's layout),
  // so a load waited for layer by layer (64 MiB slices) keeps 8 slices in
  // flight in 512 MiB of staging, not 2: each slice's scatter then has time
  // to finish before its slot is needed again, also when the device's CUs
  // are busy with other work.
  uint64_t stride = 0;
  if (piped) {
    uint64_t chunk = 0;
    for (uint32_t li = 0; li < num_layers; ++li)
      chunk = std::max({chunk, layers[li].layout.block_size_bytes,
                        layers[li].layout.bytes_per_block});
    stride = std::min(x->slot_bytes, planner.max_slice_bytes(chunk));
  } else {
    for (const StagedStep& st : sp.steps)
      if (st.ordered_layer < 0) stride = std::max<uint64_t>(stride, st.n_chunks * st.chunk_bytes);
  }
  stride = (stride + 255) & ~uint64_t(255);
  size_t n_slots = 1;
  if (stride > 0)
    n_slots = static_cast<size_t>(
        std::max<uint64_t>(1, std::min<uint64_t>(kEngineSlots, 2 * x->slot_bytes / stride)));
  auto slot_base = [&](size_t j) {
    return x->staging + static_cast<uint64_t>(j % n_slots) * stride;
  };
  // Per step its slice number (SIZE_MAX: copied in place); per slice its step.
  std::vector<size_t> slice_of, slice_steps;
  auto index = [&]() {
    for (size_t si = slice_of.size(); si < sp.steps.size(); ++si) {
      if (sp.steps[si].ordered_layer >= 0) {
        slice_of.push_back(SIZE_MAX);
      } else {
        slice_of.push_back(slice_steps.size());
        slice_steps.push_back(si);
      }
    }
  };
  index();
  ChunkDesc* hd = piped ? nullptr : small_desc(x, sp.n_desc);
  if (!hd) {
    // Room for every descriptor of the call, reserved before the first part
    // is uploaded: growing the buffers later would wait for its copies.
    uint64_t bound = sp.n_desc;
    if (piped) {  // with the first layer's mark tables, when the kernel copies it
      bound = 1 + 2 * ((2ull * num_layers + 1) * sizeof(uint32_t) / sizeof(ChunkDesc) + 1);
      for (uint32_t li = 0; li < num_layers; ++li)
        bound += (pending && li >= head ? pending->max_blocks : layers[li].num_blocks) *
                 (layers[li].layout.segments ? layers[li].layout.segments : 1);
    }
    if (int rc = ensure_desc_capacity(x, static_cast<size_t>(bound))) return rc;
    hd = x->h_desc;
    // A later part's upload waits for everything the stream holds so far.
    if (piped) PF_HIP(hipEventRecord(x->parts_ready, x->stream));
  }
  // Descriptors of the steps not written yet, then uploaded (launches index
  // them from the start of the device copy).
  size_t written = 0, uploaded = 0;
  auto publish = [&]() -> int {
    for (size_t si = written; si < sp.steps.size(); ++si) {
      const StagedStep& st = sp.steps[si];
      if (st.ordered_layer >= 0) continue;
      const uint64_t slot = slot_base(slice_of[si]);
      for_each_step_chunk(plans, sp, st, [&](const Chunk& c, size_t k) {
        const uint64_t at = slot + k * st.chunk_bytes;
        hd[st.desc_first + k] = is_save ? ChunkDesc{c.dev, at} : ChunkDesc{at, c.dev};
      });
    }
    written = sp.steps.size();
    if (hd == x->h_small) {
      x->desc_base = x->h_small;
      x->small_inflight = true;
      return PF_OK;
    }
    if (sp.n_desc > uploaded) {
      if (int rc = upload_desc(x, sp.n_desc - uploaded, uploaded)) return rc;
      uploaded = sp.n_desc;
    }
    x->desc_base = x->d_desc;
    return PF_OK;
  };
  uint64_t head_bytes = 0;
  std::chrono::steady_clock::time_point head_start;
  if (kernel_head) {
    // The first layers by the zero-copy kernel (marked, with their events),
    // the slices' descriptors after the kernel's.
    std::vector<LayerPlan>& hp = x->plans_rest;
    hp.resize(head);
    for (uint32_t li = 0; li < head; ++li) std::swap(hp[li], plans[li]);
    size_t used = 0;
    for (uint32_t li = 0; li < head; ++li) head_bytes += hp[li].chunks.size() * hp[li].chunk_bytes;
    head_start = std::chrono::steady_clock::now();
    if (int rc = kernel_direct(x, layers, hp, false, layer_events, sig, false, 0, 0, &used))
      return rc;
    PF_HIP(hipEventRecord(x->head_done, x->stream));
    uploaded = std::max<size_t>(used, 1);
    planner.start_descriptors_at(uploaded);
    tr.mark("head", used);
  }
  if (int rc = publish()) return rc;
  tr.mark("desc", sp.n_desc);
  PinnedCache pinned;
  // The host-contiguous runs of a slice, each one engine copy.
  auto queue_copies = [&](size_t si) -> int {
    const StagedStep& st = sp.steps[si];
    const size_t j = slice_of[si];
    EngineSignal* es = &x->eng_sig[j % n_slots];
    const uint64_t slot = slot_base(j), cb = st.chunk_bytes;
    uint64_t run_host = 0, run_at = 0, run_bytes = 0;
    int rc = PF_OK;
    auto flush = [&]() {
      if (run_bytes == 0 || rc != PF_OK) return;
      x->last_dma++;
      if (pinned.covers(run_host, run_bytes)) {
        engine_signal_add(es, 1);
        rc = is_save ? engine_copy(x->device, true, run_host, run_at, run_bytes, es,
                                   static_cast<unsigned>(j))
                     : engine_copy(x->device, false, run_at, run_host, run_bytes, es,
                                   static_cast<unsigned>(j));
        return;
      }
      hipError_t e =
          is_save ? hipMemcpyAsync(reinterpret_cast<void*>(run_host),
                                   reinterpret_cast<void*>(run_at), run_bytes, hipMemcpyDefault,
                                   x->dma)
                  : hipMemcpyAsync(reinterpret_cast<void*>(run_at),
                                   reinterpret_cast<void*>(run_host), run_bytes, hipMemcpyDefault,
                                   x->dma);
      if (e == hipSuccess) e = hipStreamSynchronize(x->dma);
      if (e != hipSuccess)
        rc = hip_fail(e, is_save ? "staged hipMemcpyAsync (D2H)" : "staged hipMemcpyAsync (H2D)");
    };
    for_each_step_chunk(plans, sp, st, [&](const Chunk& c, size_t k) {
      if (run_bytes > 0 && c.host == run_host + run_bytes) {
        run_bytes += cb;
        return;
      }
      flush();
      run_host = c.host;
      run_at = slot + k * cb;
      run_bytes = cb;
    });
    flush();
    tr.mark("q", j);
    return rc;
  };
  // A marked load's layers are marked by the scatters of their slices where
  // every slice holding a piece of the layer can run the marking kernel
  // (16-byte aligned, at most kSliceMarkLayers layers): the layer's counter
  // adds up over those launches.  Per call layer: 1 so, 0 marked by a
  // marking kernel after its last slice, -1 not decided yet (decided at its
  // first slice, when every slice holding it is known).
  std::vector<signed char> self_marked(slice_marks ? num_layers : 0, -1);
  auto markable = [&](size_t si) {
    const StagedStep& st = sp.steps[si];
    if (st.ordered_layer >= 0 || st.piece_end - st.piece_begin > kSliceMarkLayers ||
        !aligned16(st.chunk_bytes) || !aligned16(slot_base(slice_of[si])))
      return false;
    bool al = true;
    for_each_step_chunk(plans, sp, st, [&](const Chunk& c, size_t) { al = al && aligned16(c.dev); });
    return al;
  };
  auto kernel = [&](size_t si) -> int {
    const StagedStep& st = sp.steps[si];
    const uint64_t slot = slot_base(slice_of[si]);
    bool al16 = aligned16(st.chunk_bytes) && aligned16(slot);
    for_each_step_chunk(plans, sp, st,
                        [&](const Chunk& c, size_t) { al16 = al16 && aligned16(c.dev); });
    // A slice's scatter marks the layers it completes: beside other work
    // filling every CU, each kernel of ours waits for one of that work's
    // kernels to end, so a layer lands after one such wait instead of two (a
    // scatter, then a marking kernel).
    if (slice_marks) {
      for (size_t pi = st.piece_begin; pi < st.piece_end; ++pi) {
        const uint32_t li = sp.pieces[pi].layer;
        if (self_marked[li] >= 0) continue;
        bool ok = true;  // this slice is the layer's first
        for (size_t k = si; ok && static_cast<int64_t>(k) <= sp.done_at[li]; ++k)
          ok = markable(k);
        self_marked[li] = ok ? 1 : 0;
      }
      SliceMarks m{};
      bool counts = false;
      for (size_t pi = st.piece_begin; pi < st.piece_end && m.n < kSliceMarkLayers; ++pi) {
        const Piece& pc = sp.pieces[pi];
        const LayerPlan& p = plans[pc.layer];
        m.layer[m.n] = pc.layer;
        m.chunk_start[m.n + 1] = m.chunk_start[m.n] + static_cast<uint32_t>(pc.end - pc.begin);
        if (self_marked[pc.layer] == 1) {
          const uint64_t tile = uint64_t(kMarkedScatterThreads) * marked_unroll(p.chunk_bytes);
          const uint64_t tpc = (p.chunk_bytes / 16 + tile - 1) / tile;
          m.tiles[m.n] = static_cast<uint32_t>(p.chunks.size() * tpc);
          counts = true;
        }
        ++m.n;
      }
      if (counts) {
        m.counters = x->d_counters;
        m.targets = *sig;
        return launch_marked_scatter(x, st.desc_first, st.n_chunks, st.chunk_bytes, m);
      }
    }
    return launch(x, st.desc_first, st.n_chunks, st.chunk_bytes, al16, is_save);
  };
  // Kernels of slot s done (waited for on the host).
  auto kernels_done = [&](size_t s) -> int {
    PF_HIP(hipEventRecord(x->eng_ev[s], x->stream));
    PF_HIP(hipEventSynchronize(x->eng_ev[s]));
    return PF_OK;
  };
  if (is_save) {
    auto save_step = [&](size_t si) -> int {
      if (sp.steps[si].ordered_layer >= 0)  // not produced for saves; copied in place
        return dma_layer(x, plans[static_cast<size_t>(sp.steps[si].ordered_layer)], true, false);
      const size_t s = slice_of[si] % n_slots;
      // The slot's previous copies (of this call or an earlier one) are done.
      if (int rc = engine_signal_wait(&x->eng_sig[s])) return rc;
      if (int rc = kernel(si)) return rc;
      if (int rc = kernels_done(s)) return rc;
      return queue_copies(si);
    };
    size_t si = 0;
    for (; si < sp.steps.size(); ++si)
      if (int rc = save_step(si)) return rc;
    if (piped) {
      // The first layers' copies run on the engine while the rest is
      // listed and planned.
      if (pending)
        if (int rc = pending->ready()) return rc;
      if (int rc = plan_range(layers, head, num_layers, true, &plans)) return rc;
      if (int rc = check_devices(layers, plans, head, num_layers)) return rc;
      if (int rc = planner.add(plans, head, num_layers)) return rc;
      if (int rc = planner.cut()) return rc;
      index();
      if (int rc = publish()) return rc;
      tr.mark("rest", sp.n_desc);
      for (; si < sp.steps.size(); ++si)
        if (int rc = save_step(si)) return rc;
    }
    if (wait_save) return engine_drain(x);
    return PF_OK;
  }
  // The first slots' copies; a pipelined load's other layers meanwhile.
  size_t queued = 0;
  auto queue_free_slots = [&]() -> int {
    for (; queued < slice_steps.size() && queued < n_slots; ++queued)
      if (int rc = queue_copies(slice_steps[queued])) return rc;
    return PF_OK;
  };
  if (int rc = queue_free_slots()) return rc;
  if (piped) {
    if (pending)
      if (int rc = pending->ready()) return rc;
    if (int rc = plan_range(layers, head, num_layers, false, &plans)) return rc;
    if (int rc = check_devices(layers, plans, head, num_layers)) return rc;
    if (int rc = planner.add(plans, head, num_layers)) return rc;
    if (int rc = planner.cut()) return rc;
    index();
    if (int rc = publish()) return rc;
    tr.mark("rest", sp.n_desc);
    // The copy engine starts once the kernel is done with the link, or once
    // the kernel has had the time its bytes take on the link at 40 GB/s:
    // a kernel slowed by other work holding the CUs leaves the link idle
    // (beside a GEMM the Llama prefix's first layer took 2.2 ms by the
    // kernel, and the engine waited throughout).  On an idle device the
    // kernel ends first and has the link to itself.
    if (kernel_head) {
      const auto limit = head_start + std::chrono::microseconds(100 + head_bytes / 40000);
      for (;;) {
        const hipError_t q = hipEventQuery(x->head_done);
        if (q == hipSuccess) break;
        if (q != hipErrorNotReady) return hip_fail(q, "first-layer kernel");
        if (std::chrono::steady_clock::now() >= limit) break;
        std::this_thread::yield();
      }
      tr.mark("engine", 0);
    }
    if (int rc = queue_free_slots()) return rc;
  }
  size_t next_layer = kernel_head ? head : 0;  // the kernel completes its own layers
  auto complete = [&](int64_t step) -> int {
    std::vector<uint32_t> ids;
    while (next_layer < plans.size() && sp.done_at[next_layer] == step)
      ids.push_back(static_cast<uint32_t>(next_layer++));
    if (ids.empty()) return PF_OK;
    const uint32_t last = ids.back();
    for (uint32_t li : ids)
      if (layer_events && layer_events[li])
        PF_HIP(hipEventRecord(static_cast<hipEvent_t>(layer_events[li]), x->stream));
    if (sig) {
      // Layers their slices' scatters marked are left out.
      ids.erase(std::remove_if(ids.begin(), ids.end(),
                               [&](uint32_t li) {
                                 return li < self_marked.size() && self_marked[li] == 1;
                               }),
                ids.end());
      if (!ids.empty())
        if (int rc = mark_layers(x, ids, *sig)) return rc;
    }
    tr.mark("L", last);
    return PF_OK;
  };
  if (int rc = complete(-1)) return rc;
  // A slot is refilled once its scatter is done.  Scattered slices wait for
  // that in order.  The host waits for the oldest one when the engine would
  // otherwise be left with only the copy it is running (two slots: each
  // refill must be queued while the other slot's copy runs), or when the
  // next slice to scatter has not been queued yet; with more slots in
  // flight it refills whatever scatters have ended and moves on: beside
  // other work holding every CU a scatter can wait a whole kernel of that
  // work (up to a millisecond), and the slices behind it are scattered and
  // marked meanwhile.  Slice `queued` reuses the slot of the oldest waiting
  // slice, queued - n_slots.
  std::deque<size_t> scattered;
  auto refill = [&](bool block) -> int {
    while (!scattered.empty() && queued < slice_steps.size()) {
      const size_t s = scattered.front() % n_slots;
      if (block) {
        PF_HIP(hipEventSynchronize(x->eng_ev[s]));
        block = false;
      } else {
        const hipError_t q = hipEventQuery(x->eng_ev[s]);
        if (q == hipErrorNotReady) break;
        if (q != hipSuccess) return hip_fail(q, "staged scatter");
      }
      scattered.pop_front();
      if (int rc = queue_copies(slice_steps[queued++])) return rc;
    }
    return PF_OK;
  };
  for (size_t si = 0; si < sp.steps.size(); ++si) {
    const StagedStep& st = sp.steps[si];
    if (st.ordered_layer >= 0) {
      if (int rc = dma_layer(x, plans[static_cast<size_t>(st.ordered_layer)], false, false))
        return rc;
      if (int rc = complete(static_cast<int64_t>(si))) return rc;
      continue;
    }
    const size_t j = slice_of[si], s = j % n_slots;
    while (j >= queued) {
      if (scattered.empty())  // cannot happen: slice queued - n_slots was scattered
        return fail(PF_ERR_STORAGE, "staged load: a slice's slot was never freed");
      if (int rc = refill(true)) return rc;
    }
    // The first layer's slices are waited for by polling: the interrupt
    // wake costs about 25 us, and the first layer gates its consumer.
    const bool first_layer = !kernel_head && static_cast<int64_t>(si) <= sp.done_at[0];
    if (int rc = engine_signal_wait(&x->eng_sig[s], first_layer)) return rc;
    tr.mark("c", j);
    if (int rc = kernel(si)) return rc;
    if (queued < slice_steps.size()) {
      PF_HIP(hipEventRecord(x->eng_ev[s], x->stream));
      scattered.push_back(j);
    }
    // The layers the slice completes are marked behind its scatter.
    if (int rc = complete(static_cast<int64_t>(si))) return rc;
    const bool engine_short = queued < slice_steps.size() && queued <= j + 2;
    if (int rc = refill(engine_short)) return rc;
  }
  return PF_OK;
}

uint32_t pipeline_head(const pf_layer_xfer* layers, uint32_t num_layers);

// A staged call.  `pending`: layers from pending->head on are listed once
// pending->ready() returns.
int staged(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers, bool is_save,
           pf_event* layer_events, const SignalTargets* sig, bool wait_save,
           const PendingLayers* pending) {
  if (x->staging == 0 || x->slot_bytes == 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "transfer context has no staging buffer");
  StagedTrace tr;
  std::vector<LayerPlan>& plans = x->plans;
  plans.resize(num_layers);
  // Layers planned before the first copies: all, or a pipelined call's
  // first layer (the layers listed so far, when the rest are pending).  A
  // save's first copy then starts after planning and gathering 1 of the
  // Llama prefix's 32 layers (40 MiB) instead of all 40,960 chunks and a
  // full slice, and the rest is planned under that copy.
  uint32_t head = pending ? pending->head : num_layers;
  if (!pending && x->engine_ok && pipeline_head(layers, num_layers) > 0) head = 1;
  if (int rc = plan_range(layers, 0, head, is_save, &plans)) return rc;
  const bool engines = x->engine_ok && hosts_pinned(plans, 0, head);
  if (head < num_layers && !engines) {
    if (pending)
      if (int rc = pending->ready()) return rc;
    if (int rc = plan_range(layers, head, num_layers, is_save, &plans)) return rc;
    head = num_layers;
  }
  // A pipelined load whose caller waits layer by layer (marks or per-layer
  // events) copies its first layer through the copy engines by default, as
  // one copy (the planner's first slice holds it whole) and one scatter that
  // marks it itself: beside a GEMM whose workgroups fill every CU's
  // registers, each kernel of ours waits for one of the GEMM's kernels to
  // end, so the layer lands after one such wait (the Llama prefix's first
  // layer 1.57-1.65 ms after the call, 0.93-0.98 ms idle), and the load
  // makes no shader traffic over the host link (the GEMM 1.01-1.04x slower
  // while it runs).  The context's staged_head may send the first layer by
  // the zero-copy kernel instead (1.50-1.58 ms beside that GEMM, 0.94-1.02
  // ms idle, the GEMM 1.04-1.06x).  A load completed as a whole stays staged
  // throughout.
  const bool kernel_head = x->staged_head == PF_STAGED_HEAD_KERNEL && engines && !is_save &&
                           head > 0 && head < num_layers &&
                           (sig != nullptr || layer_events != nullptr);
  // A load waited for layer by layer (marks or per-layer events) keeps its
  // slices at most kLayeredLoadSlice, so each Llama layer (40 MiB) is a copy
  // of its own and lands on its own; larger slices would join 3-4 layers in
  // one copy.  Other calls take the context's slice sizes.
  uint64_t slice = x->staged_slice[is_save ? 0 : 1];
  if (!is_save && (sig || layer_events)) slice = std::min(slice, kLayeredLoadSlice);
  StagedPlan sp;
  StagedPlanner planner(x->slot_bytes, slice, is_save, num_layers, &sp);
  if (!is_save && (sig || layer_events) && !kernel_head) {
    for (uint32_t li = 0; li < head; ++li)
      if (!plans[li].ordered && !plans[li].chunks.empty()) {
        planner.start_with_layer(plans[li].chunks.size() * plans[li].chunk_bytes);
        break;
      }
  }
  // A marked load through the copy engines marks the layers a slice holds
  // whole from inside that slice's scatter.
  const bool slice_marks = !is_save && sig && engines;
  if (!kernel_head) {
    if (int rc = planner.add(plans, 0, head)) return rc;
    if (int rc = planner.cut()) return rc;
  }
  if (int rc = check_devices(layers, plans, 0, head)) return rc;
  // Nothing of an earlier staged call may still use the slots.
  if (int rc = engine_drain(x)) return rc;
  if (engines) {
    if (int rc = ensure_counters(x, num_layers)) return rc;  // queued device routes
    PF_HIP(hipEventSynchronize(x->staging_free));
    tr.mark("start", sp.steps.size());
    int rc = staged_engine(x, layers, num_layers, plans, planner, sp, head, kernel_head,
                           slice_marks, pending, is_save, layer_events, sig, wait_save, tr);
    // A layer's tile counter adds up over the scatters of its slices; a call
    // that stopped between two of them leaves counts behind.  Once its
    // kernels have ended they are cleared, so the next marked call starts
    // from 0.
    if (rc != PF_OK && slice_marks) {
      const hipError_t e1 = hipStreamSynchronize(x->stream);
      const hipError_t e2 =
          e1 == hipSuccess ? hipMemset(x->d_counters, 0, num_layers * sizeof(uint32_t)) : e1;
      if (e2 != hipSuccess) (void)hipGetLastError();
    }
    PF_HIP(hipEventRecord(x->staging_free, x->stream));
    tr.print(is_save);
    return rc;
  }
  // One lane when a save's order matters (host regions that overlap must
  // be written in list order); otherwise slices alternate between the two
  // streams, each with a tile queue of its own for queued launches.
  const int lanes = (is_save && !save_hosts_disjoint(plans)) ? 1 : 2;
  hipStream_t lane_s[2] = {x->stream, x->dma};
  {
    int k = 0;
    for (StagedStep& st : sp.steps)
      st.lane = st.ordered_layer >= 0 ? 0 : (k++ % lanes);
  }
  if (int rc = ensure_counters(x, plans.size())) return rc;  // queued device routes
  ChunkDesc* hd = small_desc(x, sp.n_desc);
  if (!hd) {
    if (int rc = ensure_desc_capacity(x, sp.n_desc)) return rc;
    hd = x->h_desc;
  }
  for (const StagedStep& st : sp.steps) {
    if (st.ordered_layer >= 0) continue;
    const uint64_t slot = x->staging + static_cast<uint64_t>(st.lane) * x->slot_bytes;
    for_each_step_chunk(plans, sp, st, [&](const Chunk& c, size_t k) {
      const uint64_t at = slot + k * st.chunk_bytes;
      hd[st.desc_first + k] = is_save ? ChunkDesc{c.dev, at} : ChunkDesc{at, c.dev};
    });
  }
  if (hd == x->h_small) {
    x->desc_base = x->h_small;
    x->small_inflight = true;
  } else if (int rc = upload_desc(x, sp.n_desc)) {
    return rc;
  }
  // lane_open[l]: lane l has work the other lane has not waited for.
  bool lane_open[2] = {false, false};
  auto join = [&](int to, int from) -> int {
    if (!lane_open[from]) return PF_OK;
    PF_HIP(hipEventRecord(x->lane_mark[from], lane_s[from]));
    PF_HIP(hipStreamWaitEvent(lane_s[to], x->lane_mark[from], 0));
    lane_open[from] = false;
    return PF_OK;
  };
  // Lane 1 starts after the descriptors are uploaded and after everything
  // earlier calls left on the context's stream.
  lane_open[0] = true;
  if (lanes == 2)
    if (int rc = join(1, 0)) return rc;
  lane_open[0] = false;
  // Load completion of the layers done after step s (s = -1: before any), on
  // lane `to`: once every step so far is done, then in layer order.
  size_t next_layer = 0;
  auto complete = [&](int64_t s, int to) -> int {
    if (is_save) return PF_OK;
    std::vector<uint32_t> ids;
    while (next_layer < plans.size() && sp.done_at[next_layer] == s)
      ids.push_back(static_cast<uint32_t>(next_layer++));
    if (ids.empty()) return PF_OK;
    if (int rc = join(to, 1 - to)) return rc;
    for (uint32_t li : ids)
      if (layer_events && layer_events[li])
        PF_HIP(hipEventRecord(static_cast<hipEvent_t>(layer_events[li]), lane_s[to]));
    if (sig)
      if (int rc = mark_layers(x, ids, *sig, lane_s[to])) return rc;
    // A later layer's completion on the other lane comes after these.
    lane_open[to] = true;
    return PF_OK;
  };
  if (int rc = complete(-1, 0)) return rc;
  hipError_t e = hipSuccess;
  for (size_t si = 0; si < sp.steps.size(); ++si) {
    const StagedStep& st = sp.steps[si];
    const int L = st.lane;
    if (st.ordered_layer >= 0) {
      // In place, after everything before it, and before anything after it.
      if (int rc = join(0, 1)) return rc;
      if (int rc = dma_layer(x, plans[static_cast<size_t>(st.ordered_layer)], is_save, false))
        return rc;
      lane_open[0] = true;
      if (lanes == 2)
        if (int rc = join(1, 0)) return rc;
    } else {
      const uint64_t slot = x->staging + static_cast<uint64_t>(L) * x->slot_bytes;
      const uint64_t cb = st.chunk_bytes;
      bool al16 = aligned16(cb) && aligned16(slot);
      for_each_step_chunk(plans, sp, st,
                          [&](const Chunk& c, size_t) { al16 = al16 && aligned16(c.dev); });
      // The host-contiguous runs of the step, each one DMA copy to or from
      // its place in the slot.
      auto copy_runs = [&]() {
        uint64_t run_host = 0, run_at = 0, run_bytes = 0;
        auto flush = [&]() {
          if (run_bytes == 0 || e != hipSuccess) return;
          if (is_save)
            e = hipMemcpyAsync(reinterpret_cast<void*>(run_host),
                               reinterpret_cast<void*>(run_at), run_bytes, hipMemcpyDefault,
                               lane_s[L]);
          else
            e = hipMemcpyAsync(reinterpret_cast<void*>(run_at),
                               reinterpret_cast<void*>(run_host), run_bytes, hipMemcpyDefault,
                               lane_s[L]);
          x->last_dma++;
        };
        for_each_step_chunk(plans, sp, st, [&](const Chunk& c, size_t k) {
          if (run_bytes > 0 && c.host == run_host + run_bytes) {
            run_bytes += cb;
            return;
          }
          flush();
          run_host = c.host;
          run_at = slot + k * cb;
          run_bytes = cb;
        });
        flush();
      };
      if (is_save) {
        if (int rc = launch(x, st.desc_first, st.n_chunks, cb, al16, true, false, nullptr,
                            lane_s[L]))
          return rc;
        copy_runs();
        if (e != hipSuccess) return hip_fail(e, "staged hipMemcpyAsync (D2H)");
      } else {
        copy_runs();
        if (e != hipSuccess) return hip_fail(e, "staged hipMemcpyAsync (H2D)");
        if (int rc = launch(x, st.desc_first, st.n_chunks, cb, al16, false, false, nullptr,
                            lane_s[L]))
          return rc;
      }
      lane_open[L] = true;
    }
    if (int rc = complete(static_cast<int64_t>(si), L)) return rc;
  }
  if (is_save && wait_save) {
    PF_HIP(hipStreamSynchronize(x->dma));
    PF_HIP(hipStreamSynchronize(x->stream));
    return PF_OK;
  }
  // The context's stream ends after all of the call's work.
  if (int rc = join(0, 1)) return rc;
  PF_HIP(hipEventRecord(x->staging_free, x->stream));
  return PF_OK;
}

// True when the host side of a layer's chunks lies in pinned host memory
// (judged by the first chunk): a zero-copy transfer over the host link.
bool host_side_pinned(const LayerPlan& p) {
  uint64_t b = 0, e = 0;
  return !p.chunks.empty() && pinned_lookup(p.chunks[0].host, p.chunk_bytes, &b, &e);
}

bool host_sourced(const LayerPlan& p, bool is_save) { return !is_save && host_side_pinned(p); }

// ---- kernel mode ----------------------------------------------------------
// One step of a kernel-mode call: a DMA copy of an ordered layer, or one
// launch over the consecutive layers [li, lj).
struct Step {
  size_t li, lj;
  bool dma;
  bool aligned;
  size_t tab = 0;      // marked launch: u32 offset of its table in the aux area
  uint32_t groups = 0; // marked launch: non-empty layers in it
};

// desc_off > 0: a later part of one pipelined call.  Its descriptors go
// after the earlier parts' (whose copies may still read theirs), in room
// the caller has reserved, and never in place.  layer_base: the call-wide
// index of plans[0] (marks and their counters are per call-wide layer).
// *used (if given): the descriptor slots of d_desc from desc_off on that
// this call's launches read (chunks, then the marks' tables), 0 when they
// read in place.
int kernel_direct(pf_xfer* x, const pf_layer_xfer* layers, const std::vector<LayerPlan>& plans,
                  bool is_save, pf_event* layer_events, const SignalTargets* sig,
                  bool wait_save, size_t desc_off = 0, uint32_t layer_base = 0,
                  size_t* used = nullptr) {
  if (used) *used = 0;
  if (int rc = check_all_kernel(layers, plans, true)) return rc;
  size_t total = 0;
  std::vector<size_t> first(plans.size());
  for (size_t li = 0; li < plans.size(); ++li) {
    first[li] = total;
    if (!plans[li].ordered) total += plans[li].chunks.size();
  }
  // Without per-layer events, consecutive layers with the same chunk size and
  // alignment share one launch (marks keep per-layer completion inside it).
  std::vector<Step> steps;
  std::vector<uint32_t> aux;  // marked launches: chunk_start[n+1], then layer[n]
  for (size_t li = 0; li < plans.size();) {
    const LayerPlan& p = plans[li];
    if (p.ordered) {
      steps.push_back({li, li + 1, true, false});
      ++li;
      continue;
    }
    const bool al = chunks_aligned(p);
    // Marks inside the launch cost nothing while the host link is the bound
    // (sources in pinned memory) but slow an HBM-bound launch; loads from
    // device memory are split per layer and marked after each launch.
    const bool host_src = !p.chunks.empty() && host_sourced(p, is_save);
    const bool per_layer = layer_events || (sig && !p.chunks.empty() && !host_src);
    size_t lj = li + 1;
    if (!per_layer) {
      while (lj < plans.size() && !plans[lj].ordered &&
             plans[lj].chunk_bytes == p.chunk_bytes &&
             (plans[lj].chunks.empty() || (chunks_aligned(plans[lj]) == al &&
                                           (!sig || host_sourced(plans[lj], is_save)))))
        ++lj;
    }
    Step st{li, lj, false, al};
    if (sig && al && !per_layer) {
      st.tab = aux.size();
      uint32_t start = 0;
      std::vector<uint32_t> ids;
      for (size_t k = li; k < lj; ++k) {
        if (plans[k].chunks.empty()) continue;
        aux.push_back(start);
        ids.push_back(static_cast<uint32_t>(layer_base + k));
        start += static_cast<uint32_t>(plans[k].chunks.size());
      }
      aux.push_back(start);
      aux.insert(aux.end(), ids.begin(), ids.end());
      st.groups = static_cast<uint32_t>(ids.size());
    }
    steps.push_back(st);
    li = lj;
  }
  if (total > 0xffffffffull) return fail(PF_ERR_INVALID_ARGUMENT, "too many chunks");
  const size_t aux_desc = (aux.size() * sizeof(uint32_t) + sizeof(ChunkDesc) - 1) /
                          sizeof(ChunkDesc);
  // Counters for marks and the tile queue of queued launches.
  if (int rc = ensure_counters(x, layer_base + plans.size())) return rc;
  ChunkDesc* hd = desc_off ? nullptr : small_desc(x, total + aux_desc);
  if (desc_off) {
    if (desc_off + total + aux_desc > x->h_cap || desc_off + total + aux_desc > x->d_cap)
      return fail(PF_ERR_INVALID_ARGUMENT, "descriptor room not reserved");
    hd = x->h_desc + desc_off;
  } else if (!hd) {
    if (int rc = ensure_desc_capacity(x, total + aux_desc)) return rc;
    hd = x->h_desc;
  }
  size_t d = 0;
  for (size_t li = 0; li < plans.size(); ++li) {
    if (plans[li].ordered) continue;
    for (const Chunk& c : plans[li].chunks)
      hd[d++] = is_save ? ChunkDesc{c.dev, c.host} : ChunkDesc{c.host, c.dev};
  }
  if (!aux.empty()) std::memcpy(hd + total, aux.data(), aux.size() * sizeof(uint32_t));
  if (hd == x->h_small) {
    // Read in place by the launches below; the next in-place call waits for
    // the stream to drain.
    x->desc_base = x->h_small;
    x->small_inflight = true;
  } else {
    if (int rc = upload_desc(x, total + aux_desc, desc_off)) return rc;
    if (used) *used = total + aux_desc;
  }
  const uint32_t* d_aux = reinterpret_cast<const uint32_t*>(x->desc_base + total);
  for (const Step& st : steps) {
    if (st.dma) {
      if (int rc = dma_layer(x, plans[st.li], is_save, false)) return rc;
      if (layer_events && layer_events[st.li])
        PF_HIP(hipEventRecord(static_cast<hipEvent_t>(layer_events[st.li]), x->stream));
      if (int rc = mark_layer(x, static_cast<uint32_t>(layer_base + st.li), sig)) return rc;
      continue;
    }
    size_t n = 0;
    for (size_t k = st.li; k < st.lj; ++k) n += plans[k].chunks.size();
    LayerMarks marks{};
    const bool marked = st.groups > 0;
    if (marked) {
      marks.chunk_start = d_aux + st.tab;
      marks.layer = d_aux + st.tab + st.groups + 1;
      marks.n = st.groups;
      marks.counters = x->d_counters;
      marks.targets = *sig;
    }
    // The launch shape follows the first non-empty layer's host side.
    bool host_side = false;
    for (size_t k = st.li; k < st.lj; ++k)
      if (!plans[k].chunks.empty()) {
        host_side = host_side_pinned(plans[k]);
        break;
      }
    if (int rc = launch(x, first[st.li], n, plans[st.li].chunk_bytes, st.aligned, is_save,
                        host_side, marked ? &marks : nullptr))
      return rc;
    if (layer_events && layer_events[st.li])
      PF_HIP(hipEventRecord(static_cast<hipEvent_t>(layer_events[st.li]), x->stream));
    if (sig) {
      // Layers the launch did not mark: empty ones, and all of an unaligned launch.
      std::vector<uint32_t> rest;
      for (size_t k = st.li; k < st.lj; ++k)
        if (!marked || plans[k].chunks.empty())
          rest.push_back(static_cast<uint32_t>(layer_base + k));
      if (int rc = mark_layers(x, rest, *sig)) return rc;
    }
  }
  if (is_save && wait_save) PF_HIP(hipStreamSynchronize(x->stream));
  return PF_OK;
}

// Layers in the first part of a pipelined call, or 0 for a call issued
// whole.  Copies over the host link of at least 8 layers and
// kPipelineMinChunks chunks (of the order of the chunk counts whose planning
// takes ~0.1 ms) start with an eighth of their layers: that part's copy
// (2.9 ms for a Llama prefix, 0.37 ms for one tensor-parallel rank's) hides
// the planning of the rest, and one more launch boundary costs under 1%.
// Copies between device buffers, HBM-bound at about 0.05 ms for such a
// first part, are issued whole, as one launch.
constexpr uint64_t kPipelineMinChunks = 16384;

}  // namespace

uint32_t pf::pipeline_head_layers(uint32_t num_layers, uint64_t chunks) {
  return num_layers < 8 || chunks < kPipelineMinChunks ? 0 : num_layers / 8;
}

namespace {

uint32_t pipeline_head(const pf_layer_xfer* layers, uint32_t num_layers) {
  if (num_layers < 8) return 0;
  uint64_t chunks = 0;
  const pf_block_xfer* first = nullptr;
  for (uint32_t i = 0; i < num_layers; ++i) {
    chunks += layers[i].num_blocks * (layers[i].layout.segments ? layers[i].layout.segments : 1);
    if (!first && layers[i].num_blocks > 0 && layers[i].blocks) first = layers[i].blocks;
  }
  uint64_t b = 0, e = 0;
  if (!first || !pinned_lookup(first->k_host, 1, &b, &e)) return 0;
  return pipeline_head_layers(num_layers, chunks);
}

// pending: the layers from `head` on are filled in by pending->ready(),
// called once the first part is issued.
int kernel_pipelined(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                     uint32_t head, bool is_save, bool wait_save, const SignalTargets* sig,
                     pf_event* layer_events, const PendingLayers* pending = nullptr) {
  std::vector<LayerPlan>& first = x->plans;
  std::vector<LayerPlan>& rest = x->plans_rest;
  if (int rc = plan_all(layers, head, is_save, &first)) return rc;
  for (uint32_t li = 0; li < head; ++li)
    apply_write_policy(layers[li], is_save, false, &first[li]);
  // Room for every descriptor of the call and both parts' mark tables
  // (at most 2L+1 words each), reserved before the first part is uploaded:
  // growing the buffers later would wait for the first copy.
  uint64_t bound = 1 + 2 * ((2ull * num_layers + 1) * sizeof(uint32_t) / sizeof(ChunkDesc) + 1);
  for (uint32_t i = 0; i < num_layers; ++i)
    bound += (pending && i >= head ? pending->max_blocks : layers[i].num_blocks) *
             (layers[i].layout.segments ? layers[i].layout.segments : 1);
  if (int rc = ensure_desc_capacity(x, static_cast<size_t>(bound))) return rc;
  if (int rc = ensure_counters(x, num_layers)) return rc;  // marks of both parts
  PF_HIP(hipEventRecord(x->parts_ready, x->stream));
  // The second part's descriptors go after everything the first part's
  // launches read: its chunks and its mark tables.
  size_t n_first = 0;
  if (int rc = kernel_direct(x, layers, first, is_save, layer_events, sig, false, 0, 0,
                             &n_first))
    return rc;
  if (pending)
    if (int rc = pending->ready()) return rc;
  int rc = plan_all(layers + head, num_layers - head, is_save, &rest);
  if (rc == PF_OK) {
    for (uint32_t li = head; li < num_layers; ++li)
      apply_write_policy(layers[li], is_save, false, &rest[li - head]);
    // The first part may have read its descriptors in place (h_small); the
    // second always uploads, after the first part's.
    rc = kernel_direct(x, layers + head, rest, is_save, layer_events ? layer_events + head : nullptr,
                       sig, wait_save, n_first > 0 ? n_first : 1, head);
  }
  return rc;  // on an error, run() drains both streams (copies and the upload)
}

int run_locked(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers, uint32_t mode,
               bool is_save, pf_event* layer_events, bool wait_save, const SignalTargets* sig,
               const PendingLayers* pending);

// One transfer call.  A call that fails part-way returns with none of its
// copies in flight, so the caller may reuse or free the buffers at once.
int run(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers, uint32_t mode,
        bool is_save, pf_event* layer_events, bool wait_save = true,
        const SignalTargets* sig = nullptr, const PendingLayers* pending = nullptr) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  if (num_layers > 0 && !layers) return fail(PF_ERR_INVALID_ARGUMENT, "null layer list");
  std::lock_guard<std::mutex> lk(x->mu);
  x->last_kernels = 0;
  x->last_dma = 0;
  PF_HIP(hipSetDevice(x->device));
  const int rc =
      run_locked(x, layers, num_layers, mode, is_save, layer_events, wait_save, sig, pending);
  if (rc != PF_OK) {
    (void)hipStreamSynchronize(x->dma);
    (void)hipStreamSynchronize(x->stream);
    const std::string msg = pf_last_error();
    (void)engine_drain(x);
    (void)fail(rc, msg);  // the call's own error
  }
  return rc;
}

// PF_MODE_AUTO: the staged mode when the context has staging and the host
// side's contiguous runs (in list order, as the staged mode copies them)
// average at least kAutoMinRunBytes, else the kernel mode.  A DMA copy costs
// about 10 us to issue and start, so 1 MiB runs (18 us on the link) keep the
// link busy from the context's two streams; a restore of blocks saved
// together (one host region per layer and segment) is one run per region.
constexpr uint64_t kAutoMinRunBytes = 1ull << 20;

uint32_t auto_mode(const pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers) {
  if (x->staging == 0 || x->slot_bytes == 0) return PF_MODE_KERNEL;
  uint64_t bytes = 0, runs = 0;
  for (uint32_t li = 0; li < num_layers; ++li) {
    const pf_layer_xfer& lx = layers[li];
    if (lx.num_blocks == 0 || !lx.blocks) continue;
    const pf_kv_layout& l = lx.layout;
    const bool split = layout_kind(l) == PF_LAYOUT_SPLIT;
    const uint64_t seg = l.bytes_per_block;
    const uint64_t step = split ? seg : l.block_size_bytes;
    if (step == 0 || step > x->slot_bytes) return PF_MODE_KERNEL;
    const pf_block_xfer* b = lx.blocks;
    runs += 1;
    for (uint64_t j = 1; j < lx.num_blocks; ++j)
      if (b[j].k_host != b[j - 1].k_host + step) ++runs;
    bytes += lx.num_blocks * step;
    if (split) {
      auto v = [&](uint64_t j) { return b[j].v_host ? b[j].v_host : b[j].k_host + seg; };
      runs += 1;
      for (uint64_t j = 1; j < lx.num_blocks; ++j)
        if (v(j) != v(j - 1) + seg) ++runs;
      bytes += lx.num_blocks * seg;
    }
  }
  return runs > 0 && bytes / runs >= kAutoMinRunBytes ? PF_MODE_STAGED : PF_MODE_KERNEL;
}

}  // namespace

uint32_t pf::resolve_mode(const pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                          uint32_t mode) {
  return mode == PF_MODE_AUTO ? auto_mode(x, layers, num_layers) : mode;
}

namespace {

int run_locked(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers, uint32_t mode,
               bool is_save, pf_event* layer_events, bool wait_save, const SignalTargets* sig,
               const PendingLayers* pending) {
  std::vector<LayerPlan>& plans = x->plans;
  if (mode == PF_MODE_AUTO) mode = auto_mode(x, layers, num_layers);
  if (mode == PF_MODE_KERNEL) {
    // A large call: its first layers are planned and launched before the
    // rest are planned, so the planning of the rest (about 3 ns a chunk)
    // overlaps their copy.  Marks carry call-wide layer indices; per-layer
    // events stay with their layers.
    const uint32_t head = pending ? pending->head : pipeline_head(layers, num_layers);
    if (head > 0 && head < num_layers)
      return kernel_pipelined(x, layers, num_layers, head, is_save, wait_save,
                              is_save ? nullptr : sig, is_save ? nullptr : layer_events,
                              pending);
  }
  if (mode == PF_MODE_STAGED)
    return staged(x, layers, num_layers, is_save, layer_events, sig, wait_save, pending);
  if (pending)
    if (int rc = pending->ready()) return rc;
  if (int rc = plan_all(layers, num_layers, is_save, &plans)) return rc;
  switch (mode) {
    case PF_MODE_DMA_REFERENCE:
    case PF_MODE_DMA_BATCHED: {
      const bool per_chunk_sync = is_save && mode == PF_MODE_DMA_REFERENCE;
      for (uint32_t li = 0; li < num_layers; ++li) {
        if (int rc = dma_layer(x, plans[li], is_save, per_chunk_sync)) return rc;
        if (!is_save && layer_events && layer_events[li])
          PF_HIP(hipEventRecord(static_cast<hipEvent_t>(layer_events[li]), x->stream));
        if (!is_save)
          if (int rc = mark_layer(x, li, sig)) return rc;
      }
      if (is_save && wait_save) PF_HIP(hipStreamSynchronize(x->stream));
      return PF_OK;
    }
    case PF_MODE_KERNEL:
      for (uint32_t li = 0; li < num_layers; ++li)
        apply_write_policy(layers[li], is_save, false, &plans[li]);
      return kernel_direct(x, layers, plans, is_save, layer_events, is_save ? nullptr : sig,
                           wait_save);
    default:
      return fail(PF_ERR_INVALID_ARGUMENT, strf("unknown transfer mode %u", mode));
  }
}

// A marked load's signal targets, checked: 1..PF_MAX_LAYER_SIGNALS of them,
// each with num_layers words the device may write.
int signal_targets(const pf_layer_signal* signals, uint32_t num_signals, uint32_t num_layers,
                   SignalTargets* out) {
  if (num_signals == 0 || num_signals > PF_MAX_LAYER_SIGNALS || !signals)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("a marked load takes 1..%d signal targets, got %u", PF_MAX_LAYER_SIGNALS,
                     num_signals));
  SignalTargets& t = *out;
  RangeCache rc;
  for (uint32_t i = 0; i < num_signals; ++i) {
    const pf_layer_signal& g = signals[i];
    if (g.value == 0 || g.reserved != 0 || g.host_memory > 1 || (g.words & 7u) != 0)
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("signal target %u: words must be 8-byte aligned, value nonzero, "
                       "host_memory 0 or 1",
                       i));
    // The kernels write these words: they must be mapped for the device.
    if (num_layers > 0 && !rc.check(g.words, static_cast<uint64_t>(num_layers) * 8u))
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("signal target %u: [0x%llx, +%llu) is not inside one device, IPC or "
                       "pinned allocation",
                       i, (unsigned long long)g.words,
                       (unsigned long long)num_layers * 8ull));
    t.words[i] = g.words;
    t.value[i] = g.value;
    // Words in pinned host memory get system-scope stores even when the
    // caller did not say so: the host has to see them.
    uint64_t pb = 0, pe = 0;
    if (g.host_memory || (num_layers > 0 && pinned_lookup(g.words, 8, &pb, &pe)))
      t.host_mask |= 1u << i;
  }
  t.count = num_signals;
  return PF_OK;
}

}  // namespace

int pf::save_layers_begin(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                          uint32_t mode) {
  return run(x, layers, num_layers, mode, true, nullptr, false);
}

int pf::mark_all_layers(pf_xfer* x, const pf_layer_signal& g, uint32_t num_layers) {
  if (!x || num_layers == 0) return PF_OK;
  RangeCache rc;
  if (g.value == 0 || (g.words & 7u) != 0 ||
      !rc.check(g.words, static_cast<uint64_t>(num_layers) * 8u))
    return fail(PF_ERR_INVALID_ARGUMENT, "layer words are not inside one allocation");
  SignalTargets t{};
  t.words[0] = g.words;
  t.value[0] = g.value;
  t.host_mask = g.host_memory ? 1u : 0u;
  t.count = 1;
  std::vector<uint32_t> ids(num_layers);
  for (uint32_t i = 0; i < num_layers; ++i) ids[i] = i;
  std::lock_guard<std::mutex> lk(x->mu);
  PF_HIP(hipSetDevice(x->device));
  if (int r = mark_layers(x, ids, t)) return r;
  PF_HIP(hipStreamSynchronize(x->stream));
  return PF_OK;
}

extern "C" {

// ---------------------------------------------------------------------------
// transfer.rs primitives.
// ---------------------------------------------------------------------------
int pf_copy_gpu_to_cpu(uint64_t gpu_base, uint64_t offset, void* cpu_buffer,
                       uint64_t cpu_buffer_len, uint64_t size) {
  if (!cpu_buffer && size > 0) return fail(PF_ERR_INVALID_ARGUMENT, "null CPU buffer");
  if (cpu_buffer_len < size)
    return fail(PF_ERR_STORAGE, strf("CPU buffer too small: %llu bytes, need %llu bytes",
                                     (unsigned long long)cpu_buffer_len,
                                     (unsigned long long)size));
  hipError_t e = hipMemcpy(cpu_buffer, reinterpret_cast<void*>(gpu_base + offset), size,
                           hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyDtoH");
  return PF_OK;
}

int pf_copy_cpu_to_gpu_async(uint64_t gpu_base, uint64_t offset, const void* cpu_buffer,
                             uint64_t cpu_buffer_len, uint64_t size, pf_stream stream) {
  if (!cpu_buffer && size > 0) return fail(PF_ERR_INVALID_ARGUMENT, "null CPU buffer");
  if (cpu_buffer_len < size)
    return fail(PF_ERR_STORAGE, strf("CPU buffer too small: %llu bytes, need %llu bytes",
                                     (unsigned long long)cpu_buffer_len,
                                     (unsigned long long)size));
  hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(gpu_base + offset), cpu_buffer, size,
                                hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyHtoDAsync");
  return PF_OK;
}

int pf_batch_copy_segments_to_gpu(const uint64_t* gpu_offsets, const uint64_t* cpu_ptrs,
                                  uint64_t count, uint64_t segment_size,
                                  const pf_kv_layout* layout, pf_stream stream,
                                  uint64_t* out_batches) {
  if (out_batches) *out_batches = 0;
  if (!layout) return fail(PF_ERR_INVALID_ARGUMENT, "null layout");
  if (count > 0 && (!gpu_offsets || !cpu_ptrs))
    return fail(PF_ERR_INVALID_ARGUMENT, "null transfer list");
  uint64_t batches = 0;
  uint64_t i = 0;
  while (i < count) {
    uint64_t n = 1;
    while (i + n < count && gpu_offsets[i + n] == gpu_offsets[i] + n * segment_size &&
           cpu_ptrs[i + n] == cpu_ptrs[i] + n * segment_size)
      ++n;
    uint64_t total = 0;
    if (__builtin_mul_overflow(segment_size, n, &total))
      return fail(PF_ERR_STORAGE, "batch_copy_segments_to_gpu: total_size overflow");
    int rc = pf_copy_cpu_to_gpu_async(layout->data_ptr, gpu_offsets[i],
                                      reinterpret_cast<const void*>(cpu_ptrs[i]), total,
                                      total, stream);
    // Copies already issued stay queued on the stream, as in the reference.
    if (out_batches) *out_batches = batches;
    if (rc) return rc;
    ++batches;
    i += n;
  }
  if (out_batches) *out_batches = batches;
  return PF_OK;
}

int pf_copy_block_gpu_to_cpu(const pf_kv_layout* layout, uint64_t block_idx, void* dst) {
  if (!layout) return fail(PF_ERR_INVALID_ARGUMENT, "null layout");
  if (!dst) return fail(PF_ERR_INVALID_ARGUMENT, "null destination");
  uint64_t off = 0;
  const pf_kv_layout& l = *layout;
  if (pf_is_contiguous_layout(layout)) {
    if (int rc = segment_offset(l, block_idx, 0, &off)) return rc;
    // The reference bounds only the first segment here (transfer.rs:206-208)
    // and would read past the tensor for a whole block that does not fit.
    uint64_t end = 0;
    if (__builtin_add_overflow(off, l.block_size_bytes, &end) || end > l.size_bytes)
      return fail(PF_ERR_STORAGE,
                  strf("Block %llu exceeds registered memory (offset %llu, size %llu, "
                       "limit %llu)",
                       (unsigned long long)block_idx, (unsigned long long)off,
                       (unsigned long long)l.block_size_bytes,
                       (unsigned long long)l.size_bytes));
    return pf_copy_gpu_to_cpu(l.data_ptr, off, dst, l.block_size_bytes, l.block_size_bytes);
  }
  for (uint64_t s = 0; s < l.segments; ++s) {
    if (int rc = segment_offset(l, block_idx, s, &off)) return rc;
    uint8_t* d = static_cast<uint8_t*>(dst) + s * l.bytes_per_block;
    if (int rc = pf_copy_gpu_to_cpu(l.data_ptr, off, d, l.bytes_per_block, l.bytes_per_block))
      return rc;
  }
  return PF_OK;
}

// ---------------------------------------------------------------------------
// Loads that allocate nothing: the plan of pf_load_layers in PF_MODE_KERNEL,
// with its descriptors and tile queue in the library's static device scratch
// (pf_runtime.cpp) and its work on the caller's stream.
// ---------------------------------------------------------------------------
int pf_load_layers_noalloc(pf_stream stream, const pf_layer_xfer* layers, uint32_t num_layers) {
  if (num_layers > 0 && !layers) return fail(PF_ERR_INVALID_ARGUMENT, "null layer list");
  // Chunks the call plans (duplicates included): two per block of a split
  // layer, one per block otherwise.  Checked before planning, so nothing is
  // issued and the planning buffers below stay bounded.
  uint64_t planned = 0;
  for (uint32_t i = 0; i < num_layers; ++i)
    planned += layers[i].num_blocks * (layout_kind(layers[i].layout) == PF_LAYOUT_SPLIT ? 2 : 1);
  if (planned > PF_NOALLOC_MAX_CHUNKS)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("pf_load_layers_noalloc: %llu chunks exceed the %u-chunk scratch",
                     (unsigned long long)planned, (unsigned)PF_NOALLOC_MAX_CHUNKS));
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Not under graph capture: the scratch holds whatever descriptors the last
  // call on the device left, so a replayed graph would copy another call's
  // blocks.  Refused before anything is issued.
  hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
  PF_HIP(hipStreamIsCapturing(s, &capturing));
  if (capturing != hipStreamCaptureStatusNone)
    return fail(PF_ERR_UNSUPPORTED,
                "pf_load_layers_noalloc: the stream is capturing a graph; the shared "
                "scratch cannot hold a captured call's descriptors");
  int dev = 0;
  if (s) PF_HIP(hipStreamGetDevice(s, &dev));
  else PF_HIP(hipGetDevice(&dev));
  NoAllocScratch* sc = nullptr;
  if (int rc = noalloc_scratch(dev, &sc)) return rc;
  // Host-side planning buffers, kept by the thread for its later calls.
  thread_local std::vector<LayerPlan> plans;
  thread_local std::vector<ChunkDesc> descs;
  if (plans.size() < num_layers) plans.resize(num_layers);
  size_t total = 0;
  RangeCache ranges;
  for (uint32_t i = 0; i < num_layers; ++i) {
    LayerPlan& p = plans[i];
    if (int rc = plan_layer(layers[i], false, &p)) return rc;
    apply_write_policy(layers[i], false, false, &p);
    if (p.chunks.empty() || p.ordered) continue;
    if (int rc = check_device_tensor(ranges, layers[i].layout)) return rc;
    if (int rc = check_host_chunks(ranges, p)) return rc;
    total += p.chunks.size();
  }
  descs.resize(total);
  size_t d = 0;
  for (uint32_t i = 0; i < num_layers; ++i)
    if (!plans[i].ordered)
      for (const Chunk& c : plans[i].chunks) descs[d++] = ChunkDesc{c.host, c.dev};

  std::lock_guard<std::mutex> lk(sc->mu);
  int prev = 0;
  PF_HIP(hipGetDevice(&prev));
  if (prev != dev) PF_HIP(hipSetDevice(dev));
  ChunkDesc* d_desc = reinterpret_cast<ChunkDesc*>(sc->base + kNoAllocQueueBytes);
  uint32_t* queue = reinterpret_cast<uint32_t*>(sc->base);
  auto issue = [&]() -> int {
    // A pageable source: the call returns once the bytes have been taken,
    // so the thread's buffer may be refilled by its next call.
    if (total > 0)
      PF_HIP(hipMemcpyAsync(d_desc, descs.data(), total * sizeof(ChunkDesc),
                            hipMemcpyHostToDevice, s));
    size_t first = 0;
    uint64_t dma = 0;
    for (uint32_t li = 0; li < num_layers;) {
      const LayerPlan& p = plans[li];
      if (p.ordered) {
        if (int rc = dma_copies(s, p, false, false, &dma)) return rc;
        ++li;
        continue;
      }
      if (p.chunks.empty()) {
        ++li;
        continue;
      }
      // Consecutive layers of the same chunk size and alignment share one
      // launch, whose shape follows its first layer's host side.
      const bool al = chunks_aligned(p);
      size_t n = p.chunks.size();
      uint32_t lj = li + 1;
      while (lj < num_layers && !plans[lj].ordered &&
             (plans[lj].chunks.empty() ||
              (plans[lj].chunk_bytes == p.chunk_bytes && chunks_aligned(plans[lj]) == al))) {
        n += plans[lj].chunks.size();
        ++lj;
      }
      const bool host = host_side_pinned(p);
      if (int rc = check_launch_size(n, p.chunk_bytes)) return rc;
      const hipError_t e = issue_copy(
          s, d_desc + first, n, p.chunk_bytes, al,
          host ? PF_LOAD_HOST_DEFAULT_THREADS : PF_LOAD_DEFAULT_THREADS,
          host ? PF_LOAD_HOST_DEFAULT_UNROLL : (PF_LOAD_DEFAULT_UNROLL & ~PF_KERNEL_AUTO),
          host ? PF_LOAD_HOST_DEFAULT_GRID : 0, 0, nullptr, queue);
      if (e != hipSuccess) return hip_fail(e, "gather/scatter kernel launch");
      first += n;
      li = lj;
    }
    return PF_OK;
  };
  const int rc = issue();
  // A call that failed part-way leaves nothing in flight.
  if (rc != PF_OK) (void)hipStreamSynchronize(s);
  if (prev != dev) (void)hipSetDevice(prev);
  return rc;
}

namespace {

// Bit b of a stream's CU mask enables compute unit b of the device in the
// runtime's numbering, which deals the bits to the XCDs round-robin: bit b
// is on XCD b mod n_xcd (measured on MI355X by recording each workgroup's
// XCC_ID and HW_ID: bits 0-7 are one CU on each of the 8 XCDs, the next 8 a
// second CU of each, in its next shader engine).  Every launch is split
// across all XCDs, so a mask that leaves an XCD without a CU would leave
// that XCD's share of every launch waiting forever: refused.
int check_cu_mask(int device, const uint32_t* mask, uint32_t words) {
  int cus = 0, xcds = 0;
  PF_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  PF_HIP(hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, device));
  if (xcds <= 0) xcds = 1;
  std::vector<int> per_xcd(static_cast<size_t>(xcds), 0);
  for (uint32_t b = 0; b < words * 32u && b < static_cast<uint32_t>(cus); ++b)
    if (mask[b / 32] >> (b % 32) & 1u) ++per_xcd[b % static_cast<uint32_t>(xcds)];
  for (int i = 0; i < xcds; ++i)
    if (per_xcd[static_cast<size_t>(i)] == 0)
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("CU mask leaves XCD %d without a compute unit (bit b of the mask is "
                       "on XCD b mod %d, bits below %d count)",
                       i, xcds, cus));
  return PF_OK;
}

// (Re)creates the context's two streams: plain non-blocking ones, or
// CU-masked ones (HIP creates those as blocking streams: they also order
// with the null stream).
int create_lane_streams(pf_xfer* x, const uint32_t* mask, uint32_t words) {
  if (words) {  // bits past the device's CUs are dropped
    int cus = 0;
    PF_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, x->device));
    words = std::min(words, static_cast<uint32_t>(cus + 31) / 32u);
  }
  hipStream_t s[2] = {nullptr, nullptr};
  hipError_t e = hipSuccess;
  for (int i = 0; i < 2 && e == hipSuccess; ++i)
    e = words ? hipExtStreamCreateWithCUMask(&s[i], words, mask)
              : hipStreamCreateWithFlags(&s[i], hipStreamNonBlocking);
  if (e != hipSuccess) {
    for (hipStream_t t : s)
      if (t) (void)hipStreamDestroy(t);
    return hip_fail(e, words ? "hipExtStreamCreateWithCUMask" : "hipStreamCreateWithFlags");
  }
  if (x->stream) (void)hipStreamDestroy(x->stream);
  if (x->dma) (void)hipStreamDestroy(x->dma);
  x->stream = s[0];
  x->dma = s[1];
  return PF_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Transfer contexts.
// ---------------------------------------------------------------------------
int pf_xfer_create(int device, uint64_t staging_bytes, pf_xfer** out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "null output");
  *out = nullptr;
  if (int rc = pf_init(device)) return rc;
  pf_xfer* x = new pf_xfer();
  x->device = device;
  // PEGAFLOW_STAGED_HEAD=kernel (or =engine): new contexts (the engine's
  // included) copy a layer-by-layer staged load's first layer by the
  // zero-copy kernel (or through the copy engines, the default).
  if (const char* head = std::getenv("PEGAFLOW_STAGED_HEAD")) {
    if (std::strcmp(head, "kernel") == 0) x->staged_head = PF_STAGED_HEAD_KERNEL;
    if (std::strcmp(head, "engine") == 0) x->staged_head = PF_STAGED_HEAD_ENGINE;
  }
  auto cleanup = [&](int rc) {
    pf_xfer_destroy(x);
    return rc;
  };
  // PEGAFLOW_CUS_PER_XCD=<k>: new contexts (the engine's included) run
  // their kernels on k compute units of each XCD (pf_cu_mask_per_xcd).
  if (const char* k = std::getenv("PEGAFLOW_CUS_PER_XCD")) {
    uint32_t mask[64];
    const unsigned long cus = std::strtoul(k, nullptr, 10);
    int rc = pf_cu_mask_per_xcd(device, static_cast<uint32_t>(cus), mask, 64);
    if (rc == PF_OK) rc = create_lane_streams(x, mask, 64);
    if (rc != PF_OK) return cleanup(rc);
  } else if (int rc = create_lane_streams(x, nullptr, 0)) {
    return cleanup(rc);
  }
  hipError_t e = hipEventCreateWithFlags(&x->desc_uploaded, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&x->parts_ready, hipEventDisableTiming);
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&x->h_small), kHostDescMax * sizeof(ChunkDesc),
                      hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void**>(&x->h_boot), 2 * sizeof(ChunkDesc),
                      hipHostMallocMapped | hipHostMallocCoherent);
  for (int s = 0; s < 2 && e == hipSuccess; ++s)
    e = hipEventCreateWithFlags(&x->lane_mark[s], hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&x->staging_free, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&x->head_done, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(x->staging_free, x->stream);
  if (e == hipSuccess && staging_bytes > 0 && engine_copies_available(device)) {
    for (int s = 0; s < kEngineSlots && e == hipSuccess; ++s)
      e = hipEventCreateWithFlags(&x->eng_ev[s], hipEventDisableTiming);
    int rc = PF_OK;
    for (int s = 0; s < kEngineSlots && e == hipSuccess && rc == PF_OK; ++s)
      rc = engine_signal_create(&x->eng_sig[s]);
    if (rc != PF_OK) return cleanup(rc);
    x->engine_ok = e == hipSuccess;
  }
  if (e != hipSuccess) return cleanup(hip_fail(e, "pf_xfer_create"));
  if (staging_bytes > 0) {
    const uint64_t slot = (staging_bytes / 2) & ~uint64_t(255);
    if (slot == 0) return cleanup(fail(PF_ERR_INVALID_ARGUMENT, "staging buffer too small"));
    void* p = nullptr;
    e = hipMalloc(&p, slot * 2);
    if (e != hipSuccess) return cleanup(hip_fail(e, "hipMalloc(staging)"));
    x->staging = reinterpret_cast<uint64_t>(p);
    x->slot_bytes = slot;
  }
  e = hipStreamSynchronize(x->stream);
  if (e != hipSuccess) return cleanup(hip_fail(e, "pf_xfer_create"));
  *out = x;
  return PF_OK;
}

int pf_xfer_destroy(pf_xfer* x) {
  if (!x) return PF_OK;
  (void)hipSetDevice(x->device);
  if (x->stream) (void)hipStreamSynchronize(x->stream);
  if (x->dma) (void)hipStreamSynchronize(x->dma);
  (void)engine_drain(x);
  for (EngineSignal& s : x->eng_sig) engine_signal_destroy(&s);
  for (hipEvent_t ev : x->eng_ev)
    if (ev) (void)hipEventDestroy(ev);
  if (x->staging_free) (void)hipEventDestroy(x->staging_free);
  if (x->head_done) (void)hipEventDestroy(x->head_done);
  if (x->d_desc) (void)hipFree(x->d_desc);
  if (x->d_counters) (void)hipFree(x->d_counters);
  if (x->h_desc) (void)hipHostFree(x->h_desc);
  if (x->h_small) (void)hipHostFree(x->h_small);
  if (x->h_boot) (void)hipHostFree(x->h_boot);
  if (x->staging) (void)hipFree(reinterpret_cast<void*>(x->staging));
  if (x->desc_uploaded) (void)hipEventDestroy(x->desc_uploaded);
  if (x->parts_ready) (void)hipEventDestroy(x->parts_ready);
  for (auto& t : x->timers) {
    (void)hipEventDestroy(t.first);
    (void)hipEventDestroy(t.second);
  }
  for (int s = 0; s < 2; ++s)
    if (x->lane_mark[s]) (void)hipEventDestroy(x->lane_mark[s]);
  for (ScatterTrial& t : x->trials) {
    if (t.start) (void)hipEventDestroy(t.start);
    if (t.stop) (void)hipEventDestroy(t.stop);
  }
  if (x->stream) (void)hipStreamDestroy(x->stream);
  if (x->dma) (void)hipStreamDestroy(x->dma);
  delete x;
  return PF_OK;
}

pf_stream pf_xfer_stream(pf_xfer* x) { return x ? x->stream : nullptr; }

int pf_xfer_synchronize(pf_xfer* x) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  PF_HIP(hipStreamSynchronize(x->dma));
  PF_HIP(hipStreamSynchronize(x->stream));
  return engine_drain(x);
}

int pf_xfer_set_kernel_shape(pf_xfer* x, uint32_t threads, uint32_t unroll) {
  for (uint32_t r = PF_ROUTE_SAVE_DEVICE; r <= PF_ROUTE_LOAD_HOST; ++r)
    if (int rc = pf_xfer_set_kernel_shape_dir(x, r, threads, unroll)) return rc;
  return PF_OK;
}

int pf_xfer_set_kernel_shape_dir(pf_xfer* x, uint32_t direction, uint32_t threads,
                                 uint32_t unroll) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  if (direction > PF_ROUTE_LOAD_HOST)
    return fail(PF_ERR_INVALID_ARGUMENT, "direction must be a route, 0..3 (PF_ROUTE_*)");
  if (threads && (threads < 64 || threads > 1024 || threads % 64))
    return fail(PF_ERR_INVALID_ARGUMENT, "threads must be a multiple of 64 in [64, 1024]");
  const uint32_t u = unroll & 0xffu;
  if (unroll && u != 1 && u != 2 && u != 4 && u != 8 && u != 16)
    return fail(PF_ERR_INVALID_ARGUMENT, "unroll must be 1, 2, 4, 8 or 16");
  if (unroll & ~(0xffu | PF_KERNEL_NONTEMPORAL | PF_KERNEL_XCD_MAJOR | PF_KERNEL_AUTO))
    return fail(PF_ERR_INVALID_ARGUMENT, "unknown kernel flag");
  if ((unroll & PF_KERNEL_AUTO) && direction != PF_ROUTE_LOAD_DEVICE)
    return fail(PF_ERR_INVALID_ARGUMENT, "PF_KERNEL_AUTO applies to the scatter route only");
  std::lock_guard<std::mutex> lk(x->mu);
  if (threads) x->threads[direction] = threads;
  if (unroll) x->unroll[direction] = unroll;
  if (direction == PF_ROUTE_LOAD_DEVICE && (threads || unroll)) scatter_trials_reset(x);
  return PF_OK;
}

int pf_xfer_route_shape(pf_xfer* x, uint32_t route, uint32_t* threads, uint32_t* unroll,
                        int* decided) {
  if (!x || !threads || !unroll || !decided) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  if (route > PF_ROUTE_LOAD_HOST)
    return fail(PF_ERR_INVALID_ARGUMENT, "route must be 0..3 (PF_ROUTE_*)");
  std::lock_guard<std::mutex> lk(x->mu);
  *threads = x->threads[route];
  *unroll = x->unroll[route];
  *decided = 1;
  if (route == PF_ROUTE_LOAD_DEVICE && (x->unroll[route] & PF_KERNEL_AUTO)) {
    (void)hipSetDevice(x->device);
    scatter_trials_update(x);
    const int pick = x->scatter_choice >= 0 ? x->scatter_choice : 0;
    *threads = kScatterShapes[pick][0];
    *unroll = kScatterShapes[pick][1];
    *decided = x->scatter_choice >= 0 ? 1 : 0;
  }
  return PF_OK;
}

int pf_xfer_set_route_grid(pf_xfer* x, uint32_t route, uint32_t workgroups) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  if (route > PF_ROUTE_LOAD_HOST)
    return fail(PF_ERR_INVALID_ARGUMENT, "route must be 0..3 (PF_ROUTE_*)");
  if (workgroups > (1u << 20))
    return fail(PF_ERR_INVALID_ARGUMENT, "at most 2^20 persistent workgroups");
  std::lock_guard<std::mutex> lk(x->mu);
  x->grid[route] = workgroups;
  return PF_OK;
}

int pf_xfer_last_stats(pf_xfer* x, uint64_t* kernel_launches, uint64_t* dma_copies) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  if (kernel_launches) *kernel_launches = x->last_kernels;
  if (dma_copies) *dma_copies = x->last_dma;
  return PF_OK;
}

int pf_xfer_set_max_grid(pf_xfer* x, uint32_t max_workgroups) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  std::lock_guard<std::mutex> lk(x->mu);
  x->max_grid = max_workgroups;
  return PF_OK;
}

int pf_xfer_set_staged_slices(pf_xfer* x, uint64_t save_bytes, uint64_t load_bytes) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  std::lock_guard<std::mutex> lk(x->mu);
  if (save_bytes) x->staged_slice[0] = save_bytes;
  if (load_bytes) x->staged_slice[1] = load_bytes;
  return PF_OK;
}

int pf_xfer_set_staged_head(pf_xfer* x, uint32_t route) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  if (route != PF_STAGED_HEAD_KERNEL && route != PF_STAGED_HEAD_ENGINE)
    return fail(PF_ERR_INVALID_ARGUMENT, strf("unknown staged head route %u", route));
  std::lock_guard<std::mutex> lk(x->mu);
  x->staged_head = route;
  return PF_OK;
}

int pf_cu_mask_per_xcd(int device, uint32_t cus_per_xcd, uint32_t* mask, uint32_t words) {
  if (!mask || words == 0) return fail(PF_ERR_INVALID_ARGUMENT, "null or empty mask");
  int cus = 0, xcds = 0;
  PF_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  PF_HIP(hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, device));
  if (xcds <= 0) xcds = 1;
  const uint64_t bits = uint64_t(cus_per_xcd) * uint64_t(xcds);
  if (cus_per_xcd == 0 || bits > static_cast<uint64_t>(cus))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("%u CUs per XCD: the device has %d CUs on %d XCDs", cus_per_xcd, cus, xcds));
  if (bits > uint64_t(words) * 32u)
    return fail(PF_ERR_INVALID_ARGUMENT, strf("a mask of %u words holds fewer than %llu bits",
                                              words, static_cast<unsigned long long>(bits)));
  for (uint32_t w = 0; w < words; ++w) mask[w] = 0;
  for (uint64_t b = 0; b < bits; ++b) mask[b / 32] |= 1u << (b % 32);
  return PF_OK;
}

int pf_xfer_set_cu_mask(pf_xfer* x, const uint32_t* mask, uint32_t words) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  if (words && !mask) return fail(PF_ERR_INVALID_ARGUMENT, "null mask");
  if (words > 64) return fail(PF_ERR_INVALID_ARGUMENT, "a CU mask has at most 64 words");
  std::lock_guard<std::mutex> lk(x->mu);
  PF_HIP(hipSetDevice(x->device));
  if (words)
    if (int rc = check_cu_mask(x->device, mask, words)) return rc;
  // Everything issued on the old streams ends first.
  PF_HIP(hipStreamSynchronize(x->dma));
  PF_HIP(hipStreamSynchronize(x->stream));
  if (int rc = engine_drain(x)) return rc;
  return create_lane_streams(x, mask, words);
}

int pf_xfer_set_timing(pf_xfer* x, int enable) {
  if (!x) return fail(PF_ERR_INVALID_ARGUMENT, "null transfer context");
  std::lock_guard<std::mutex> lk(x->mu);
  x->timing = enable != 0;
  return PF_OK;
}

int pf_xfer_last_kernel_ms(pf_xfer* x, float* ms, uint64_t* launches) {
  if (!x || !ms) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> lk(x->mu);
  float total = 0.0f;
  const uint64_t n = x->timing ? x->last_kernels : 0;
  for (uint64_t i = 0; i < n && i < x->timers.size(); ++i) {
    PF_HIP(hipEventSynchronize(x->timers[i].second));
    float t = 0.0f;
    PF_HIP(hipEventElapsedTime(&t, x->timers[i].first, x->timers[i].second));
    total += t;
  }
  *ms = total;
  if (launches) *launches = n;
  return PF_OK;
}

int pf_save_layers(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                   uint32_t mode) {
  return run(x, layers, num_layers, mode, true, nullptr);
}

int pf_load_layers(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                   uint32_t mode, pf_event* layer_events) {
  return run(x, layers, num_layers, mode, false, layer_events);
}

int pf_load_layers_marked(pf_xfer* x, const pf_layer_xfer* layers, uint32_t num_layers,
                          uint32_t mode, const pf_layer_signal* signals,
                          uint32_t num_signals) {
  SignalTargets t{};
  if (int rc = signal_targets(signals, num_signals, num_layers, &t)) return rc;
  return run(x, layers, num_layers, mode, false, nullptr, true, &t);
}

}  // extern "C"

namespace pf {

int save_layers_pending_begin(pf_xfer* x, pf_layer_xfer* layers, uint32_t num_layers,
                              uint32_t mode, const PendingLayers& pending) {
  return run(x, layers, num_layers, mode, true, nullptr, false, nullptr, &pending);
}

int load_layers_pending(pf_xfer* x, pf_layer_xfer* layers, uint32_t num_layers, uint32_t mode,
                        pf_event* layer_events, const pf_layer_signal* signals,
                        uint32_t num_signals, const PendingLayers& pending) {
  SignalTargets t{};
  if (num_signals > 0)
    if (int rc = signal_targets(signals, num_signals, num_layers, &t)) return rc;
  return run(x, layers, num_layers, mode, false, layer_events, true,
             num_signals > 0 ? &t : nullptr, &pending);
}

}  // namespace pf
