// pf_kernels.hip — gfx950 gather/scatter kernels of the KV-block transfer
// path, plus the synthetic-data, verification and spin kernels used by the
// benchmark and the parity tests.
//
// The transfer is pure data movement (no contraction, so no MFMA).  A launch
// moves `n_chunks` chunks of `chunk_bytes` each, described by (src, dst)
// address pairs in device memory.  Addresses may be HBM (the paged layer
// tensor, a staging buffer) or host-mapped pinned memory (zero-copy over the
// host link).  The same kernel therefore serves:
//   * save:    paged layer tensor -> pinned host (or HBM staging), a gather;
//   * restore: pinned host (or HBM staging) -> paged layer tensor, a scatter.
//
// Work decomposition: a chunk is split into tiles of blockDim.x * UNROLL
// 16-byte elements.  One workgroup copies one tile: every lane issues UNROLL
// independent 16-byte loads (global_load_dwordx4) before its UNROLL stores,
// so each wave keeps UNROLL * 1 KiB in flight — enough to cover HBM latency
// and, for zero-copy, the much longer host-link read latency.  Consecutive
// lanes touch consecutive 16-byte words, so every wave instruction covers one
// contiguous 1 KiB span (fully coalesced).  No LDS: source and destination
// share the same byte order within a chunk.
#include <hip/hip_runtime.h>

#include "pf_common.h"

namespace pf {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Global-address-space views: the addresses arrive as integers, and without
// the address space the compiler would emit generic (flat) accesses.
typedef __attribute__((address_space(1))) u32x4 g_u32x4;
typedef __attribute__((address_space(1))) uint8_t g_u8;
typedef __attribute__((address_space(1))) uint64_t g_u64;

template <bool NT>
__device__ __forceinline__ u32x4 load16(const g_u32x4* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

template <bool NT>
__device__ __forceinline__ void store16(g_u32x4* p, u32x4 v) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

// NTL / NTS select non-temporal (streaming) loads / stores: every byte is
// touched exactly once, so there is nothing to gain from keeping it in L2 or
// the MALL, and streaming accesses leave those caches to other traffic.
// Workgroup -> tile order.  Workgroups are dealt round-robin to the 8 XCDs
// (workgroup b runs on XCD b % 8).  With xcd_major set (and one workgroup
// per tile), XCD x instead takes one contiguous range of tiles:
//   n = 8q + r tiles; XCD x owns q + (x < r) tiles starting at x*q + min(x, r);
//   workgroup b = 8i + x handles the i-th of them.
// The workgroups with b % 8 == x number exactly q + (x < r), so this is a
// bijection of [0, n).
__device__ __forceinline__ uint32_t tile_of(uint32_t b, uint32_t n, bool xcd_major) {
  if (!xcd_major) return b;
  const uint32_t x = b & 7u, i = b >> 3, q = n >> 3, r = n & 7u;
  return x * q + (x < r ? x : r) + i;
}

// ---------------------------------------------------------------------------
// Layer completion marks.  A load that covers several layers in one launch
// can still report each layer as soon as its bytes are in place: every
// workgroup, after its stores, bumps its layer's tile counter, and the
// workgroup that brings the counter to the layer's tile count writes the
// call's value into word[layer] of each signal target (host-mapped pinned
// memory, device memory, or another process's IPC-mapped device memory).
//
// Visibility.  Each XCD has its own L2, so a byte stored by one workgroup is
// visible to readers on other XCDs only once it has left that L2.  A
// release fence at agent scope per workgroup would write the whole L2 back
// every time (measured: 2.2x slower from pinned memory, 40x from HBM).
// Instead the marking kernel stores its bytes as agent-scope relaxed atomic
// stores, which write through the L2 to the device's coherence point (the
// sc1 policy), and waits for every store's acknowledgement (s_waitcnt 0)
// before the workgroup barrier; only then does one lane bump the counter
// (an agent-scope atomic).  The finishing workgroup acquires at agent scope,
// puts the counter back to 0 (ready for the next launch on the stream) and
// writes the marks as release stores, at system scope for host memory.  A
// reader that sees word[layer] == value and then acquires, or starts a
// kernel afterwards, sees every byte of that layer.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void write_marks(const SignalTargets& t, uint32_t layer) {
  for (uint32_t i = 0; i < t.count; ++i) {
    uint64_t* w = reinterpret_cast<uint64_t*>(t.words[i]) + layer;
    if ((t.host_mask >> i) & 1u)
      __hip_atomic_store(w, t.value[i], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    else
      __hip_atomic_store(w, t.value[i], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// 16 bytes as two agent-coherent (write-through) 8-byte stores.
__device__ __forceinline__ void store16_coherent(g_u32x4* p, u32x4 v) {
  g_u64* q = reinterpret_cast<g_u64*>(p);
  __hip_atomic_store(q, static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, static_cast<uint64_t>(v.z) | (static_cast<uint64_t>(v.w) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by one lane per workgroup once the workgroup's stores of chunk c are
// acknowledged.  marks.chunk_start[0..n] are the launch-relative first
// chunks of its layers (increasing, chunk_start[0] == 0 <= c <
// chunk_start[n]); the search keeps chunk_start[lo] <= c < chunk_start[hi].
__device__ __forceinline__ void tile_done(const LayerMarks& m, uint32_t c,
                                          uint32_t tiles_per_chunk) {
  uint32_t lo = 0, hi = m.n;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (m.chunk_start[mid] <= c) lo = mid;
    else hi = mid;
  }
  const uint32_t layer = m.layer[lo];
  const uint32_t tiles = (m.chunk_start[lo + 1] - m.chunk_start[lo]) * tiles_per_chunk;
  uint32_t* cnt = m.counters + layer;
  const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
  if (prev + 1 == tiles) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    write_marks(m.targets, layer);
  }
}

// tile_done for k tiles of group g of a slice's marks at once, counted
// toward the layer's tiles over all its launches.  The group table lives in
// the kernel's arguments; it is read with constant indices only, so it
// stays in scalar registers.
__device__ __forceinline__ void slice_tiles_done(const SliceMarks& m, uint32_t g, uint32_t k) {
  uint32_t layer = 0, tiles = 0;
#pragma unroll
  for (uint32_t i = 0; i < kSliceMarkLayers; ++i)
    if (i == g) {
      layer = m.layer[i];
      tiles = m.tiles[i];
    }
  if (tiles == 0) return;  // marked by another kernel
  uint32_t* cnt = m.counters + layer;
  const uint32_t prev = __hip_atomic_fetch_add(cnt, k, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
  if (prev + k == tiles) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    write_marks(m.targets, layer);
  }
}

// The group of chunk c: the last g < n with chunk_start[g] <= c.
__device__ __forceinline__ uint32_t slice_group_of(const SliceMarks& m, uint32_t c) {
  uint32_t g = 0;
#pragma unroll
  for (uint32_t i = 1; i < kSliceMarkLayers; ++i)
    if (i < m.n && m.chunk_start[i] <= c) g = i;
  return g;
}

// A marked copy between device buffers (the staged load's scatter of a
// slice whose layers it reports itself): a fixed map like
// copy_chunks_v16_kernel.  Workgroup w copies tiles w, w + grid, ..., which
// run through the launch's layers in order, and reports the tiles it
// finished of a layer once, when it moves on to the next layer or ends, not
// once per tile: one counter takes one add at a time, and per-tile adds
// (2,560 for a 40 MiB layer, in a queued launch) held such a copy at a
// fraction of HBM rate.
//
// Visibility differs from the marking protocol above: the bytes are stored
// as ordinary (write-back) stores, and before a workgroup reports a layer,
// every wave's stores are acknowledged (s_waitcnt 0), the workgroup meets
// at its barrier, and one lane issues an agent-scope release fence, which
// writes its XCD's L2 back to the device's coherence point; then it adds to
// the counter.  The finishing workgroup acquires and writes the marks as
// above.  A fence writes back the whole L2, so it pays per workgroup, not
// per store: with 128 workgroups a 40 MiB layer took 24.8 us, against 35.9
// with write-through stores and 73 with 1,280 workgroups.  The report
// condition depends only on the tile index, so it is uniform across the
// workgroup and its barrier is reached by every lane.
template <int UNROLL, bool NTL>
__global__ void __launch_bounds__(1024)
copy_chunks_marked_kernel(const ChunkDesc* __restrict__ descs, uint32_t tiles_per_chunk,
                          uint32_t n_tiles, uint32_t chunk16, SliceMarks marks) {
  const uint32_t stride = blockDim.x;
  const uint32_t tile_elems = stride * UNROLL;
  uint32_t group = 0, done = 0;
  for (uint32_t t = blockIdx.x; t < n_tiles; t += gridDim.x) {
    const uint32_t c = t / tiles_per_chunk;
    const uint32_t g = slice_group_of(marks, c);
    if (done > 0 && g != group) {
      __builtin_amdgcn_s_waitcnt(0);  // every store of this wave acknowledged
      __syncthreads();
      if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        slice_tiles_done(marks, group, done);
      }
      done = 0;
    }
    group = g;
    const uint32_t tile = t - c * tiles_per_chunk;
    const ChunkDesc d = descs[c];
    const g_u32x4* __restrict__ src = reinterpret_cast<const g_u32x4*>(d.src);
    g_u32x4* __restrict__ dst = reinterpret_cast<g_u32x4*>(d.dst);
    const uint32_t tile_base = tile * tile_elems;
    const uint32_t base = tile_base + threadIdx.x;
    u32x4 v[UNROLL];
    if (tile_base + tile_elems <= chunk16) {
      // Every load of the tile in flight before its stores.
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = load16<NTL>(src + base + u * stride);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) store16<true>(dst + base + u * stride, v[u]);
    } else {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t e = base + u * stride;
        if (e < chunk16) v[u] = load16<NTL>(src + e);
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t e = base + u * stride;
        if (e < chunk16) store16<true>(dst + e, v[u]);
      }
    }
    ++done;
  }
  if (done > 0) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      slice_tiles_done(marks, group, done);
    }
  }
}

template <int UNROLL, bool NTL, bool NTS>
__global__ void __launch_bounds__(1024)
copy_chunks_v16_kernel(const ChunkDesc* __restrict__ descs,
                       uint32_t tiles_per_chunk, uint32_t n_tiles,
                       uint32_t chunk16, uint32_t xcd_major) {
  const uint32_t stride = blockDim.x;
  const uint32_t tile_elems = stride * UNROLL;
  const bool remap = xcd_major && gridDim.x == n_tiles;
  for (uint32_t b = blockIdx.x; b < n_tiles; b += gridDim.x) {
    const uint32_t t = tile_of(b, n_tiles, remap);
    const uint32_t c = t / tiles_per_chunk;
    const uint32_t tile = t - c * tiles_per_chunk;
    const ChunkDesc d = descs[c];
    const g_u32x4* __restrict__ src = reinterpret_cast<const g_u32x4*>(d.src);
    g_u32x4* __restrict__ dst = reinterpret_cast<g_u32x4*>(d.dst);
    const uint32_t tile_base = tile * tile_elems;
    const uint32_t base = tile_base + threadIdx.x;
    u32x4 v[UNROLL];
    if (tile_base + tile_elems <= chunk16) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = load16<NTL>(src + base + u * stride);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) store16<NTS>(dst + base + u * stride, v[u]);
    } else {
      // Partial last tile of a chunk: guarded per element.
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t e = base + u * stride;
        if (e < chunk16) v[u] = load16<NTL>(src + e);
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t e = base + u * stride;
        if (e < chunk16) store16<NTS>(dst + e, v[u]);
      }
    }
  }
}

// Copies over the host link take their tiles from a work queue instead of a
// fixed workgroup -> tile map.  Workgroups are dealt to the 8 XCDs
// statically, and when the copy reads or writes host memory the XCDs
// progress at very different rates (the link is not shared fairly between
// them): with a fixed map the copy ends when the slowest XCD does, and a
// marked load's layers land only when the slowest XCD gets to them
// (measured: the first of 32 Llama layers after half the load).  Here a
// small persistent grid pulls tile indices from one counter, so the fast
// XCDs take more tiles and tiles, hence layers, finish in order; with few
// requests in flight the link also runs closer to its peak (Llama restore
// 24.1 -> 23.3 ms of kernel time with 64 workgroups).
//
// The queue is two words, queue[0] the next tile and queue[1] the
// workgroups that have left, both 0 when a launch starts.  A workgroup
// leaves after a pull past the last tile, and counts itself out with an
// acquire-release add; the last one out has seen every workgroup's final
// pull, so it puts both words back to 0.  The launch therefore leaves the
// queue as it found it, whatever the host knows of earlier launches: a
// replayed graph or a launch on another stream after this one finds 0.
// Launches that run at the same time need queues of their own.  MARK adds
// the per-layer completion marks, with agent-coherent stores (see
// write_marks).
template <int UNROLL, bool NTL, bool NTS, bool MARK>
__global__ void __launch_bounds__(1024)
copy_chunks_queue_kernel(const ChunkDesc* __restrict__ descs, uint32_t tiles_per_chunk,
                         uint32_t n_tiles, uint32_t chunk16, LayerMarks marks,
                         uint32_t* queue) {
  __shared__ uint32_t s_tile;
  const uint32_t stride = blockDim.x;
  const uint32_t tile_elems = stride * UNROLL;
  for (;;) {
    if (threadIdx.x == 0)
      s_tile = __hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t t = s_tile;
    __syncthreads();  // every lane has read s_tile before it is written again
    if (t >= n_tiles) {  // uniform: the queue is empty for every later pull too
      if (threadIdx.x == 0) {
        const uint32_t out = __hip_atomic_fetch_add(queue + 1, 1u, __ATOMIC_ACQ_REL,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (out + 1 == gridDim.x) {
          __hip_atomic_store(queue, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(queue + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      break;
    }
    const uint32_t c = t / tiles_per_chunk;
    const uint32_t tile = t - c * tiles_per_chunk;
    const ChunkDesc d = descs[c];
    const g_u32x4* __restrict__ src = reinterpret_cast<const g_u32x4*>(d.src);
    g_u32x4* __restrict__ dst = reinterpret_cast<g_u32x4*>(d.dst);
    const uint32_t tile_base = tile * tile_elems;
    const uint32_t base_e = tile_base + threadIdx.x;
    u32x4 v[UNROLL];
    if (tile_base + tile_elems <= chunk16) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) v[u] = load16<NTL>(src + base_e + u * stride);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        if constexpr (MARK) store16_coherent(dst + base_e + u * stride, v[u]);
        else store16<NTS>(dst + base_e + u * stride, v[u]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t e = base_e + u * stride;
        if (e < chunk16) v[u] = load16<NTL>(src + e);
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const uint32_t e = base_e + u * stride;
        if (e < chunk16) {
          if constexpr (MARK) store16_coherent(dst + e, v[u]);
          else store16<NTS>(dst + e, v[u]);
        }
      }
    }
    if constexpr (MARK) {
      __builtin_amdgcn_s_waitcnt(0);  // every store of this wave acknowledged
      __syncthreads();
      if (threadIdx.x == 0) tile_done(marks, c, tiles_per_chunk);
    }
  }
}

// Marks the listed layers (layers with nothing to copy, and layers copied by
// DMA earlier on the same stream).
__global__ void mark_layers_kernel(LayerList list, SignalTargets t) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < list.n) write_marks(t, list.ids[i]);
}

// Bounded device-side wait: lane 0 polls *word until it reaches `value` or
// `max_ticks` of the device wall clock have passed, so the wave always ends.
// On a timeout *timed_out (if given) is set to 1.
__global__ void wait_word_kernel(const uint64_t* word, uint64_t value, uint64_t max_ticks,
                                 uint32_t* timed_out) {
  if (threadIdx.x != 0) return;
  const uint64_t start = static_cast<uint64_t>(wall_clock64());
  while (__hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < value) {
    if (static_cast<uint64_t>(wall_clock64()) - start >= max_ticks) {
      if (timed_out)
        __hip_atomic_store(timed_out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Fallback for chunks whose addresses or size are not 16-byte aligned.
__global__ void __launch_bounds__(1024)
copy_chunks_b1_kernel(const ChunkDesc* __restrict__ descs, uint32_t n_chunks,
                      uint64_t chunk_bytes) {
  for (uint32_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const ChunkDesc d = descs[c];
    const g_u8* __restrict__ src = reinterpret_cast<const g_u8*>(d.src);
    g_u8* __restrict__ dst = reinterpret_cast<g_u8*>(d.dst);
    for (uint64_t i = threadIdx.x; i < chunk_bytes; i += blockDim.x) dst[i] = src[i];
  }
}

// Upper bound on workgroups per launch; larger tile counts loop.
static constexpr uint32_t kMaxGrid = 1u << 20;

template <int UNROLL, bool NTL, bool NTS>
static void launch_v16_nt(dim3 grid, dim3 block, hipStream_t stream, const ChunkDesc* d,
                          uint32_t tpc, uint32_t n_tiles, uint32_t c16, uint32_t xcd) {
  hipLaunchKernelGGL((copy_chunks_v16_kernel<UNROLL, NTL, NTS>), grid, block, 0, stream, d,
                     tpc, n_tiles, c16, xcd);
}

template <int UNROLL>
static hipError_t launch_v16(const ChunkDesc* d_descs, uint32_t tiles_per_chunk,
                             uint32_t n_tiles, uint32_t chunk16, uint32_t threads,
                             uint32_t flags, uint32_t max_grid, hipStream_t stream) {
  const uint32_t cap = max_grid ? max_grid : kMaxGrid;
  const dim3 grid(n_tiles < cap ? n_tiles : cap), block(threads);
  const uint32_t xcd = (flags & PF_KERNEL_XCD_MAJOR) ? 1u : 0u;
  switch (flags & PF_KERNEL_NONTEMPORAL) {
    case 0:
      launch_v16_nt<UNROLL, false, false>(grid, block, stream, d_descs, tiles_per_chunk, n_tiles,
                                          chunk16, xcd);
      break;
    case PF_KERNEL_NT_LOADS:
      launch_v16_nt<UNROLL, true, false>(grid, block, stream, d_descs, tiles_per_chunk, n_tiles,
                                         chunk16, xcd);
      break;
    case PF_KERNEL_NT_STORES:
      launch_v16_nt<UNROLL, false, true>(grid, block, stream, d_descs, tiles_per_chunk, n_tiles,
                                         chunk16, xcd);
      break;
    default:
      launch_v16_nt<UNROLL, true, true>(grid, block, stream, d_descs, tiles_per_chunk, n_tiles,
                                        chunk16, xcd);
      break;
  }
  return hipGetLastError();
}

template <int UNROLL, bool NTL, bool NTS>
static void launch_queue_nt(dim3 grid, dim3 block, hipStream_t stream, const ChunkDesc* d,
                            uint32_t tpc, uint32_t n_tiles, uint32_t c16,
                            const LayerMarks* marks, uint32_t* queue) {
  if (marks)
    hipLaunchKernelGGL((copy_chunks_queue_kernel<UNROLL, NTL, NTS, true>), grid, block, 0,
                       stream, d, tpc, n_tiles, c16, *marks, queue);
  else
    hipLaunchKernelGGL((copy_chunks_queue_kernel<UNROLL, NTL, NTS, false>), grid, block, 0,
                       stream, d, tpc, n_tiles, c16, LayerMarks{}, queue);
}

template <int UNROLL>
static void launch_queue(dim3 grid, dim3 block, hipStream_t stream, const ChunkDesc* d,
                         uint32_t tpc, uint32_t n_tiles, uint32_t c16, uint32_t flags,
                         const LayerMarks* marks, uint32_t* queue) {
  switch (flags & PF_KERNEL_NONTEMPORAL) {
    case 0:
      launch_queue_nt<UNROLL, false, false>(grid, block, stream, d, tpc, n_tiles, c16, marks,
                                            queue);
      break;
    case PF_KERNEL_NT_LOADS:
      launch_queue_nt<UNROLL, true, false>(grid, block, stream, d, tpc, n_tiles, c16, marks,
                                           queue);
      break;
    case PF_KERNEL_NT_STORES:
      launch_queue_nt<UNROLL, false, true>(grid, block, stream, d, tpc, n_tiles, c16, marks,
                                           queue);
      break;
    default:
      launch_queue_nt<UNROLL, true, true>(grid, block, stream, d, tpc, n_tiles, c16, marks,
                                          queue);
      break;
  }
}

// Tiles of a launch: every tile index < n_tiles maps to chunk < n_chunks and
// element offsets < tiles_per_chunk * tile_elems; elements >= chunk16 are
// masked, and the full-tile path is taken only when the whole tile lies
// below chunk16.  chunk16 < 2^31 and tile_elems <= 16384 keep
// tile_base + tile_elems in 32 bits.
static bool tile_geometry(uint32_t n_chunks, uint64_t chunk_bytes, uint32_t threads,
                          uint32_t unroll, uint32_t* tpc, uint32_t* n_tiles, uint32_t* c16) {
  const uint64_t chunk16 = chunk_bytes / 16;
  if (chunk16 >= (1ull << 31)) return false;
  const uint64_t tile_elems = static_cast<uint64_t>(threads) * unroll;
  if (tile_elems == 0) return false;
  const uint64_t tiles_per_chunk = (chunk16 + tile_elems - 1) / tile_elems;
  const uint64_t tiles = tiles_per_chunk * n_chunks;
  if (tiles > 0xffffffffull) return false;
  *tpc = static_cast<uint32_t>(tiles_per_chunk);
  *n_tiles = static_cast<uint32_t>(tiles);
  *c16 = static_cast<uint32_t>(chunk16);
  return true;
}

// `unroll` carries the loads in flight per lane (low byte) and the
// PF_KERNEL_NT_LOADS / PF_KERNEL_NT_STORES / PF_KERNEL_XCD_MAJOR flags.
hipError_t launch_copy_chunks(const ChunkDesc* d_descs, uint32_t n_chunks,
                              uint64_t chunk_bytes, bool aligned16,
                              uint32_t threads, uint32_t unroll,
                              uint32_t max_grid, hipStream_t stream) {
  if (n_chunks == 0 || chunk_bytes == 0) return hipSuccess;
  if (threads == 0 || threads > 1024 || threads % 64 != 0) return hipErrorInvalidValue;
  const uint32_t flags = unroll & (PF_KERNEL_NONTEMPORAL | PF_KERNEL_XCD_MAJOR);
  unroll &= 0xffu;
  if (max_grid > kMaxGrid) max_grid = kMaxGrid;
  if (!aligned16) {
    const uint32_t grid = n_chunks < kMaxGrid ? n_chunks : kMaxGrid;
    hipLaunchKernelGGL(copy_chunks_b1_kernel, dim3(grid), dim3(threads), 0,
                       stream, d_descs, n_chunks, chunk_bytes);
    return hipGetLastError();
  }
  uint32_t tpc = 0, ntl = 0, c16 = 0;
  if (!tile_geometry(n_chunks, chunk_bytes, threads, unroll, &tpc, &ntl, &c16))
    return hipErrorInvalidValue;
  switch (unroll) {
    case 1: return launch_v16<1>(d_descs, tpc, ntl, c16, threads, flags, max_grid, stream);
    case 2: return launch_v16<2>(d_descs, tpc, ntl, c16, threads, flags, max_grid, stream);
    case 4: return launch_v16<4>(d_descs, tpc, ntl, c16, threads, flags, max_grid, stream);
    case 8: return launch_v16<8>(d_descs, tpc, ntl, c16, threads, flags, max_grid, stream);
    case 16: return launch_v16<16>(d_descs, tpc, ntl, c16, threads, flags, max_grid, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_copy_chunks_queue(const ChunkDesc* d_descs, uint32_t n_chunks,
                                    uint64_t chunk_bytes, uint32_t threads, uint32_t unroll,
                                    uint32_t grid, const LayerMarks* marks,
                                    uint32_t* queue, uint32_t* n_tiles, hipStream_t stream) {
  *n_tiles = 0;
  if (n_chunks == 0 || chunk_bytes == 0) return hipSuccess;
  if (threads == 0 || threads > 1024 || threads % 64 != 0 || grid == 0 || !queue)
    return hipErrorInvalidValue;
  if (marks && (marks->n == 0 || !marks->chunk_start || !marks->layer || !marks->counters ||
                marks->targets.count == 0 || marks->targets.count > kMaxSignalTargets))
    return hipErrorInvalidValue;
  const uint32_t flags = unroll & PF_KERNEL_NONTEMPORAL;
  unroll &= 0xffu;
  uint32_t tpc = 0, ntiles = 0, c16 = 0;
  if (!tile_geometry(n_chunks, chunk_bytes, threads, unroll, &tpc, &ntiles, &c16))
    return hipErrorInvalidValue;
  if (static_cast<uint64_t>(ntiles) + grid > 0xffffffffull) return hipErrorInvalidValue;
  if (grid > kMaxGrid) return hipErrorInvalidValue;
  const dim3 g(grid), b(threads);
  switch (unroll) {
    case 1: launch_queue<1>(g, b, stream, d_descs, tpc, ntiles, c16, flags, marks, queue); break;
    case 2: launch_queue<2>(g, b, stream, d_descs, tpc, ntiles, c16, flags, marks, queue); break;
    case 4: launch_queue<4>(g, b, stream, d_descs, tpc, ntiles, c16, flags, marks, queue); break;
    case 8: launch_queue<8>(g, b, stream, d_descs, tpc, ntiles, c16, flags, marks, queue); break;
    case 16: launch_queue<16>(g, b, stream, d_descs, tpc, ntiles, c16, flags, marks, queue); break;
    default: return hipErrorInvalidValue;
  }
  *n_tiles = ntiles;
  return hipGetLastError();
}

template <int UNROLL>
static void launch_marked(dim3 g, dim3 b, hipStream_t stream, bool ntl, const ChunkDesc* d,
                          uint32_t tpc, uint32_t ntiles, uint32_t c16, const SliceMarks& m) {
  if (ntl)
    hipLaunchKernelGGL((copy_chunks_marked_kernel<UNROLL, true>), g, b, 0, stream, d, tpc,
                       ntiles, c16, m);
  else
    hipLaunchKernelGGL((copy_chunks_marked_kernel<UNROLL, false>), g, b, 0, stream, d, tpc,
                       ntiles, c16, m);
}

hipError_t launch_copy_chunks_marked(const ChunkDesc* d_descs, uint32_t n_chunks,
                                     uint64_t chunk_bytes, uint32_t threads, uint32_t unroll,
                                     uint32_t grid, const SliceMarks& marks,
                                     hipStream_t stream) {
  if (n_chunks == 0 || chunk_bytes == 0) return hipSuccess;
  if (threads == 0 || threads > 1024 || threads % 64 != 0 || grid == 0 || grid > kMaxGrid)
    return hipErrorInvalidValue;
  if (marks.n == 0 || marks.n > kSliceMarkLayers || !marks.counters ||
      marks.targets.count == 0 || marks.targets.count > kMaxSignalTargets ||
      marks.chunk_start[0] != 0 || marks.chunk_start[marks.n] != n_chunks)
    return hipErrorInvalidValue;
  const bool ntl = (unroll & PF_KERNEL_NT_LOADS) != 0;
  unroll &= 0xffu;
  uint32_t tpc = 0, ntiles = 0, c16 = 0;
  if (!tile_geometry(n_chunks, chunk_bytes, threads, unroll, &tpc, &ntiles, &c16))
    return hipErrorInvalidValue;
  // Groups in chunk order, each counting at least its own tiles.
  for (uint32_t g = 0; g < marks.n; ++g)
    if (marks.chunk_start[g + 1] <= marks.chunk_start[g] ||
        (marks.tiles[g] != 0 &&
         static_cast<uint64_t>(marks.tiles[g]) <
             static_cast<uint64_t>(marks.chunk_start[g + 1] - marks.chunk_start[g]) * tpc))
      return hipErrorInvalidValue;
  if (static_cast<uint64_t>(ntiles) + grid > 0xffffffffull) return hipErrorInvalidValue;
  const dim3 g(grid < ntiles ? grid : ntiles), b(threads);
  switch (unroll) {
    case 1: launch_marked<1>(g, b, stream, ntl, d_descs, tpc, ntiles, c16, marks); break;
    case 2: launch_marked<2>(g, b, stream, ntl, d_descs, tpc, ntiles, c16, marks); break;
    case 4: launch_marked<4>(g, b, stream, ntl, d_descs, tpc, ntiles, c16, marks); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_mark_layers(const LayerList& list, const SignalTargets& t,
                              hipStream_t stream) {
  if (list.n == 0) return hipSuccess;
  if (list.n > kLayerListMax || t.count == 0 || t.count > kMaxSignalTargets)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(mark_layers_kernel, dim3(1), dim3(kLayerListMax), 0, stream, list, t);
  return hipGetLastError();
}

hipError_t launch_wait_word(uint64_t word, uint64_t value, uint64_t max_ticks,
                            uint64_t timed_out, hipStream_t stream) {
  hipLaunchKernelGGL(wait_word_kernel, dim3(1), dim3(64), 0, stream,
                     reinterpret_cast<const uint64_t*>(word), value, max_ticks,
                     reinterpret_cast<uint32_t*>(timed_out));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic data: splitmix64 words, word[i] = mix64(seed + (off+i+1)*GAMMA).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__global__ void __launch_bounds__(256)
fill_random_kernel(uint64_t* __restrict__ dst, uint64_t n_words, uint64_t seed,
                   uint64_t word_offset) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n_words; i += step)
    dst[i] = mix64(seed + (word_offset + i + 1) * kGamma);
}

__global__ void __launch_bounds__(256)
verify_random_kernel(const uint64_t* __restrict__ src, uint64_t n_words,
                     uint64_t seed, uint64_t word_offset,
                     unsigned long long* count) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  unsigned long long bad = 0;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n_words; i += step)
    bad += src[i] != mix64(seed + (word_offset + i + 1) * kGamma);
  if (bad) atomicAdd(count, bad);
}

// One workgroup per chunk (grid-stride over chunks).
__global__ void __launch_bounds__(256)
verify_random_chunks_kernel(const uint64_t* __restrict__ addrs,
                            const uint64_t* __restrict__ word_offsets, uint64_t n,
                            uint64_t chunk_words, uint64_t seed,
                            unsigned long long* count) {
  unsigned long long bad = 0;
  for (uint64_t c = blockIdx.x; c < n; c += gridDim.x) {
    const g_u64* src = reinterpret_cast<const g_u64*>(addrs[c]);
    const uint64_t off = word_offsets[c];
    for (uint64_t i = threadIdx.x; i < chunk_words; i += blockDim.x)
      bad += src[i] != mix64(seed + (off + i + 1) * kGamma);
  }
  if (bad) atomicAdd(count, bad);
}

__global__ void __launch_bounds__(256)
compare_kernel(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
               uint64_t n, unsigned long long* count) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  unsigned long long bad = 0;
  const bool aligned = ((reinterpret_cast<uint64_t>(a) | reinterpret_cast<uint64_t>(b)) & 7) == 0;
  uint64_t tail_start = 0;
  if (aligned) {
    const uint64_t* wa = reinterpret_cast<const uint64_t*>(a);
    const uint64_t* wb = reinterpret_cast<const uint64_t*>(b);
    const uint64_t nw = n / 8;
    for (uint64_t i = tid; i < nw; i += step) {
      uint64_t x = wa[i] ^ wb[i];
      for (int k = 0; k < 8; ++k) bad += ((x >> (8 * k)) & 0xff) != 0;
    }
    tail_start = nw * 8;
  }
  for (uint64_t i = tail_start + tid; i < n; i += step) bad += a[i] != b[i];
  if (bad) atomicAdd(count, bad);
}

__global__ void spin_kernel(uint64_t ticks) {
  if (threadIdx.x == 0) {
    const uint64_t start = static_cast<uint64_t>(wall_clock64());
    while (static_cast<uint64_t>(wall_clock64()) - start < ticks)
      __builtin_amdgcn_s_sleep(4);
  }
}

static uint32_t grid_for(uint64_t items, uint32_t threads) {
  uint64_t g = (items + threads - 1) / threads;
  if (g > 65536) g = 65536;
  if (g == 0) g = 1;
  return static_cast<uint32_t>(g);
}

hipError_t launch_fill_random(uint64_t dst, uint64_t size_bytes, uint64_t seed,
                              uint64_t word_offset, hipStream_t stream) {
  const uint64_t n = size_bytes / 8;
  hipLaunchKernelGGL(fill_random_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                     stream, reinterpret_cast<uint64_t*>(dst), n, seed,
                     word_offset);
  return hipGetLastError();
}

hipError_t launch_verify_random(uint64_t addr, uint64_t size_bytes,
                                uint64_t seed, uint64_t word_offset,
                                unsigned long long* d_count,
                                hipStream_t stream) {
  const uint64_t n = size_bytes / 8;
  hipLaunchKernelGGL(verify_random_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                     stream, reinterpret_cast<const uint64_t*>(addr), n, seed,
                     word_offset, d_count);
  return hipGetLastError();
}

hipError_t launch_verify_random_chunks(const uint64_t* d_addrs,
                                       const uint64_t* d_word_offsets,
                                       uint64_t n, uint64_t chunk_bytes,
                                       uint64_t seed,
                                       unsigned long long* d_count,
                                       hipStream_t stream) {
  const uint32_t grid = n < 65536 ? static_cast<uint32_t>(n) : 65536u;
  hipLaunchKernelGGL(verify_random_chunks_kernel, dim3(grid), dim3(256), 0, stream,
                     d_addrs, d_word_offsets, n, chunk_bytes / 8, seed, d_count);
  return hipGetLastError();
}

hipError_t launch_compare(uint64_t a, uint64_t b, uint64_t size_bytes,
                          unsigned long long* d_count, hipStream_t stream) {
  hipLaunchKernelGGL(compare_kernel, dim3(grid_for(size_bytes / 8 + 1, 256)),
                     dim3(256), 0, stream, reinterpret_cast<const uint8_t*>(a),
                     reinterpret_cast<const uint8_t*>(b), size_bytes, d_count);
  return hipGetLastError();
}

hipError_t launch_spin(uint64_t ticks, hipStream_t stream) {
  hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(64), 0, stream, ticks);
  return hipGetLastError();
}

}  // namespace pf
