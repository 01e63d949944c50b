/*
 * pf_oracle.c — CPU restatement of PegaFlow's KV-block transfer path.
 *
 * TEST INFRASTRUCTURE ONLY: what the HIP product path is tested against, and
 * the CPU baseline timed beside it.  Nothing in the product loads this file.
 *
 * Reference: xiaguan/pegaflow (Rust).  The reference cannot be built here (no
 * Rust toolchain, and its cudarc dependency needs CUDA), so this is a
 * restatement pinned by the checks in tests/test_oracle.py.  Each function
 * cites the reference lines it follows.  Host memcpy stands in for
 * cuMemcpyDtoH_v2 / cuMemcpyHtoDAsync_v2 (transfer.rs:69, 101).
 */
#include "pf_oracle.h"

#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void set_err(char* err, size_t errlen, const char* fmt, ...) {
  if (!err || errlen == 0) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, errlen, fmt, ap);
  va_end(ap);
}

static int mul_ovf(uint64_t a, uint64_t b, uint64_t* out) {
  return __builtin_mul_overflow(a, b, out);
}
static int add_ovf(uint64_t a, uint64_t b, uint64_t* out) {
  return __builtin_add_overflow(a, b, out);
}

/* lib.rs:389-449 (register_context_layer's layout validation) and the
 * KVCacheRegistration it builds (lib.rs:457-465). */
int or_layout_init(uint64_t data_ptr, uint64_t size_bytes, uint64_t num_blocks,
                   uint64_t bytes_per_block, uint64_t kv_stride_bytes,
                   uint64_t segments, or_layout* out, char* err,
                   size_t errlen) {
  if (bytes_per_block == 0 || num_blocks == 0 || segments == 0) {
    set_err(err, errlen, "invalid KV cache layout for layer");
    return OR_ERR;
  }
  if (segments > 1 && kv_stride_bytes == 0) {
    set_err(err, errlen,
            "kv_stride_bytes must be > 0 when segments > 1 for layer");
    return OR_ERR;
  }
  uint64_t block_size, max_block_offset, max_segment_offset, max_offset, end;
  if (mul_ovf(bytes_per_block, segments, &block_size)) {
    set_err(err, errlen, "block size overflow: bytes_per_block=%llu segments=%llu",
            (unsigned long long)bytes_per_block, (unsigned long long)segments);
    return OR_ERR;
  }
  if (mul_ovf(num_blocks - 1, bytes_per_block, &max_block_offset)) {
    set_err(err, errlen, "num_blocks %llu too large",
            (unsigned long long)num_blocks);
    return OR_ERR;
  }
  if (mul_ovf(segments - 1, kv_stride_bytes, &max_segment_offset)) {
    set_err(err, errlen, "segments/stride overflow (segments=%llu, stride=%llu)",
            (unsigned long long)segments, (unsigned long long)kv_stride_bytes);
    return OR_ERR;
  }
  if (add_ovf(max_block_offset, max_segment_offset, &max_offset)) {
    set_err(err, errlen, "layout offset overflow");
    return OR_ERR;
  }
  if (add_ovf(max_offset, bytes_per_block, &end)) {
    set_err(err, errlen, "layout end overflow");
    return OR_ERR;
  }
  if (end > size_bytes) {
    set_err(err, errlen,
            "registered memory too small: need at least %llu bytes, got %llu",
            (unsigned long long)end, (unsigned long long)size_bytes);
    return OR_ERR;
  }
  out->data_ptr = data_ptr;
  out->size_bytes = size_bytes;
  out->num_blocks = num_blocks;
  out->bytes_per_block = bytes_per_block;
  out->block_size_bytes = block_size;
  out->kv_stride_bytes = kv_stride_bytes;
  out->segments = segments;
  return OR_OK;
}

/* transfer.rs:18-47.  The final `offset + bytes_per_block` is unchecked in
 * the reference; an overflow there is treated as exceeding the limit. */
int or_segment_offset(const or_layout* reg, uint64_t block_idx,
                      uint64_t segment_idx, uint64_t* out, char* err,
                      size_t errlen) {
  if (segment_idx >= reg->segments) {
    set_err(err, errlen, "Segment index out of range");
    return OR_ERR;
  }
  uint64_t base, seg_off, offset, end;
  if (mul_ovf(block_idx, reg->bytes_per_block, &base)) {
    set_err(err, errlen, "Block offset overflow");
    return OR_ERR;
  }
  if (mul_ovf(segment_idx, reg->kv_stride_bytes, &seg_off)) {
    set_err(err, errlen, "Segment offset overflow");
    return OR_ERR;
  }
  if (add_ovf(base, seg_off, &offset)) {
    set_err(err, errlen, "Combined offset overflow");
    return OR_ERR;
  }
  if (add_ovf(offset, reg->bytes_per_block, &end) || end > reg->size_bytes) {
    set_err(err, errlen,
            "Block %llu segment %llu exceeds registered memory (offset %llu, "
            "size %llu, limit %llu)",
            (unsigned long long)block_idx, (unsigned long long)segment_idx,
            (unsigned long long)offset,
            (unsigned long long)reg->bytes_per_block,
            (unsigned long long)reg->size_bytes);
    return OR_ERR;
  }
  *out = offset;
  return OR_OK;
}

/* transfer.rs:50-52. */
int or_is_contiguous(const or_layout* reg) {
  return reg->segments <= 1 || reg->kv_stride_bytes == reg->bytes_per_block;
}

/* gpu_worker.rs:218 and 326 select the split path; transfer.rs:206 the
 * contiguous one; everything else is the strided per-segment save of
 * transfer.rs:217-239 paired with the whole-block load of
 * gpu_worker.rs:260-282. */
int or_layout_kind(const or_layout* reg) {
  if (reg->segments == 2 && reg->kv_stride_bytes > reg->bytes_per_block)
    return OR_SPLIT;
  if (or_is_contiguous(reg)) return OR_CONTIGUOUS;
  return OR_STRIDED;
}

/* transfer.rs:134-177. */
uint64_t or_merge_runs(const uint64_t* gpu_off, const uint64_t* cpu_addr,
                       uint64_t n, uint64_t seg, uint64_t* run_start,
                       uint64_t* run_count) {
  uint64_t runs = 0, i = 0;
  while (i < n) {
    uint64_t count = 1;
    while (i + count < n) {
      uint64_t expect_gpu = gpu_off[i] + count * seg;
      uint64_t expect_cpu = cpu_addr[i] + count * seg;
      if (gpu_off[i + count] == expect_gpu && cpu_addr[i + count] == expect_cpu)
        count++;
      else
        break;
    }
    if (run_start) run_start[runs] = i;
    if (run_count) run_count[runs] = count;
    runs++;
    i += count;
  }
  return runs;
}

/* lib.rs:590-621 (filtering) and 598-603 (range error). */
int or_plan_save(const or_layout* reg, const int32_t* block_ids, uint64_t n,
                 const uint8_t* skip, int64_t* out_idx, uint64_t* out_n,
                 char* err, size_t errlen) {
  uint64_t k = 0;
  for (uint64_t i = 0; i < n; i++) {
    if (block_ids[i] < 0) continue;
    uint64_t b = (uint64_t)block_ids[i];
    if (b >= reg->num_blocks) {
      set_err(err, errlen,
              "block %llu out of range for layer (%llu blocks registered)",
              (unsigned long long)b, (unsigned long long)reg->num_blocks);
      return OR_ERR;
    }
    if (skip && skip[i]) continue;
    out_idx[k++] = (int64_t)b;
  }
  *out_n = k;
  return OR_OK;
}

/* lib.rs:636-679 (split: separate K and V regions, block i at i*segment) and
 * lib.rs:706-747 (contiguous: block i at i*block_size). */
int or_save_host_layout(const or_layout* reg, uint64_t n, uint64_t k_base,
                        uint64_t v_base, uint64_t* k_dst, uint64_t* v_dst) {
  int split = reg->segments == 2 && reg->kv_stride_bytes > reg->bytes_per_block;
  for (uint64_t i = 0; i < n; i++) {
    if (split) {
      k_dst[i] = k_base + i * reg->bytes_per_block;
      v_dst[i] = v_base + i * reg->bytes_per_block;
    } else {
      k_dst[i] = k_base + i * reg->block_size_bytes;
      v_dst[i] = 0;
    }
  }
  return split;
}

/* lib.rs:1032-1043: negative ids and missing slots are skipped. */
uint64_t or_plan_load(const int32_t* block_ids, const uint8_t* present,
                      uint64_t n, uint64_t* out_pos) {
  uint64_t k = 0;
  for (uint64_t i = 0; i < n; i++) {
    if (block_ids[i] < 0) continue;
    if (present && !present[i]) continue;
    out_pos[k++] = i;
  }
  return k;
}

/* gpu_worker.rs:321-372 with copy_block_gpu_to_cpu (transfer.rs:201-239).
 * The split path computes every offset before the first copy
 * (gpu_worker.rs:334-341); the per-block paths fail at the first bad block.
 * Either way an error means the reference returned Err and the caller drops
 * the destination, so the list is only produced when every offset is valid. */
uint64_t or_save_copies(const or_layout* reg, uint64_t dev,
                        const int64_t* block_idx, const uint64_t* k_dst,
                        const uint64_t* v_dst, uint64_t n, uint64_t* src,
                        uint64_t* dst, uint64_t* size, char* err,
                        size_t errlen) {
  const uint64_t seg = reg->bytes_per_block;
  uint64_t c = 0, off;
  int kind = or_layout_kind(reg);
  if (kind == OR_SPLIT) {
    for (uint64_t i = 0; i < n; i++) { /* K copies, gpu_worker.rs:344-349 */
      if (or_segment_offset(reg, (uint64_t)block_idx[i], 0, &off, err, errlen))
        return (uint64_t)-1;
      src[c] = dev + off; dst[c] = k_dst[i]; size[c] = seg; c++;
    }
    for (uint64_t i = 0; i < n; i++) { /* V copies, gpu_worker.rs:352-360 */
      if (or_segment_offset(reg, (uint64_t)block_idx[i], 1, &off, err, errlen))
        return (uint64_t)-1;
      uint64_t v = v_dst && v_dst[i] ? v_dst[i] : k_dst[i] + seg;
      src[c] = dev + off; dst[c] = v; size[c] = seg; c++;
    }
    return c;
  }
  for (uint64_t i = 0; i < n; i++) {
    if (kind == OR_CONTIGUOUS) { /* transfer.rs:206-210 */
      if (or_segment_offset(reg, (uint64_t)block_idx[i], 0, &off, err, errlen))
        return (uint64_t)-1;
      if (off + reg->block_size_bytes > reg->size_bytes) {
        set_err(err, errlen,
                "Block %llu exceeds registered memory (offset %llu, size %llu, "
                "limit %llu)",
                (unsigned long long)block_idx[i], (unsigned long long)off,
                (unsigned long long)reg->block_size_bytes,
                (unsigned long long)reg->size_bytes);
        return (uint64_t)-1;
      }
      src[c] = dev + off; dst[c] = k_dst[i]; size[c] = reg->block_size_bytes;
      c++;
    } else { /* transfer.rs:217-239 */
      for (uint64_t s = 0; s < reg->segments; s++) {
        if (or_segment_offset(reg, (uint64_t)block_idx[i], s, &off, err, errlen))
          return (uint64_t)-1;
        src[c] = dev + off; dst[c] = k_dst[i] + s * seg; size[c] = seg; c++;
      }
    }
  }
  return c;
}

/* gpu_worker.rs:211-283 with batch_copy_segments_to_gpu (transfer.rs:116-198).
 * For the non-split paths the reference copies block_size_bytes starting at
 * segment_offset(b, 0), which only bounds offset + bytes_per_block; a copy that
 * would run past size_bytes (possible only for a strided multi-segment layout)
 * is reported as an error here, where the reference would write out of
 * bounds. */
uint64_t or_load_copies(const or_layout* reg, uint64_t dev,
                        const int64_t* block_idx, const uint64_t* k_src,
                        const uint64_t* v_src, uint64_t n, uint64_t* src,
                        uint64_t* dst, uint64_t* size, char* err,
                        size_t errlen) {
  if (n == 0) return 0; /* gpu_worker.rs:214-216 */
  uint64_t c = 0;
  uint64_t* gpu = (uint64_t*)malloc(sizeof(uint64_t) * n * 2);
  uint64_t* cpu = (uint64_t*)malloc(sizeof(uint64_t) * n * 2);
  uint64_t* rs = (uint64_t*)malloc(sizeof(uint64_t) * n);
  uint64_t* rc = (uint64_t*)malloc(sizeof(uint64_t) * n);
  uint64_t result = (uint64_t)-1;
  const uint64_t seg = reg->bytes_per_block;
  if (or_layout_kind(reg) == OR_SPLIT) {
    for (uint64_t i = 0; i < n; i++) { /* gpu_worker.rs:226-240 */
      uint64_t ko, vo;
      if (or_segment_offset(reg, (uint64_t)block_idx[i], 0, &ko, err, errlen) ||
          or_segment_offset(reg, (uint64_t)block_idx[i], 1, &vo, err, errlen))
        goto done;
      gpu[i] = ko; cpu[i] = k_src[i];
      gpu[n + i] = vo;
      cpu[n + i] = v_src && v_src[i] ? v_src[i] : k_src[i] + seg;
    }
    for (int half = 0; half < 2; half++) { /* K batch, then V batch */
      uint64_t runs = or_merge_runs(gpu + half * n, cpu + half * n, n, seg, rs, rc);
      for (uint64_t r = 0; r < runs; r++) {
        uint64_t j = half * n + rs[r];
        src[c] = cpu[j]; dst[c] = dev + gpu[j]; size[c] = rc[r] * seg; c++;
      }
    }
  } else {
    const uint64_t bs = reg->block_size_bytes; /* gpu_worker.rs:262-272 */
    for (uint64_t i = 0; i < n; i++) {
      uint64_t off;
      if (or_segment_offset(reg, (uint64_t)block_idx[i], 0, &off, err, errlen))
        goto done;
      if (off + bs > reg->size_bytes) {
        set_err(err, errlen,
                "Block %llu exceeds registered memory (offset %llu, size %llu, "
                "limit %llu)",
                (unsigned long long)block_idx[i], (unsigned long long)off,
                (unsigned long long)bs, (unsigned long long)reg->size_bytes);
        goto done;
      }
      gpu[i] = off; cpu[i] = k_src[i];
    }
    uint64_t runs = or_merge_runs(gpu, cpu, n, bs, rs, rc);
    for (uint64_t r = 0; r < runs; r++) {
      uint64_t j = rs[r];
      src[c] = cpu[j]; dst[c] = dev + gpu[j]; size[c] = rc[r] * bs; c++;
    }
  }
  result = c;
done:
  free(gpu); free(cpu); free(rs); free(rc);
  return result;
}

typedef struct {
  const uint64_t *src, *dst, *size;
  uint64_t begin, end;
} copy_share;

static void* copy_worker(void* arg) {
  copy_share* s = (copy_share*)arg;
  for (uint64_t i = s->begin; i < s->end; i++)
    memcpy((void*)(uintptr_t)s->dst[i], (const void*)(uintptr_t)s->src[i],
           (size_t)s->size[i]);
  return NULL;
}

void or_run_copies(const uint64_t* src, const uint64_t* dst,
                   const uint64_t* size, uint64_t n, int nthreads) {
  if (nthreads <= 1 || n < 2) {
    copy_share s = {src, dst, size, 0, n};
    copy_worker(&s);
    return;
  }
  if ((uint64_t)nthreads > n) nthreads = (int)n;
  uint64_t total = 0;
  for (uint64_t i = 0; i < n; i++) total += size[i];
  copy_share* shares = (copy_share*)calloc((size_t)nthreads, sizeof(copy_share));
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  uint64_t i = 0, acc = 0;
  for (int t = 0; t < nthreads; t++) {
    uint64_t target = total / (uint64_t)nthreads * (uint64_t)(t + 1);
    shares[t].src = src; shares[t].dst = dst; shares[t].size = size;
    shares[t].begin = i;
    while (i < n && (acc < target || t == nthreads - 1)) acc += size[i++];
    shares[t].end = i;
  }
  for (int t = 1; t < nthreads; t++)
    pthread_create(&th[t], NULL, copy_worker, &shares[t]);
  copy_worker(&shares[0]);
  for (int t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
  free(shares);
  free(th);
}

int or_process_save(const or_layout* reg, uint64_t dev,
                    const int64_t* block_idx, const uint64_t* k_dst,
                    const uint64_t* v_dst, uint64_t n, char* err,
                    size_t errlen) {
  uint64_t cap = n * (reg->segments > 2 ? reg->segments : 2) + 1;
  uint64_t* src = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint64_t* dst = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint64_t* size = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint64_t c = or_save_copies(reg, dev, block_idx, k_dst, v_dst, n, src, dst,
                              size, err, errlen);
  int rc = OR_ERR;
  if (c != (uint64_t)-1) {
    or_run_copies(src, dst, size, c, 1);
    rc = OR_OK;
  }
  free(src); free(dst); free(size);
  return rc;
}

int or_process_load(const or_layout* reg, uint64_t dev,
                    const int64_t* block_idx, const uint64_t* k_src,
                    const uint64_t* v_src, uint64_t n, uint64_t* out_batches,
                    char* err, size_t errlen) {
  uint64_t cap = n * 2 + 1;
  uint64_t* src = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint64_t* dst = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint64_t* size = (uint64_t*)malloc(sizeof(uint64_t) * cap);
  uint64_t c = or_load_copies(reg, dev, block_idx, k_src, v_src, n, src, dst,
                              size, err, errlen);
  int rc = OR_ERR;
  if (c != (uint64_t)-1) {
    or_run_copies(src, dst, size, c, 1);
    if (out_batches) *out_batches = c;
    rc = OR_OK;
  }
  free(src); free(dst); free(size);
  return rc;
}

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

void or_fill_random(uint64_t dst, uint64_t size_bytes, uint64_t seed,
                    uint64_t word_offset) {
  uint64_t* w = (uint64_t*)(uintptr_t)dst;
  uint64_t n = size_bytes / 8;
  for (uint64_t i = 0; i < n; i++)
    w[i] = mix64(seed + (word_offset + i + 1) * 0x9E3779B97F4A7C15ULL);
}

/* write_packed_file, seal_offload.rs:397-441: per block, per slot, the K half
 * then the V half when the slot has a V pointer, else the whole slot. */
uint64_t or_pack_blocks(uint64_t n, uint64_t s, const uint64_t* k,
                        const uint64_t* v, const uint64_t* size, uint64_t out,
                        uint64_t* offs) {
  uint64_t off = 0;
  for (uint64_t b = 0; b < n; b++) {
    if (offs) offs[b] = off;
    for (uint64_t j = 0; j < s; j++) {
      const uint64_t i = b * s + j;
      if (v[i]) {
        const uint64_t half = size[i] / 2;
        if (out) {
          memcpy((uint8_t*)(uintptr_t)(out + off), (const void*)(uintptr_t)k[i], half);
          memcpy((uint8_t*)(uintptr_t)(out + off + half), (const void*)(uintptr_t)v[i], half);
        }
        off += 2 * half;
      } else {
        if (out) memcpy((uint8_t*)(uintptr_t)(out + off), (const void*)(uintptr_t)k[i], size[i]);
        off += size[i];
      }
    }
  }
  return off;
}

/* rebuild_sealed_block, seal_offload.rs:869-909. */
void or_unpack_block(uint64_t base, uint64_t s, const uint8_t* is_split,
                     const uint64_t* size, uint64_t* k, uint64_t* v) {
  uint64_t off = 0;
  for (uint64_t j = 0; j < s; j++) {
    k[j] = base + off;
    v[j] = is_split[j] ? base + off + size[j] / 2 : 0;
    off += size[j];
  }
}
