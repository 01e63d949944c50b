// pf_layout.cpp — error reporting and the layout arithmetic of the transfer
// path (KVCacheRegistration, segment_offset, is_contiguous_layout).
#include <cstdarg>
#include <cstdio>

#include "pf_common.h"

namespace pf {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

std::string strf(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return std::string(buf);
}

int hip_fail(hipError_t e, const char* what) {
  return fail(PF_ERR_HIP, strf("%s failed: %s (%d)", what, hipGetErrorString(e),
                               static_cast<int>(e)));
}

// transfer.rs:18-47.  The reference leaves `offset + bytes_per_block`
// unchecked; an overflow there is reported as exceeding the limit.
int segment_offset(const pf_kv_layout& l, uint64_t block, uint64_t seg,
                   uint64_t* out) {
  if (seg >= l.segments) return fail(PF_ERR_STORAGE, "Segment index out of range");
  uint64_t base, seg_off, offset, end;
  if (__builtin_mul_overflow(block, l.bytes_per_block, &base))
    return fail(PF_ERR_STORAGE, "Block offset overflow");
  if (__builtin_mul_overflow(seg, l.kv_stride_bytes, &seg_off))
    return fail(PF_ERR_STORAGE, "Segment offset overflow");
  if (__builtin_add_overflow(base, seg_off, &offset))
    return fail(PF_ERR_STORAGE, "Combined offset overflow");
  if (__builtin_add_overflow(offset, l.bytes_per_block, &end) ||
      end > l.size_bytes)
    return fail(PF_ERR_STORAGE,
                strf("Block %llu segment %llu exceeds registered memory "
                     "(offset %llu, size %llu, limit %llu)",
                     (unsigned long long)block, (unsigned long long)seg,
                     (unsigned long long)offset,
                     (unsigned long long)l.bytes_per_block,
                     (unsigned long long)l.size_bytes));
  *out = offset;
  return PF_OK;
}

}  // namespace pf

using namespace pf;

extern "C" {

const char* pf_last_error(void) { return g_last_error.c_str(); }

const char* pf_version(void) { return "pegaflow_hip 0.1.0 (gfx950)"; }

// register_context_layer's layout checks (lib.rs:389-449) and the
// KVCacheRegistration they build (lib.rs:457-465).
int pf_layout_init(uint64_t data_ptr, uint64_t size_bytes, uint64_t num_blocks,
                   uint64_t bytes_per_block, uint64_t kv_stride_bytes,
                   uint64_t segments, pf_kv_layout* out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "null layout");
  if (bytes_per_block == 0 || num_blocks == 0 || segments == 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "invalid KV cache layout");
  if (segments > 1 && kv_stride_bytes == 0)
    return fail(PF_ERR_INVALID_ARGUMENT,
                "kv_stride_bytes must be > 0 when segments > 1");
  uint64_t block_size, max_block_offset, max_segment_offset, max_offset, end;
  if (__builtin_mul_overflow(bytes_per_block, segments, &block_size))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("block size overflow: bytes_per_block=%llu segments=%llu",
                     (unsigned long long)bytes_per_block,
                     (unsigned long long)segments));
  if (__builtin_mul_overflow(num_blocks - 1, bytes_per_block, &max_block_offset))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("num_blocks %llu too large", (unsigned long long)num_blocks));
  if (__builtin_mul_overflow(segments - 1, kv_stride_bytes, &max_segment_offset))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("segments/stride overflow (segments=%llu, stride=%llu)",
                     (unsigned long long)segments,
                     (unsigned long long)kv_stride_bytes));
  if (__builtin_add_overflow(max_block_offset, max_segment_offset, &max_offset))
    return fail(PF_ERR_INVALID_ARGUMENT, "layout offset overflow");
  if (__builtin_add_overflow(max_offset, bytes_per_block, &end))
    return fail(PF_ERR_INVALID_ARGUMENT, "layout end overflow");
  if (end > size_bytes)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("registered memory too small: need at least %llu bytes, "
                     "got %llu",
                     (unsigned long long)end, (unsigned long long)size_bytes));
  out->data_ptr = data_ptr;
  out->size_bytes = size_bytes;
  out->num_blocks = num_blocks;
  out->bytes_per_block = bytes_per_block;
  out->block_size_bytes = block_size;
  out->kv_stride_bytes = kv_stride_bytes;
  out->segments = segments;
  return PF_OK;
}

int pf_segment_offset(const pf_kv_layout* layout, uint64_t block_idx,
                      uint64_t segment_idx, uint64_t* out_offset) {
  if (!layout || !out_offset) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  return segment_offset(*layout, block_idx, segment_idx, out_offset);
}

int pf_is_contiguous_layout(const pf_kv_layout* layout) {
  if (!layout) {
    fail(PF_ERR_INVALID_ARGUMENT, "null layout");
    return 0;
  }
  return layout->segments <= 1 ||
         layout->kv_stride_bytes == layout->bytes_per_block;
}

int pf_layout_kind(const pf_kv_layout* layout) {
  if (!layout) return fail(PF_ERR_INVALID_ARGUMENT, "null layout"), -1;
  return layout_kind(*layout);
}

// transfer.rs:134-177: a run grows while both the device offset and the host
// address continue exactly `segment_size` past the run's start.
uint64_t pf_count_merged_runs(const uint64_t* gpu_offsets,
                              const uint64_t* cpu_ptrs, uint64_t count,
                              uint64_t segment_size) {
  uint64_t runs = 0, i = 0;
  while (i < count) {
    uint64_t n = 1;
    while (i + n < count && gpu_offsets[i + n] == gpu_offsets[i] + n * segment_size &&
           cpu_ptrs[i + n] == cpu_ptrs[i] + n * segment_size)
      ++n;
    ++runs;
    i += n;
  }
  return runs;
}

}  // extern "C"
