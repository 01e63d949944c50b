/*
 * pf_oracle.h — CPU restatement of PegaFlow's KV-block transfer path.
 *
 * TEST INFRASTRUCTURE ONLY.  The HIP product path is tested against this
 * oracle, and it is the CPU baseline timed beside it.  Only tests/, the smoke check and
 * the benchmark's CPU-baseline leg may load it; the product never does.
 *
 * Every function restates one piece of the reference (xiaguan/pegaflow) with
 * host memcpy standing in for the cuMemcpy* DMA calls.  Addresses are plain
 * host addresses carried as uint64_t.
 */
#ifndef PF_ORACLE_H
#define PF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KVCacheRegistration, pegaflow-core/src/lib.rs:100-112. */
typedef struct or_layout {
  uint64_t data_ptr;
  uint64_t size_bytes;
  uint64_t num_blocks;
  uint64_t bytes_per_block;
  uint64_t block_size_bytes;
  uint64_t kv_stride_bytes;
  uint64_t segments;
} or_layout;

enum { OR_OK = 0, OR_ERR = 1 };
enum { OR_SPLIT = 0, OR_CONTIGUOUS = 1, OR_STRIDED = 2 };

/* register_context_layer validation, lib.rs:389-449. */
int or_layout_init(uint64_t data_ptr, uint64_t size_bytes, uint64_t num_blocks,
                   uint64_t bytes_per_block, uint64_t kv_stride_bytes,
                   uint64_t segments, or_layout* out, char* err,
                   size_t errlen);

/* segment_offset, transfer.rs:18-47. */
int or_segment_offset(const or_layout* reg, uint64_t block_idx,
                      uint64_t segment_idx, uint64_t* out, char* err,
                      size_t errlen);

/* is_contiguous_layout, transfer.rs:50-52. */
int or_is_contiguous(const or_layout* reg);

/* Dispatch of gpu_worker.rs:218 / 326 (split) and transfer.rs:206 (contiguous). */
int or_layout_kind(const or_layout* reg);

/* Greedy run merging of batch_copy_segments_to_gpu, transfer.rs:134-177.
 * Writes (start index, count) per run; returns the number of runs. */
uint64_t or_merge_runs(const uint64_t* gpu_off, const uint64_t* cpu_addr,
                       uint64_t n, uint64_t seg, uint64_t* run_start,
                       uint64_t* run_count);

/* Save filtering, lib.rs:590-621: skips block_id < 0 and entries whose
 * skip[i] is non-zero (hash already sealed or slot inflight, lib.rs:613-620);
 * block_id >= num_blocks is an error (lib.rs:598-603).  Writes the kept block
 * indices in order; *out_n receives their count. */
int or_plan_save(const or_layout* reg, const int32_t* block_ids, uint64_t n,
                 const uint8_t* skip, int64_t* out_idx, uint64_t* out_n,
                 char* err, size_t errlen);

/* Host destinations of a save batch of n kept blocks, lib.rs:636-747:
 * split layout -> k_dst[i] = k_base + i*seg, v_dst[i] = v_base + i*seg;
 * otherwise     -> k_dst[i] = k_base + i*block_size_bytes, v_dst[i] = 0.
 * Returns 1 when the split layout was used. */
int or_save_host_layout(const or_layout* reg, uint64_t n, uint64_t k_base,
                        uint64_t v_base, uint64_t* k_dst, uint64_t* v_dst);

/* Load filtering, lib.rs:1032-1043: keeps entries with block_id >= 0 whose
 * slot is present (present[i] != 0).  Writes kept positions into out_pos. */
uint64_t or_plan_load(const int32_t* block_ids, const uint8_t* present,
                      uint64_t n, uint64_t* out_pos);

/* The copy list a save task issues (gpu_worker.rs:321-372 with
 * transfer.rs:201-239): one entry per cuMemcpyDtoH call, in call order.
 * dev is the host copy of the layer tensor (the data_ptr it stands for is
 * replaced by dev).  Capacity of the out arrays: n * segments.
 * Returns the number of copies or (uint64_t)-1 on error. */
uint64_t or_save_copies(const or_layout* reg, uint64_t dev,
                        const int64_t* block_idx, const uint64_t* k_dst,
                        const uint64_t* v_dst, uint64_t n, uint64_t* src,
                        uint64_t* dst, uint64_t* size, char* err,
                        size_t errlen);

/* The copy list a load task issues (gpu_worker.rs:211-283 with
 * transfer.rs:116-198): one entry per merged cuMemcpyHtoDAsync run, K runs
 * before V runs.  Capacity: n * 2.  Returns the count or (uint64_t)-1. */
uint64_t or_load_copies(const or_layout* reg, uint64_t dev,
                        const int64_t* block_idx, const uint64_t* k_src,
                        const uint64_t* v_src, uint64_t n, uint64_t* src,
                        uint64_t* dst, uint64_t* size, char* err,
                        size_t errlen);

/* Executes a copy list with memcpy on nthreads threads (copies split into
 * nthreads contiguous shares of roughly equal bytes). */
void or_run_copies(const uint64_t* src, const uint64_t* dst,
                   const uint64_t* size, uint64_t n, int nthreads);

/* process_save_task / process_load_task on host memory, single thread. */
int or_process_save(const or_layout* reg, uint64_t dev,
                    const int64_t* block_idx, const uint64_t* k_dst,
                    const uint64_t* v_dst, uint64_t n, char* err,
                    size_t errlen);
int or_process_load(const or_layout* reg, uint64_t dev,
                    const int64_t* block_idx, const uint64_t* k_src,
                    const uint64_t* v_src, uint64_t n, uint64_t* out_batches,
                    char* err, size_t errlen);

/* Synthetic contents: word[i] = mix64(seed + (word_offset+i+1)*0x9E3779B97F4A7C15),
 * mix64 being the splitmix64 finaliser.  size_bytes must be a multiple of 8. */
void or_fill_random(uint64_t dst, uint64_t size_bytes, uint64_t seed,
                    uint64_t word_offset);

/* Packed block file (seal_offload.rs:379-448): n blocks of s slots each,
 * slot j of block b described by k[b*s+j], v[b*s+j] (0 for a contiguous
 * slot) and size[b*s+j] (K + V bytes).  Writes the file bytes to out (NULL:
 * size only) and returns the total size; the block offsets go to offs[n]. */
uint64_t or_pack_blocks(uint64_t n, uint64_t s, const uint64_t* k,
                        const uint64_t* v, const uint64_t* size, uint64_t out,
                        uint64_t* offs);
/* rebuild_sealed_block (seal_offload.rs:869-909): the K/V addresses of the s
 * slots of one block read to address base. */
void or_unpack_block(uint64_t base, uint64_t s, const uint8_t* is_split,
                     const uint64_t* size, uint64_t* k, uint64_t* v);

#ifdef __cplusplus
}
#endif

#endif /* PF_ORACLE_H */
