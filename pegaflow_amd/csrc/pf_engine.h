// pf_engine.h — internal declarations of the engine: pool allocator, pinned
// pool, block store, per-device workers and PegaEngine (the roles of
// pegaflow-core/src/{allocator,pinned_pool,storage,gpu_worker,lib}.rs).
#pragma once

#include <condition_variable>
#include <cstdint>
#include <deque>
#include <list>
#include <map>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "pf_common.h"

namespace pf {

// ---------------------------------------------------------------------------
// Byte allocator over a region, in fixed units (ScaledOffsetAllocator,
// allocator.rs:66-171): requests round up to whole units; free regions are
// kept by offset and coalesced with their neighbours on free; allocation is
// best fit (smallest free region that holds the request, lowest offset on
// ties).
// ---------------------------------------------------------------------------
class UnitAllocator {
 public:
  // unit_size 0 picks the smallest unit that keeps the unit count within
  // 32 bits, as the reference does (allocator.rs:77-97).
  static int create(uint64_t total_bytes, uint64_t unit_size,
                    std::unique_ptr<UnitAllocator>* out);
  // PF_OK with *found = false when no region fits; PF_ERR_INVALID_ARGUMENT
  // when the request cannot be expressed in 32-bit units.
  int allocate(uint64_t size_bytes, bool* found, uint64_t* offset, uint64_t* size);
  void free(uint64_t offset);
  uint64_t unit_size() const { return unit_; }
  uint64_t total_bytes() const { return total_units_ * unit_; }
  uint64_t free_bytes() const { return free_units_ * unit_; }
  uint64_t largest_free_bytes() const;

 private:
  uint64_t unit_ = 1;
  uint64_t total_units_ = 0;
  uint64_t free_units_ = 0;
  std::map<uint64_t, uint64_t> free_by_off_;            // offset -> units
  std::multimap<uint64_t, uint64_t> free_by_size_;      // units -> offset
  std::unordered_map<uint64_t, uint64_t> used_;         // offset -> units
  void insert_free(uint64_t off, uint64_t units);
  void erase_free(std::map<uint64_t, uint64_t>::iterator it);
};

// ---------------------------------------------------------------------------
// Pinned pool (PinnedMemoryPool, pinned_pool.rs:53-185): one backing region
// plus the allocator; allocations are returned by RAII handles.
// ---------------------------------------------------------------------------
class PinnedPool;

struct PoolAllocation {
  std::shared_ptr<PinnedPool> pool;
  uint64_t offset = 0;
  uint64_t size = 0;
  uint8_t* ptr = nullptr;
  ~PoolAllocation();
};

class PinnedPool : public std::enable_shared_from_this<PinnedPool> {
 public:
  // device_backed: hipHostMalloc (mapped) through pf_pinned_allocate;
  // otherwise ordinary host memory (planning and bookkeeping without a GPU).
  static int create(uint64_t size, uint64_t unit_hint, bool device_backed, uint32_t pinned_flags,
                    std::shared_ptr<PinnedPool>* out);
  ~PinnedPool();
  std::shared_ptr<PoolAllocation> allocate(uint64_t size);
  void release(uint64_t offset);
  void usage(uint64_t* used, uint64_t* total);
  uint64_t largest_free();
  bool device_backed() const { return device_backed_; }
  uint8_t* base() const { return base_; }

 private:
  uint8_t* base_ = nullptr;
  uint64_t size_ = 0;
  bool device_backed_ = false;
  std::mutex mu_;
  std::unique_ptr<UnitAllocator> alloc_;
};

// ---------------------------------------------------------------------------
// Block store (storage.rs:136-687, without TinyLFU admission).
// ---------------------------------------------------------------------------
// Host copy of one (block, slot): LayerBlock (storage.rs:249-310).
struct LayerBlock {
  uint8_t* k_ptr = nullptr;
  uint8_t* v_ptr = nullptr;  // null for the contiguous layout
  uint64_t size = 0;          // block_size_bytes
  std::shared_ptr<PoolAllocation> k_alloc;
  std::shared_ptr<PoolAllocation> v_alloc;
};

// All slots (layer x tp_rank) of one block hash, immutable once sealed.
struct SealedBlock {
  std::vector<std::shared_ptr<LayerBlock>> slots;
  uint64_t footprint = 0;
};

struct InflightBlock {
  std::vector<std::shared_ptr<LayerBlock>> slots;
  size_t remaining = 0;
  uint64_t footprint = 0;
};

class BlockStore {
 public:
  explicit BlockStore(std::shared_ptr<PinnedPool> pool) : pool_(std::move(pool)) {}
  // Allocation with eviction of least-recently-used sealed blocks in batches
  // of 64 until the largest free region fits (storage.rs:405-433).
  std::shared_ptr<PoolAllocation> allocate(uint64_t size);
  bool cache_contains(const std::string& key);
  bool inflight_has_slot(const std::string& key, size_t slot);
  // storage.rs:457-514.  Returns PF_OK and *inserted (false when sealed
  // already or the slot exists); errors on slot count mismatch / range.
  int insert_slot(const std::string& key, size_t slot, std::shared_ptr<LayerBlock> block,
                  size_t total_slots, bool* inserted);
  // storage.rs:529-547: every hash must be sealed; refreshes recency.
  int lookup_many(const std::vector<std::string>& keys,
                  std::vector<std::shared_ptr<SealedBlock>>* out);
  PinnedPool& pool() { return *pool_; }
  uint64_t sealed_count();
  uint64_t inflight_count();
  uint64_t evictions() const { return evictions_; }

 private:
  std::shared_ptr<PinnedPool> pool_;
  std::mutex inflight_mu_;
  std::unordered_map<std::string, InflightBlock> inflight_;
  std::mutex cache_mu_;
  std::list<std::string> lru_;  // front = most recent
  struct Entry {
    std::shared_ptr<SealedBlock> block;
    std::list<std::string>::iterator pos;
  };
  std::unordered_map<std::string, Entry> cache_;
  uint64_t evictions_ = 0;
  size_t evict_lru(size_t max_blocks);
};

}  // namespace pf
