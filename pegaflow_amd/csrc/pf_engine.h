// pf_engine.h — internal declarations of the engine: pool allocator, pinned
// pool, block store, per-device workers and PegaEngine (the roles of
// pegaflow-core/src/{allocator,pinned_pool,storage,gpu_worker,lib}.rs).
#pragma once

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <functional>
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
#include "pf_lfu.h"

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
// Block store (storage.rs:136-687; TinyLFU admission, cache.rs, opt-in).
// ---------------------------------------------------------------------------
// Host copy of one (block, slot): LayerBlock (storage.rs:249-310).
struct LayerBlock {
  uint8_t* k_ptr = nullptr;
  uint8_t* v_ptr = nullptr;  // null for the contiguous layout
  uint64_t size = 0;          // block_size_bytes
  std::shared_ptr<PoolAllocation> k_alloc;
  std::shared_ptr<PoolAllocation> v_alloc;
};

// One slot of a sealed block as a load reads it (size 0: no slot).
struct SlotView {
  const uint8_t* k_ptr = nullptr;
  const uint8_t* v_ptr = nullptr;
  uint64_t size = 0;
};

// All slots (layer x tp_rank) of one block hash, immutable once sealed.
// `views` repeats each slot's pointers and size in one contiguous array,
// built by index() when the block seals, so a load naming hundreds of blocks
// and dozens of layers reads them in order instead of chasing one pointer
// per (block, layer).
struct SealedBlock {
  std::vector<std::shared_ptr<LayerBlock>> slots;
  std::vector<SlotView> views;
  uint64_t footprint = 0;
  void index() {
    views.assign(slots.size(), SlotView{});
    for (size_t s = 0; s < slots.size(); ++s)
      if (slots[s]) views[s] = SlotView{slots[s]->k_ptr, slots[s]->v_ptr, slots[s]->size};
  }
};

struct InflightBlock {
  std::vector<std::shared_ptr<LayerBlock>> slots;
  size_t remaining = 0;
  uint64_t footprint = 0;
};

class BlockStore {
 public:
  using SealHook = std::function<void(const std::string&, const std::shared_ptr<SealedBlock>&)>;
  explicit BlockStore(std::shared_ptr<PinnedPool> pool) : pool_(std::move(pool)) {}
  // Called once per block as it seals (the seal notification of
  // storage.rs:495-504), outside the store's locks.  Set before any save.
  void set_seal_hook(SealHook h) { seal_hook_ = std::move(h); }
  // Inserts an already complete block (read back from disk) as the most
  // recently used entry; false when the key is present already.
  bool cache_insert(const std::string& key, std::shared_ptr<SealedBlock> block);
  // A sealed block without touching its recency (inspection).
  std::shared_ptr<SealedBlock> peek(const std::string& key);
  // Allocation with eviction of least-recently-used sealed blocks in batches
  // of 64 until the largest free region fits (storage.rs:405-433).  With the
  // cache empty it waits for memory that other threads' evictions are still
  // returning; null when the rest is held by loads and saves in progress.
  std::shared_ptr<PoolAllocation> allocate(uint64_t size);
  bool cache_contains(const std::string& key);
  // The layers of one save that share a hash list, with one lookup per key
  // in each map: keep[j][i] = 0 when keys[i] is sealed already or its slot
  // slots[j] is inflight (lib.rs:590-621).
  void filter_slots(const std::vector<std::string>& keys, const std::vector<size_t>& slots,
                    std::vector<std::vector<char>>* keep);
  // storage.rs:457-514 for those layers: entries[j] holds (key index, host
  // copy) for layer j, stored in slot slots[j].  Slots of sealed blocks and
  // filled slots are skipped; a block whose last slot arrives moves to the
  // cache and the seal hook runs for it.  Errors on slot count mismatch or
  // a slot out of range.
  using SlotEntries = std::vector<std::pair<uint32_t, std::shared_ptr<LayerBlock>>>;
  struct Entry {
    std::shared_ptr<SealedBlock> block;
    std::list<const std::string*>::iterator pos;
  };
  struct Prepared {
    // Complete blocks (key index, block), in the call's order.
    std::vector<std::pair<uint32_t, std::shared_ptr<SealedBlock>>> blocks;
    // Their cache nodes, made ahead of the lock by stage_nodes: the first
    // block of each key with its recency element (front = most recent).
    std::unordered_map<std::string, Entry> nodes;
    std::list<const std::string*> order;
    bool staged = false;
  };
  // When the call brings every slot of its blocks (entries[j] for slot
  // slots[j], all naming the same keys in the same order), the complete
  // blocks built from them, moving the layer blocks out of `entries`;
  // otherwise nothing.  Touches no state of the store, so it can run while
  // the copy is in flight.
  static Prepared prepare_whole(const std::vector<size_t>& slots,
                                std::vector<SlotEntries>& entries, size_t total_slots);
  // Makes the cache nodes of prepared blocks (key copies, hashing, the
  // recency elements), so that publishing them is a merge and a splice
  // under the lock.  Touches no state of the store.
  static void stage_nodes(const std::vector<std::string>& keys, Prepared* prepared);
  // Publishes the copies (moves them): blocks in `prepared` seal directly
  // unless an earlier call left part of them in flight.
  int insert_slots(const std::vector<std::string>& keys, const std::vector<size_t>& slots,
                   std::vector<SlotEntries>& entries, size_t total_slots,
                   Prepared* prepared = nullptr);
  // storage.rs:529-547: every hash must be sealed; refreshes recency.
  int lookup_many(const std::vector<std::string>& keys,
                  std::vector<std::shared_ptr<SealedBlock>>* out);
  PinnedPool& pool() { return *pool_; }
  uint64_t sealed_count();
  uint64_t inflight_count();
  uint64_t evictions() const { return evictions_.load(std::memory_order_relaxed); }
  // Evicts up to max_blocks least-recently-used sealed blocks; the count.
  size_t evict_lru(size_t max_blocks);
  // Evicts least-recently-used sealed blocks until their footprints add up
  // to `bytes` or the cache is empty (storage.rs:610-644); the count, and
  // the bytes in *freed.
  size_t evict_bytes(uint64_t bytes, uint64_t* freed);
  // TinyLFU admission (cache.rs:28-241) for a cache of `items` expected
  // entries, its sketch's row hashes seeded from `seed`; 0 items turns it
  // off (plain LRU inserts, the default here).  With it on, a newly sealed
  // block, or one read back from disk, is recorded and then refused when
  // its estimate is below that of the least recently used entry, and every
  // lookup hit is recorded.
  void set_admission(uint64_t items, uint64_t seed);
  uint64_t admission_rejections() const { return rejections_.load(std::memory_order_relaxed); }

 private:
  // Whether a key not in the cache enters it (caller holds cache_mu_).
  bool admit(const std::string& key);
  // Drops an eviction's blocks (their memory returns to the pool) and ends
  // its count in releasing_.
  void drop_evicted(std::vector<std::shared_ptr<SealedBlock>>* dropped);
  std::shared_ptr<PinnedPool> pool_;
  std::mutex inflight_mu_;
  std::unordered_map<std::string, InflightBlock> inflight_;
  std::mutex cache_mu_;
  // Recency order, front = most recent; each element points at its key in
  // cache_ (unordered_map nodes, hence keys, stay put until erased).
  std::list<const std::string*> lru_;
  std::unordered_map<std::string, Entry> cache_;
  std::atomic<uint64_t> evictions_{0};  // written under cache_mu_, read without it
  std::unique_ptr<TinyLfu> lfu_;        // under cache_mu_; null: admission off
  std::atomic<uint64_t> rejections_{0};  // written under cache_mu_
  // Evictions whose blocks are out of the cache but whose memory may not
  // be back in the pool yet (raised under cache_mu_).
  std::atomic<uint32_t> releasing_{0};
  SealHook seal_hook_;
};

// ---------------------------------------------------------------------------
// Disk tier (seal_offload.rs): sealed blocks are written in batches to packed
// files "<root>/<namespace>/<uuid>.bin" — per block, per slot, the K half
// then the V half (or the whole slot when contiguous) — and read back into
// the pinned pool when a prefix query misses.  The reference indexes blocks
// in Redis; here each packed file has a sidecar "<uuid>.json" listing its
// blocks with the reference's BlockMeta JSON, and the index is rebuilt from
// the sidecars when a tier opens an existing root.
// ---------------------------------------------------------------------------
struct DiskSlotMeta {
  bool is_split = false;
  uint64_t size = 0;  // K + V bytes of the slot
};

struct DiskBlockMeta {  // BlockMeta, seal_offload.rs:80-97
  std::string file;     // "<uuid>.bin"
  uint64_t offset = 0;  // byte offset of the block inside the file
  std::vector<DiskSlotMeta> slots;
  uint64_t total_slots = 0;
  uint64_t total_size() const {
    uint64_t s = 0;
    for (const auto& m : slots) s += m.size;
    return s;
  }
};

// serde_json's compact rendering of BlockMeta.
std::string block_meta_json(const DiskBlockMeta& m);

struct DiskConfig {
  std::string root;
  uint64_t quota_bytes = 50ull << 30;
  size_t max_pack_blocks = 64;   // seal_offload.rs:61-67
  size_t max_prefetch_tasks = 16;
  size_t io_threads = 4;  // writer threads and, as many again, reader threads
};

struct DiskStats {
  uint64_t files = 0, bytes = 0, indexed_blocks = 0;
  uint64_t offloaded_blocks = 0, written_bytes = 0;
  uint64_t prefetched_blocks = 0, read_bytes = 0;
  uint64_t pending_blocks = 0, evicted_files = 0, failures = 0;
};

enum PrefetchState : int { kPrefetchReady = 0, kPrefetchLoading = 1, kPrefetchPartialMiss = 2 };

class DiskTier {
 public:
  static int open(const DiskConfig& cfg, BlockStore* store, std::unique_ptr<DiskTier>* out);
  ~DiskTier();
  // Seal notification: queue the block for the writer threads.
  void on_seal(const std::string& key, const std::shared_ptr<SealedBlock>& block);
  // count_prefix_hit_blocks_async (lib.rs:855-941): cache hits, then blocks
  // being read, then — when the first miss is on disk — a background read of
  // the rest of the prefix.
  void query(const std::vector<std::string>& keys, int* state, uint64_t* ready,
             uint64_t* loading, uint64_t* missing);
  void flush();          // returns when every queued block is on disk
  void wait_prefetch();  // returns when no read is in flight
  DiskStats stats();
  static std::string dir_name(const std::string& ns);

 private:
  struct FileEntry {
    std::string ns_dir, uuid;
    std::vector<std::string> keys;
    uint64_t size = 0, seq = 0;
  };
  struct ReadJob {
    std::string path;
    std::vector<std::pair<std::string, DiskBlockMeta>> blocks;
    std::shared_ptr<std::atomic<size_t>> parts_left;
  };
  DiskConfig cfg_;
  BlockStore* store_ = nullptr;
  std::mutex mu_;  // index, files, pending, queues
  std::condition_variable write_cv_, read_cv_, idle_cv_;
  std::unordered_map<std::string, DiskBlockMeta> index_;
  std::map<std::string, FileEntry> files_;  // uuid -> entry
  std::map<uint64_t, std::string> by_age_;  // seq -> uuid
  uint64_t next_seq_ = 0, usage_ = 0;
  std::deque<std::pair<std::string, std::weak_ptr<SealedBlock>>> write_q_;
  size_t writing_ = 0;
  std::unordered_map<std::string, int> pending_;
  std::deque<ReadJob> read_q_;
  size_t active_tasks_ = 0, reading_ = 0;
  bool stop_ = false;
  DiskStats st_;
  std::vector<std::thread> writers_;
  std::vector<std::thread> readers_;

  void rescan();
  void writer_loop();
  void reader_loop();
  int write_packed(const std::string& ns_dir,
                   const std::vector<std::pair<std::string, std::shared_ptr<SealedBlock>>>& blocks);
  void enforce_quota_locked();
  void read_job(ReadJob& job);
};

}  // namespace pf
