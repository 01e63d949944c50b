// pf_engine.cpp — PegaEngine: instances and layer registrations, the pinned
// block store, and per-device save/load workers (the roles of
// pegaflow-core/src/{lib,storage,pinned_pool,allocator,gpu_worker}.rs).
//
// Save by hash: planning follows lib.rs:553-782 layer by layer (filtering,
// dedup against sealed and inflight blocks, the split K/V host layout), but
// all layers of a batch are then copied by one batched transfer
// (pf_save_layers) instead of one synchronous DMA per segment.
// Load by hash: lib.rs:957-1069; the device worker runs the transfer and, for
// a layered LoadState, publishes progress as layers land (one event per layer).
#include "pf_engine.h"

#include <sys/prctl.h>
#include <sys/resource.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <set>

namespace pf {

bool tracing() {
  static const bool on = [] {
    const char* v = std::getenv("PEGAFLOW_TRACE");
    return v && *v && std::strcmp(v, "0") != 0;
  }();
  return on;
}

double mono_us(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double, std::micro>(t.time_since_epoch()).count();
}

long thread_minor_faults() {
  struct rusage ru {};
  return getrusage(RUSAGE_THREAD, &ru) == 0 ? ru.ru_minflt : 0;
}

namespace {
double us_between(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
  return std::chrono::duration<double, std::micro>(b - a).count();
}

}  // namespace

// ===========================================================================
// UnitAllocator
// ===========================================================================
namespace {
constexpr uint64_t kU32Max = 0xffffffffull;
}

int UnitAllocator::create(uint64_t total_bytes, uint64_t unit_size,
                          std::unique_ptr<UnitAllocator>* out) {
  if (unit_size == 0) return fail(PF_ERR_INVALID_ARGUMENT, "unit size must be greater than zero");
  const uint64_t units = total_bytes / unit_size + (total_bytes % unit_size != 0);
  if (units > kU32Max)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("capacity %llu bytes with unit %llu overflows u32 backing allocator",
                     (unsigned long long)total_bytes, (unsigned long long)unit_size));
  auto a = std::unique_ptr<UnitAllocator>(new UnitAllocator());
  a->unit_ = unit_size;
  a->total_units_ = units;
  a->free_units_ = 0;
  if (units) a->insert_free(0, units);
  *out = std::move(a);
  return PF_OK;
}

void UnitAllocator::insert_free(uint64_t off, uint64_t units) {
  free_by_off_[off] = units;
  free_by_size_.insert({units, off});
  free_units_ += units;
}

void UnitAllocator::erase_free(std::map<uint64_t, uint64_t>::iterator it) {
  auto range = free_by_size_.equal_range(it->second);
  for (auto s = range.first; s != range.second; ++s)
    if (s->second == it->first) {
      free_by_size_.erase(s);
      break;
    }
  free_units_ -= it->second;
  free_by_off_.erase(it);
}

int UnitAllocator::allocate(uint64_t size_bytes, bool* found, uint64_t* offset, uint64_t* size) {
  *found = false;
  if (size_bytes == 0) return PF_OK;
  const uint64_t units = size_bytes / unit_ + (size_bytes % unit_ != 0);
  if (units > kU32Max)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("request %llu bytes with unit %llu overflows u32 backing allocator",
                     (unsigned long long)size_bytes, (unsigned long long)unit_));
  // Best fit; among regions of the best size, the lowest offset.
  auto s = free_by_size_.lower_bound(units);
  if (s == free_by_size_.end()) return PF_OK;
  uint64_t best_units = s->first, best_off = s->second;
  for (auto t = s; t != free_by_size_.end() && t->first == best_units; ++t)
    best_off = std::min(best_off, t->second);
  erase_free(free_by_off_.find(best_off));
  if (best_units > units) insert_free(best_off + units, best_units - units);
  used_[best_off] = units;
  *found = true;
  *offset = best_off * unit_;
  *size = units * unit_;
  return PF_OK;
}

void UnitAllocator::free(uint64_t offset_bytes) {
  const uint64_t off = offset_bytes / unit_;
  auto u = used_.find(off);
  if (u == used_.end()) return;
  uint64_t start = off, units = u->second;
  used_.erase(u);
  auto next = free_by_off_.find(start + units);
  if (next != free_by_off_.end()) {
    units += next->second;
    erase_free(next);
  }
  auto prev = free_by_off_.lower_bound(start);
  if (prev != free_by_off_.begin()) {
    --prev;
    if (prev->first + prev->second == start) {
      start = prev->first;
      units += prev->second;
      erase_free(prev);
    }
  }
  insert_free(start, units);
}

uint64_t UnitAllocator::largest_free_bytes() const {
  return free_by_size_.empty() ? 0 : free_by_size_.rbegin()->first * unit_;
}

// ===========================================================================
// PinnedPool
// ===========================================================================
PoolAllocation::~PoolAllocation() {
  if (pool) pool->release(offset);
}

int PinnedPool::create(uint64_t size, uint64_t unit_hint, bool device_backed,
                       uint32_t pinned_flags, std::shared_ptr<PinnedPool>* out) {
  if (size == 0) return fail(PF_ERR_ZERO_SIZE, "Pinned memory pool size must be greater than zero");
  // Units: the reference picks the smallest unit keeping 32-bit unit counts
  // (or the value-size hint).  Here units are also at least 256 bytes so
  // every block region starts 16-byte aligned for the vector kernels.
  uint64_t unit = unit_hint ? unit_hint : (size > kU32Max ? (size + kU32Max - 1) / kU32Max : 1);
  unit = std::max<uint64_t>(256, (unit + 255) / 256 * 256);
  std::unique_ptr<UnitAllocator> alloc;
  if (int rc = UnitAllocator::create(size, unit, &alloc)) return rc;
  auto p = std::shared_ptr<PinnedPool>(new PinnedPool());
  p->size_ = alloc->total_bytes();
  p->device_backed_ = device_backed;
  if (device_backed) {
    void* host = nullptr;
    uint64_t dev = 0;
    if (int rc = pf_pinned_allocate(p->size_, pinned_flags, &host, &dev)) return rc;
    p->base_ = static_cast<uint8_t*>(host);
  } else {
    const uint64_t rounded = (p->size_ + 4095) / 4096 * 4096;
    p->base_ = static_cast<uint8_t*>(std::aligned_alloc(4096, rounded));
    if (!p->base_) return fail(PF_ERR_STORAGE, "host pool allocation failed");
  }
  p->alloc_ = std::move(alloc);
  *out = std::move(p);
  return PF_OK;
}

PinnedPool::~PinnedPool() {
  if (!base_) return;
  if (device_backed_)
    pf_pinned_free(base_);
  else
    std::free(base_);
}

std::shared_ptr<PoolAllocation> PinnedPool::allocate(uint64_t size) {
  bool found = false;
  uint64_t off = 0, got = 0;
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (alloc_->allocate(size, &found, &off, &got) != PF_OK || !found) return nullptr;
  }
  auto a = std::make_shared<PoolAllocation>();
  a->pool = shared_from_this();
  a->offset = off;
  a->size = got;
  a->ptr = base_ + off;
  return a;
}

void PinnedPool::release(uint64_t offset) {
  std::lock_guard<std::mutex> lk(mu_);
  alloc_->free(offset);
}

void PinnedPool::usage(uint64_t* used, uint64_t* total) {
  std::lock_guard<std::mutex> lk(mu_);
  *total = alloc_->total_bytes();
  *used = *total - alloc_->free_bytes();
}

uint64_t PinnedPool::largest_free() {
  std::lock_guard<std::mutex> lk(mu_);
  return alloc_->largest_free_bytes();
}

// ===========================================================================
// BlockStore
// ===========================================================================
namespace {
constexpr size_t kReclaimBatch = 64;  // storage.rs:41
// Value size assumed by TinyLFU's sizing when no hint is given (cache.rs:14).
constexpr uint64_t kLfuDefaultValueBytes = 128ull << 20;
}

// Evicted blocks return their memory to the pool as their handles drop,
// after the cache lock is released.  Until then `releasing_` counts the
// eviction, so an allocation that finds the cache empty meanwhile waits for
// that memory instead of reporting the pool exhausted.
void BlockStore::drop_evicted(std::vector<std::shared_ptr<SealedBlock>>* dropped) {
  if (dropped->empty()) return;
  dropped->clear();
  releasing_.fetch_sub(1, std::memory_order_release);
}

size_t BlockStore::evict_lru(size_t max_blocks) {
  std::vector<std::shared_ptr<SealedBlock>> dropped;
  {
    std::lock_guard<std::mutex> lk(cache_mu_);
    while (dropped.size() < max_blocks && !lru_.empty()) {
      auto it = cache_.find(*lru_.back());
      lru_.pop_back();
      dropped.push_back(std::move(it->second.block));
      cache_.erase(it);
    }
    evictions_ += dropped.size();
    if (!dropped.empty()) releasing_.fetch_add(1, std::memory_order_relaxed);
  }
  const size_t n = dropped.size();
  drop_evicted(&dropped);
  return n;
}

size_t BlockStore::evict_bytes(uint64_t bytes, uint64_t* freed) {
  std::vector<std::shared_ptr<SealedBlock>> dropped;
  uint64_t total = 0;
  {
    std::lock_guard<std::mutex> lk(cache_mu_);
    while (total < bytes && !lru_.empty()) {
      auto it = cache_.find(*lru_.back());
      lru_.pop_back();
      total += it->second.block->footprint;
      dropped.push_back(std::move(it->second.block));
      cache_.erase(it);
    }
    evictions_ += dropped.size();
    if (!dropped.empty()) releasing_.fetch_add(1, std::memory_order_relaxed);
  }
  const size_t n = dropped.size();
  drop_evicted(&dropped);
  if (freed) *freed = total;
  return n;
}

void BlockStore::set_admission(uint64_t items, uint64_t seed) {
  std::lock_guard<std::mutex> lk(cache_mu_);
  lfu_.reset(items ? new TinyLfu(items, seed) : nullptr);
}

// cache.rs:71-95: the key is recorded whatever the outcome, then refused
// when it is colder than the least recently used entry.
bool BlockStore::admit(const std::string& key) {
  if (!lfu_) return true;
  lfu_->incr(key);
  if (!lru_.empty() && lfu_->get(key) < lfu_->get(*lru_.back())) {
    ++rejections_;
    return false;
  }
  return true;
}

std::shared_ptr<PoolAllocation> BlockStore::allocate(uint64_t size) {
  for (;;) {
    if (auto a = pool_->allocate(size)) return a;
    uint64_t largest = pool_->largest_free();
    while (largest < size) {
      if (evict_lru(kReclaimBatch) == 0) break;
      largest = pool_->largest_free();
    }
    if (largest >= size) continue;
    // The cache is empty.  Another thread's eviction (the pre-eviction
    // monitor, another save) may still be returning memory: wait for it.
    // Once none is, whatever they returned is visible to one more attempt;
    // memory still taken is held by loads or saves in progress.
    if (releasing_.load(std::memory_order_acquire) > 0) {
      std::this_thread::yield();
      continue;
    }
    return pool_->allocate(size);
  }
}

bool BlockStore::cache_contains(const std::string& key) {
  std::lock_guard<std::mutex> lk(cache_mu_);
  return cache_.count(key) != 0;
}

void BlockStore::filter_slots(const std::vector<std::string>& keys,
                              const std::vector<size_t>& slots,
                              std::vector<std::vector<char>>* keep) {
  const size_t n = keys.size();
  std::vector<char> sealed(n, 0);
  {
    std::lock_guard<std::mutex> lk(cache_mu_);
    for (size_t i = 0; i < n; ++i) sealed[i] = cache_.count(keys[i]) != 0;
  }
  keep->assign(slots.size(), std::vector<char>(n, 1));
  std::lock_guard<std::mutex> lk(inflight_mu_);
  const bool none_inflight = inflight_.empty();  // the common case: no lookups
  for (size_t i = 0; i < n; ++i) {
    if (sealed[i]) {
      for (auto& k : *keep) k[i] = 0;
      continue;
    }
    if (none_inflight) continue;
    auto it = inflight_.find(keys[i]);
    if (it == inflight_.end()) continue;
    const auto& filled = it->second.slots;
    for (size_t j = 0; j < slots.size(); ++j)
      if (slots[j] < filled.size() && filled[slots[j]]) (*keep)[j][i] = 0;
  }
}

BlockStore::Prepared BlockStore::prepare_whole(const std::vector<size_t>& slots,
                                               std::vector<SlotEntries>& entries,
                                               size_t total_slots) {
  Prepared out;
  bool whole = total_slots > 0 && entries.size() == total_slots && slots.size() == total_slots;
  if (whole) {
    std::vector<char> seen(total_slots, 0);
    for (size_t sl : slots) {
      if (sl >= total_slots || seen[sl]) {
        whole = false;
        break;
      }
      seen[sl] = 1;
    }
  }
  for (size_t j = 1; whole && j < entries.size(); ++j) {
    whole = entries[j].size() == entries[0].size();
    for (size_t k = 0; whole && k < entries[j].size(); ++k)
      whole = entries[j][k].first == entries[0][k].first;
  }
  if (!whole) return out;
  out.blocks.reserve(entries[0].size());
  for (size_t k = 0; k < entries[0].size(); ++k) {
    auto sb = std::make_shared<SealedBlock>();
    sb->slots.resize(total_slots);
    for (size_t j = 0; j < entries.size(); ++j) {
      sb->footprint += entries[j][k].second->size;
      sb->slots[slots[j]] = std::move(entries[j][k].second);  // leaves it empty
    }
    sb->index();
    out.blocks.emplace_back(entries[0][k].first, std::move(sb));
  }
  return out;
}

void BlockStore::stage_nodes(const std::vector<std::string>& keys, Prepared* p) {
  p->nodes.reserve(p->blocks.size());
  for (const auto& b : p->blocks) {
    auto ins = p->nodes.try_emplace(keys[b.first]);
    if (!ins.second) continue;  // a key named twice keeps its first block
    p->order.push_front(&ins.first->first);
    ins.first->second = Entry{b.second, p->order.begin()};
  }
  p->staged = true;
}

int BlockStore::insert_slots(const std::vector<std::string>& keys,
                             const std::vector<size_t>& slots, std::vector<SlotEntries>& entries,
                             size_t total_slots, Prepared* prepared) {
  Prepared own;
  if (!prepared) {
    own = prepare_whole(slots, entries, total_slots);
    prepared = &own;
  }
  const size_t n = keys.size();
  // Keys sealed before this call, among those of the slot entries (each key
  // looked up once, not once per layer that carries it).  Complete blocks
  // need no lookup here: the cache insert below skips a key sealed
  // meanwhile.
  std::vector<char> sealed_already(n, 0), named(n, 0);
  bool any_named = false;
  for (const auto& layer : entries)
    for (const auto& e : layer)
      if (e.second) named[e.first] = any_named = true;  // not moved into a complete block
  if (any_named) {
    std::lock_guard<std::mutex> lk(cache_mu_);
    for (size_t i = 0; i < n; ++i)
      if (named[i]) sealed_already[i] = cache_.count(keys[i]) != 0;
  }
  std::vector<std::pair<uint32_t, std::shared_ptr<SealedBlock>>> sealed;
  int err = PF_OK;
  size_t n_direct = 0;  // sealed[0, n_direct): complete blocks that never entered the inflight map
  {
    std::lock_guard<std::mutex> lk(inflight_mu_);
    // Complete blocks seal directly, unless an earlier call left part of
    // the block in flight: then its slots go back to the general path.
    const bool none_inflight = inflight_.empty();
    for (auto& p : prepared->blocks) {
      const uint32_t i = p.first;
      if (!none_inflight && inflight_.count(keys[i])) {
        for (size_t j = 0; j < entries.size(); ++j)
          entries[j].emplace_back(i, std::move(p.second->slots[slots[j]]));
        if (prepared->staged) {  // its staged node, if it is the key's, goes too
          auto it = prepared->nodes.find(keys[i]);
          if (it != prepared->nodes.end() && it->second.block == p.second) {
            prepared->order.erase(it->second.pos);
            prepared->nodes.erase(it);
          }
        }
        continue;
      }
      sealed.emplace_back(i, std::move(p.second));
    }
    prepared->blocks.clear();
    n_direct = sealed.size();
    std::vector<InflightBlock*> ib(n, nullptr);  // node pointers survive inserts
    int rc = PF_OK;
    for (size_t j = 0; j < entries.size() && rc == PF_OK; ++j) {
      const size_t slot = slots[j];
      for (auto& e : entries[j]) {
        const uint32_t i = e.first;
        if (sealed_already[i] || !e.second) continue;  // sealed above, or nothing
        if (!ib[i]) {
          auto it = inflight_.find(keys[i]);
          if (it == inflight_.end()) {
            InflightBlock fresh;
            fresh.slots.resize(total_slots);
            fresh.remaining = total_slots;
            it = inflight_.emplace(keys[i], std::move(fresh)).first;
          }
          ib[i] = &it->second;
        }
        InflightBlock& b = *ib[i];
        if (b.remaining == 0) continue;  // sealed earlier in this call
        if (slot < b.slots.size() && b.slots[slot]) continue;
        if (total_slots != b.slots.size()) {
          rc = fail(PF_ERR_STORAGE, strf("slot count mismatch: expected %zu, got %zu",
                                         b.slots.size(), total_slots));
          break;
        }
        if (slot >= b.slots.size()) {
          rc = fail(PF_ERR_STORAGE,
                    strf("slot_id %zu out of bounds (%zu slots)", slot, b.slots.size()));
          break;
        }
        b.footprint += e.second->size;
        b.slots[slot] = std::move(e.second);
        if (--b.remaining == 0) {
          auto sb = std::make_shared<SealedBlock>();
          sb->slots = std::move(b.slots);
          sb->footprint = b.footprint;
          sb->index();
          sealed.emplace_back(i, std::move(sb));
        }
      }
    }
    for (size_t k = n_direct; k < sealed.size(); ++k) inflight_.erase(keys[sealed[k].first]);
    if (rc != PF_OK && sealed.empty()) return rc;
    if (rc != PF_OK) err = rc;  // blocks completed before the error still seal
  }
  if (sealed.empty()) return PF_OK;
  std::vector<char> fresh(sealed.size(), 0);
  {
    std::lock_guard<std::mutex> lk(cache_mu_);
    size_t k = 0;
    if (prepared->staged && !lfu_) {
      // The complete blocks' nodes move in whole (no allocation or hashing
      // under the lock); those whose key was sealed meanwhile stay behind.
      // With admission on, every block goes through it, in order, below.
      cache_.merge(prepared->nodes);
      for (auto& left : prepared->nodes) prepared->order.erase(left.second.pos);
      lru_.splice(lru_.begin(), prepared->order);
      if (seal_hook_)
        for (; k < n_direct; ++k) {
          auto it = cache_.find(keys[sealed[k].first]);
          fresh[k] = it != cache_.end() && it->second.block == sealed[k].second;
        }
      k = n_direct;
    }
    // A key named twice in the call is offered once (its first block), as
    // the reference skips the second occurrence's slots before its cache.
    std::vector<char> offered;
    if (lfu_) offered.assign(n, 0);
    for (; k < sealed.size(); ++k) {
      const std::string& key = keys[sealed[k].first];
      if (lfu_) {
        if (offered[sealed[k].first] || cache_.count(key)) continue;
        offered[sealed[k].first] = 1;
        if (!admit(key)) continue;
      }
      auto ins = cache_.try_emplace(key);
      if (!ins.second) continue;  // sealed already
      lru_.push_front(&ins.first->first);
      ins.first->second = Entry{sealed[k].second, lru_.begin()};
      fresh[k] = 1;
    }
  }
  prepared->nodes.clear();  // blocks sealed by another call meanwhile
  if (seal_hook_)
    for (size_t k = 0; k < sealed.size(); ++k)
      if (fresh[k]) seal_hook_(keys[sealed[k].first], sealed[k].second);
  return err;
}

bool BlockStore::cache_insert(const std::string& key, std::shared_ptr<SealedBlock> block) {
  std::lock_guard<std::mutex> lk(cache_mu_);
  if (cache_.count(key) || !admit(key)) return false;
  auto ins = cache_.try_emplace(key);
  if (!ins.second) return false;
  lru_.push_front(&ins.first->first);
  ins.first->second = Entry{std::move(block), lru_.begin()};
  return true;
}

std::shared_ptr<SealedBlock> BlockStore::peek(const std::string& key) {
  std::lock_guard<std::mutex> lk(cache_mu_);
  auto it = cache_.find(key);
  return it == cache_.end() ? nullptr : it->second.block;
}

int BlockStore::lookup_many(const std::vector<std::string>& keys,
                            std::vector<std::shared_ptr<SealedBlock>>* out) {
  std::lock_guard<std::mutex> lk(cache_mu_);
  out->clear();
  out->reserve(keys.size());
  for (size_t i = 0; i < keys.size(); ++i) {
    auto it = cache_.find(keys[i]);
    if (it == cache_.end()) {
      const size_t sep = keys[i].find('\0');
      return fail(PF_ERR_STORAGE,
                  strf("missing KV block hash at index %zu (namespace=%s, hash_len=%zu)", i,
                       keys[i].substr(0, sep).c_str(),
                       sep == std::string::npos ? keys[i].size() : keys[i].size() - sep - 1));
    }
    lru_.splice(lru_.begin(), lru_, it->second.pos);
    if (lfu_) lfu_->incr(keys[i]);  // a hit is recorded (cache.rs:59-67)
    out->push_back(it->second.block);
  }
  return PF_OK;
}

uint64_t BlockStore::sealed_count() {
  std::lock_guard<std::mutex> lk(cache_mu_);
  return cache_.size();
}

uint64_t BlockStore::inflight_count() {
  std::lock_guard<std::mutex> lk(inflight_mu_);
  return inflight_.size();
}

// ===========================================================================
// Device worker: one save context (used by the calling thread) and one load
// thread with its own context (gpu_worker.rs:52-201).
// ===========================================================================
// The block lists of a load's later layers, which the requesting thread
// builds while the load thread already copies the first ones (a large load
// is split so that its first layers land sooner).  The requesting thread
// fills `blocks` and `bytes`, then publishes once, ready or failed; the load
// thread reads them only after wait() returns, and waits in any case before
// it lets go of the task (whose names and sealed blocks the requesting
// thread reads meanwhile).
class LaterLayers {
 public:
  uint32_t first = 0;                              // call index of blocks[0]
  std::vector<std::vector<pf_block_xfer>> blocks;  // layers first, first+1, ...
  uint64_t bytes = 0;

  void publish(int rc, std::string error) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      rc_ = rc;
      error_ = std::move(error);
      done_ = true;
    }
    cv_.notify_all();
  }
  // PF_OK once the lists are complete, or the requester's error (set as the
  // thread's last error).
  int wait() {
    std::unique_lock<std::mutex> lk(mu_);
    cv_.wait(lk, [this] { return done_; });
    return rc_ == PF_OK ? PF_OK : fail(rc_, error_);
  }

 private:
  std::mutex mu_;
  std::condition_variable cv_;
  bool done_ = false;
  int rc_ = PF_OK;
  std::string error_;
};

struct LoadTask {
  std::vector<std::string> names;
  std::vector<pf_kv_layout> layouts;
  std::vector<std::vector<pf_block_xfer>> blocks;
  std::vector<std::shared_ptr<SealedBlock>> keep;  // host copies stay alive
  pf_load_state* state = nullptr;
  uint32_t mode = PF_MODE_KERNEL;
  uint64_t bytes = 0;
  // A task that only writes a consumer's layer words (a load that failed in
  // planning or had nothing to copy): queued behind the device's earlier
  // loads so it cannot end their waits early.
  bool marks_only = false;
  pf_layer_words words{};
  uint32_t n_words = 0;
  std::chrono::steady_clock::time_point submitted = std::chrono::steady_clock::now();
  // Layers from later->first on, when their lists are still being built.
  std::shared_ptr<LaterLayers> later;
};

// A thread that runs one job at a time for the load thread: publishing each
// layer of a staged load as its mark lands, while the load thread issues the
// load, whose call drives the copy engines slice by slice and returns only
// once its copies are done.
class Publisher {
 public:
  Publisher() : thread_([this] { loop(); }) {}
  ~Publisher() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    thread_.join();
  }
  // Starts `job`; the previous job must have been waited for.
  void start(std::function<int()> job) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      job_ = std::move(job);
      finished_.store(false, std::memory_order_relaxed);
    }
    cv_.notify_all();
  }
  // True once the job has returned.
  bool finished() const { return finished_.load(std::memory_order_acquire); }
  // Waits for the job; its result, with its error message set on this thread.
  int wait() {
    std::unique_lock<std::mutex> lk(mu_);
    cv_.wait(lk, [this] { return finished(); });
    return rc_ == PF_OK ? PF_OK : fail(rc_, msg_);
  }

 private:
  void loop() {
    // Its polls sleep 10 us between reads, as the load thread's do: without
    // the load thread's timer slack (1 us) each sleep lasts about 60 us.
    (void)prctl(PR_SET_TIMERSLACK, 1000UL, 0, 0, 0);
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      cv_.wait(lk, [this] { return stop_ || job_; });
      if (!job_) return;
      std::function<int()> job = std::move(job_);
      job_ = nullptr;
      lk.unlock();
      const int rc = job();
      std::string msg = rc == PF_OK ? std::string() : std::string(pf_last_error());
      lk.lock();
      rc_ = rc;
      msg_ = std::move(msg);
      finished_.store(true, std::memory_order_release);
      cv_.notify_all();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  std::function<int()> job_;
  std::atomic<bool> finished_{true};
  int rc_ = PF_OK;
  std::string msg_;
  bool stop_ = false;
  std::thread thread_;  // last: started once the members above exist
};

class DeviceWorker {
 public:
  static int create(int device, bool with_gpu, std::shared_ptr<DeviceWorker>* out,
                    std::atomic<uint64_t>* loaded_bytes, std::atomic<uint64_t>* failures);
  ~DeviceWorker();
  // Saves the layers; `overlap` runs on the calling thread while the copy is
  // in flight, and the call returns once the bytes are in place.  With
  // `pending`, layers from pending->head on are listed by pending->ready(),
  // which the transfer calls on this thread once the first ones are issued.
  int save(std::vector<pf_layer_xfer>& layers, uint32_t mode,
           const std::function<void()>& overlap, const PendingLayers* pending = nullptr);
  int submit(LoadTask&& task);
  void wait_idle();
  // The mode a load in `mode` would run in on this device's load context.
  uint32_t resolve_load_mode(uint32_t mode, const pf_layer_xfer* layers, uint32_t n) const {
    return load_x_ ? resolve_mode(load_x_, layers, n, mode) : PF_MODE_KERNEL;
  }
  // The same for a save on this device's save context.
  uint32_t resolve_save_mode(uint32_t mode, const pf_layer_xfer* layers, uint32_t n) const {
    return save_x_ ? resolve_mode(save_x_, layers, n, mode) : PF_MODE_KERNEL;
  }
  // Hands a new task the block lists of a finished one (cleared, capacity
  // kept), so building a task allocates nothing new in steady state.
  void take_spares(LoadTask* task);

 private:
  void load_loop();
  int device_ = 0;
  bool gpu_ = false;
  pf_xfer* save_x_ = nullptr;
  pf_xfer* load_x_ = nullptr;
  std::mutex save_mu_;
  std::mutex q_mu_;
  std::condition_variable q_cv_, idle_cv_;
  std::deque<LoadTask> queue_;
  size_t busy_ = 0;
  bool stop_ = false;
  std::thread thread_;
  std::vector<hipEvent_t> events_;
  // Per-layer completion of marked loads: one word per layer in pinned host
  // memory, set to the load's ticket by the copy kernel.
  uint64_t* host_words_ = nullptr;
  size_t host_words_cap_ = 0;
  uint64_t ticket_ = 0;
  // Consumers' layer words mapped from other processes, by handle (the
  // mappings are kept for reuse; the oldest is closed beyond kMaxWordMaps).
  std::deque<std::pair<std::string, uint64_t>> word_maps_;
  std::atomic<uint64_t>* loaded_bytes_ = nullptr;
  std::atomic<uint64_t>* failures_ = nullptr;
  std::vector<std::vector<pf_block_xfer>> spare_blocks_;  // under q_mu_
  // Saves on the device's save context right now; a load issued meanwhile
  // shares the host link with them (see kLoadGridAlone).
  std::atomic<int> saves_running_{0};
  std::vector<std::shared_ptr<SealedBlock>> spare_keep_;  // under q_mu_
  std::unique_ptr<Publisher> publisher_;  // staged marked loads' layers (with a device)

  int map_layer_words(const pf_layer_words& w, uint64_t* words);
  int load_marked(std::vector<pf_layer_xfer>& layers, uint32_t mode, pf_load_state* st,
                  uint64_t consumer_words, uint64_t consumer_value, const PendingLayers* pending);
};

constexpr size_t kMaxWordMaps = 16;

// Persistent workgroups of a load over the host link.  Alone on the link,
// 32 (512 KiB in flight) restore the Llama prefix as fast as 64 (23.33 ms
// of kernel time either way) and land each layer about 0.25 ms sooner:
// layer 0 of a 4-layer marked launch 0.80 ms after the call against 1.05
// ms, since with more in flight some XCDs' tiles straggle behind the
// others'.  Beside a save, a restore needs the larger grid to keep its
// share of the link (save + restore 76 GB/s at 32 + 32 against 89 at the
// defaults, 32 + 64).
constexpr uint32_t kLoadGridAlone = 32;

// Staging of the workers' transfer contexts: two slots each of the staged
// mode's largest slice (1 GiB of HBM per device in all).
constexpr uint64_t kSaveStagingBytes = 2 * PF_STAGED_SAVE_SLICE_DEFAULT;
constexpr uint64_t kLoadStagingBytes = 2 * PF_STAGED_LOAD_SLICE_DEFAULT;

int DeviceWorker::create(int device, bool with_gpu, std::shared_ptr<DeviceWorker>* out,
                         std::atomic<uint64_t>* loaded_bytes, std::atomic<uint64_t>* failures) {
  auto w = std::make_shared<DeviceWorker>();
  w->device_ = device;
  w->gpu_ = with_gpu;
  w->loaded_bytes_ = loaded_bytes;
  w->failures_ = failures;
  if (with_gpu) {
    if (pf_xfer_create(device, kSaveStagingBytes, &w->save_x_) != PF_OK ||
        pf_xfer_create(device, kLoadStagingBytes, &w->load_x_) != PF_OK)
      return fail(PF_ERR_INIT, std::string("failed to initialize HIP: ") + pf_last_error());
    w->publisher_.reset(new Publisher());
  }
  w->thread_ = std::thread([p = w.get()] { p->load_loop(); });
  *out = std::move(w);
  return PF_OK;
}

DeviceWorker::~DeviceWorker() {
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    stop_ = true;
  }
  q_cv_.notify_all();
  if (thread_.joinable()) thread_.join();
  publisher_.reset();
  if (save_x_) pf_xfer_destroy(save_x_);
  if (load_x_) pf_xfer_destroy(load_x_);
  if (gpu_) {
    (void)hipSetDevice(device_);
    for (hipEvent_t e : events_) (void)hipEventDestroy(e);
    for (auto& m : word_maps_) (void)pf_ipc_close(m.second);
    if (host_words_) (void)pf_pinned_free(host_words_);
  }
}

// Address of the consumer's layer words in this process.
int DeviceWorker::map_layer_words(const pf_layer_words& w, uint64_t* words) {
  if (w.kind == PF_LAYER_WORDS_LOCAL) {
    *words = w.address;
    return PF_OK;
  }
  std::string key(reinterpret_cast<const char*>(w.handle), PF_IPC_HANDLE_BYTES);
  key.append(reinterpret_cast<const char*>(&w.alloc_size), sizeof(w.alloc_size));
  for (auto& m : word_maps_)
    if (m.first == key) {
      *words = m.second + w.offset;
      return PF_OK;
    }
  uint64_t base = 0;
  if (int rc = pf_ipc_open(w.handle, w.alloc_size, &base)) return rc;
  if (word_maps_.size() >= kMaxWordMaps) {
    (void)pf_ipc_close(word_maps_.front().second);
    word_maps_.pop_front();
  }
  word_maps_.emplace_back(std::move(key), base);
  *words = base + w.offset;
  return PF_OK;
}

// One launch for every layer (from pinned memory); layer l is published in
// the LoadState as soon as the kernel has marked it.  The host words are
// polled in order; a stream that went idle with a word unset means the copy
// failed.
int DeviceWorker::load_marked(std::vector<pf_layer_xfer>& layers, uint32_t mode,
                              pf_load_state* st, uint64_t consumer_words,
                              uint64_t consumer_value, const PendingLayers* pending) {
  const size_t L = layers.size();
  if (L > host_words_cap_) {
    size_t cap = 64;
    while (cap < L) cap <<= 1;
    if (host_words_) (void)pf_pinned_free(host_words_);
    host_words_ = nullptr;
    host_words_cap_ = 0;
    void* h = nullptr;
    uint64_t d = 0;
    if (int rc = pf_pinned_allocate(cap * 8, PF_PINNED_COHERENT, &h, &d)) return rc;
    host_words_ = static_cast<uint64_t*>(h);
    std::memset(host_words_, 0, cap * 8);
    host_words_cap_ = cap;
  }
  const uint64_t ticket = ++ticket_;
  pf_layer_signal sig[2] = {};
  sig[0].words = reinterpret_cast<uint64_t>(host_words_);
  sig[0].value = ticket;
  sig[0].host_memory = 1;
  uint32_t n_sig = 1;
  if (consumer_words) {
    sig[1].words = consumer_words;
    sig[1].value = consumer_value;
    n_sig = 2;
  }
  const auto t0 = std::chrono::steady_clock::now();
  auto issue = [&]() -> int {
    return pending ? load_layers_pending(load_x_, layers.data(), static_cast<uint32_t>(L), mode,
                                         nullptr, sig, n_sig, *pending)
                   : pf_load_layers_marked(load_x_, layers.data(), static_cast<uint32_t>(L), mode,
                                           sig, n_sig);
  };
  hipStream_t stream = static_cast<hipStream_t>(pf_xfer_stream(load_x_));
  // Publishes each layer in the LoadState as its word lands.  `issuing`
  // reads 1 while a staged call still runs on another thread (its copies
  // are in flight meanwhile, whatever the stream says) and 2 once it failed;
  // otherwise a stream gone idle with a word unset means the copy failed.
  std::atomic<int> issuing{0};
  auto t_first = t0;
  auto publish = [&]() -> int {
    for (size_t l = 0; l < L; ++l) {
      const uint64_t* w = host_words_ + l;
      for (uint32_t spins = 0; __atomic_load_n(w, __ATOMIC_ACQUIRE) < ticket; ++spins) {
        if (spins % 64 == 63) {
          const int state = issuing.load(std::memory_order_acquire);
          if (state == 2) return PF_ERR_STORAGE;  // the issuing thread reports why
          if (state == 0) {
            const hipError_t q = hipStreamQuery(stream);
            if (q != hipErrorNotReady && __atomic_load_n(w, __ATOMIC_ACQUIRE) < ticket)
              return fail(PF_ERR_STORAGE,
                          strf("layer %zu of a marked load was not marked (%s)", l,
                               hipGetErrorString(q)));
          }
        }
        if (spins > 256) std::this_thread::sleep_for(std::chrono::microseconds(10));
      }
      pf_load_state_set_layers_done(st, static_cast<int64_t>(l + 1));
      if (l == 0) t_first = std::chrono::steady_clock::now();
    }
    return PF_OK;
  };
  if (mode == PF_MODE_STAGED && publisher_) {
    // A staged load returns only once its copies are done.  It is issued on
    // this thread at once, and the publisher thread publishes its layers as
    // they land (that thread's wake-up overlaps the first layer's copy).
    issuing.store(1, std::memory_order_release);
    publisher_->start(publish);
    const int rc = issue();
    const std::string msg = rc == PF_OK ? std::string() : std::string(pf_last_error());
    issuing.store(rc == PF_OK ? 0 : 2, std::memory_order_release);
    const int prc = publisher_->wait();  // it reads this call's locals
    if (rc) return fail(rc, msg);
    if (prc) return prc;
  } else {
    if (int rc = issue()) return rc;
    if (int rc = publish()) return rc;
  }
  if (tracing())
    std::fprintf(stderr, "[pegaflow] marked load at=%.0fus first_layer=%.0fus\n", mono_us(t0),
                 us_between(t0, t_first));
  return pf_xfer_synchronize(load_x_);
}

int DeviceWorker::save(std::vector<pf_layer_xfer>& layers, uint32_t mode,
                       const std::function<void()>& overlap, const PendingLayers* pending) {
  if (!gpu_)
    return fail(PF_ERR_UNSUPPORTED, "storage error: engine pool is not mapped for a device");
  std::lock_guard<std::mutex> lk(save_mu_);
  struct Running {  // counted while the save is on the device
    std::atomic<int>& n;
    explicit Running(std::atomic<int>& c) : n(c) { n.fetch_add(1); }
    ~Running() { n.fetch_sub(1); }
  } running(saves_running_);
  const uint32_t n = static_cast<uint32_t>(layers.size());
  int rc = pending ? save_layers_pending_begin(save_x_, layers.data(), n, mode, *pending)
                   : save_layers_begin(save_x_, layers.data(), n, mode);
  if (rc) {
    const std::string msg = pf_last_error();
    (void)pf_xfer_synchronize(save_x_);  // nothing may still read the regions
    return fail(PF_ERR_STORAGE, "storage error: " + msg);
  }
  overlap();
  if (pf_xfer_synchronize(save_x_))
    return fail(PF_ERR_STORAGE, std::string("storage error: ") + pf_last_error());
  return PF_OK;
}

int DeviceWorker::submit(LoadTask&& task) {
  if (!gpu_)
    return fail(PF_ERR_UNSUPPORTED, "storage error: engine pool is not mapped for a device");
  {
    std::lock_guard<std::mutex> lk(q_mu_);
    if (stop_)
      return fail(PF_ERR_STORAGE,
                  strf("storage error: Load worker channel closed for device %d", device_));
    queue_.push_back(std::move(task));
    ++busy_;
  }
  q_cv_.notify_one();
  return PF_OK;
}

void DeviceWorker::take_spares(LoadTask* task) {
  std::lock_guard<std::mutex> lk(q_mu_);
  if (task->blocks.empty()) task->blocks.swap(spare_blocks_);
  if (task->keep.capacity() == 0) task->keep.swap(spare_keep_);
}

void DeviceWorker::wait_idle() {
  std::unique_lock<std::mutex> lk(q_mu_);
  idle_cv_.wait(lk, [this] { return busy_ == 0; });
}

void DeviceWorker::load_loop() {
  if (gpu_) (void)hipSetDevice(device_);
  // The loop's waits for per-layer marks sleep 10 us between polls; the
  // default 50 us timer slack would stretch each to about 60 us and delay
  // every layer's publication by as much.
  (void)prctl(PR_SET_TIMERSLACK, 1000UL, 0, 0, 0);
  for (;;) {
    LoadTask task;
    {
      std::unique_lock<std::mutex> lk(q_mu_);
      q_cv_.wait(lk, [this] { return stop_ || !queue_.empty(); });
      if (queue_.empty()) return;  // stopping and drained
      task = std::move(queue_.front());
      queue_.pop_front();
    }
    if (task.marks_only) {
      uint64_t words = 0;
      if (task.n_words > 0 && map_layer_words(task.words, &words) == PF_OK) {
        pf_layer_signal all{};
        all.words = words;
        all.value = task.words.value;
        (void)mark_all_layers(load_x_, all, task.n_words);
      }
      {
        std::lock_guard<std::mutex> lk(q_mu_);
        --busy_;
      }
      idle_cv_.notify_all();
      continue;
    }
    const auto t_begin = std::chrono::steady_clock::now();
    const size_t L = task.layouts.size();
    (void)pf_xfer_set_route_grid(load_x_, PF_ROUTE_LOAD_HOST,
                                 saves_running_.load() > 0 ? PF_LOAD_HOST_DEFAULT_GRID
                                                           : kLoadGridAlone);
    bool ok = true;
    std::vector<pf_layer_xfer> layers(L);
    for (size_t l = 0; l < L; ++l)
      layers[l] = l < task.blocks.size()
                      ? pf_layer_xfer{task.layouts[l], task.blocks[l].data(), task.blocks[l].size()}
                      : pf_layer_xfer{task.layouts[l], nullptr, 0};
    // A split load: its later layers are filled in when the transfer asks.
    std::unique_ptr<PendingLayers> pending;
    if (task.later) {
      pending.reset(new PendingLayers());
      pending->head = task.later->first;
      pending->max_blocks = task.keep.size();
      pending->ready = [&task, &layers]() -> int {
        LaterLayers& later = *task.later;
        if (int rc = later.wait()) return rc;
        for (size_t i = 0; i < later.blocks.size(); ++i) {
          const size_t l = later.first + i;
          layers[l] =
              pf_layer_xfer{task.layouts[l], later.blocks[i].data(), later.blocks[i].size()};
        }
        task.bytes += later.bytes;
        return PF_OK;
      };
    }
    while (events_.size() < L) {
      hipEvent_t e = nullptr;
      if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        ok = false;
        break;
      }
      events_.push_back(e);
    }
    // A consumer may have put one event per layer in the LoadState: those
    // are recorded instead of the worker's own, so the consumer's streams
    // can wait on each layer on the device.  Interprocess handles (a
    // consumer in another process) are opened here and closed after the
    // load; in-process events are the consumer's own and recorded as given.
    std::vector<pf_event> ipc_evs;
    uint32_t n_handles = 0;
    const uint8_t* handles = pf_load_state_event_handles(task.state, &n_handles);
    const bool local_evs = pf_load_state_events_local(task.state) != 0;
    if (ok && handles) {
      if (n_handles != L) {
        set_error(strf("storage error: LoadState carries %u layer events for %zu layers",
                       n_handles, L));
        ok = false;
      }
      for (uint32_t l = 0; ok && l < n_handles; ++l) {
        const uint8_t* slot = handles + static_cast<size_t>(l) * PF_IPC_HANDLE_BYTES;
        pf_event ev = nullptr;
        if (local_evs) {
          uint64_t a = 0;
          std::memcpy(&a, slot, sizeof(a));
          ev = reinterpret_cast<pf_event>(a);
          ok = ev != nullptr;
          if (!ok) set_error(strf("storage error: null event for layer %u", l));
        } else {
          ok = pf_ipc_event_open(slot, &ev) == PF_OK;
        }
        if (ok) ipc_evs.push_back(ev);
      }
    }
    // A consumer's layer words (device-side gating without interprocess
    // events) are marked by the same launch as the engine's own host words.
    pf_layer_words lw{};
    uint32_t n_words = 0;
    uint64_t consumer_words = 0;
    (void)pf_load_state_layer_words(task.state, &lw, &n_words);
    if (n_words > 0) {
      if (map_layer_words(lw, &consumer_words) != PF_OK) {
        ok = false;
      } else if (n_words != L) {
        set_error(strf("storage error: LoadState carries words for %u layers, load has %zu",
                       n_words, L));
        ok = false;
      }
    }
    // Per-layer completion is published only where someone can use a layer
    // early: a layered LoadState (marks written by the one launch) or a
    // consumer's interprocess events (one launch per layer, each followed by
    // its event).  Otherwise completion is published at the end.
    const bool marked = ipc_evs.empty() && (pf_load_state_num_layers(task.state) > 0);
    const bool per_layer = !ipc_evs.empty();
    // A consumer's events are recorded at issue by the kernel mode; a staged
    // load would record each only as its layer lands, after the consumer
    // was told that every record is on the stream.
    if (per_layer && task.mode == PF_MODE_STAGED) task.mode = PF_MODE_KERNEL;
    if (ok && L > 0 && marked) {
      ok = load_marked(layers, task.mode, task.state, consumer_words, lw.value, pending.get()) ==
           PF_OK;
      if (!ok) (void)pf_xfer_synchronize(load_x_);
    } else if (ok && L > 0 && !per_layer) {
      ok = (pending ? load_layers_pending(load_x_, layers.data(), static_cast<uint32_t>(L),
                                          task.mode, nullptr, nullptr, 0, *pending)
                    : pf_load_layers(load_x_, layers.data(), static_cast<uint32_t>(L),
                                     task.mode, nullptr)) == PF_OK &&
           pf_xfer_synchronize(load_x_) == PF_OK;
      if (!ok) (void)pf_xfer_synchronize(load_x_);
    } else if (ok && L > 0) {
      std::vector<pf_event> evs(events_.begin(), events_.begin() + L);
      if (!ipc_evs.empty()) evs = ipc_evs;
      ok = (pending ? load_layers_pending(load_x_, layers.data(), static_cast<uint32_t>(L),
                                          task.mode, evs.data(), nullptr, 0, *pending)
                    : pf_load_layers(load_x_, layers.data(), static_cast<uint32_t>(L),
                                     task.mode, evs.data())) == PF_OK;
      // Every record is on the stream now: a consumer may start waiting.
      if (ok && !ipc_evs.empty())
        pf_load_state_set_events_recorded(task.state, static_cast<int64_t>(L));
      // Per-layer completion: layer l is published as soon as its event fires.
      for (size_t l = 0; ok && l < L; ++l) {
        ok = hipEventSynchronize(static_cast<hipEvent_t>(evs[l])) == hipSuccess;
        if (ok) pf_load_state_set_layers_done(task.state, static_cast<int64_t>(l + 1));
      }
      if (!ok) (void)pf_xfer_synchronize(load_x_);
    }
    if (!local_evs)
      for (pf_event ev : ipc_evs) (void)pf_event_destroy(ev);
    // A failed load still ends the consumer's device waits (the LoadState
    // says it failed).
    if (!ok && consumer_words) {
      pf_layer_signal all{};
      all.words = consumer_words;
      all.value = lw.value;
      (void)mark_all_layers(load_x_, all, n_words);
    }
    if (tracing()) {
      const auto t_end = std::chrono::steady_clock::now();
      std::fprintf(stderr,
                   "[pegaflow] load device=%d layers=%zu bytes=%llu queued=%.0fus copy=%.0fus "
                   "(%.2f GB/s) marked=%d per_layer_events=%d ok=%d\n",
                   device_, L, (unsigned long long)task.bytes, us_between(task.submitted, t_begin),
                   us_between(t_begin, t_end), task.bytes / us_between(t_begin, t_end) / 1e3,
                   (int)marked, (int)per_layer, (int)ok);
    }
    // The requesting thread is done with the task's blocks only once it has
    // published the later layers (a load that failed before asking for them
    // waits here).
    if (task.later) {
      if (task.later->wait() != PF_OK && ok) {
        ok = false;  // cannot happen: a load that used them asked first
      }
      for (auto& b : task.later->blocks) task.blocks.push_back(std::move(b));
      task.later.reset();
    }
    // The copies are over (a failed load drained its stream above): the
    // task's lists go back for the next load before the completion is
    // published, so a caller that issues its next load at once finds them.
    task.keep.clear();
    for (auto& b : task.blocks) b.clear();
    {
      std::lock_guard<std::mutex> lk(q_mu_);
      if (spare_blocks_.empty()) spare_blocks_.swap(task.blocks);
      if (spare_keep_.capacity() == 0) spare_keep_.swap(task.keep);
    }
    if (ok) {
      pf_load_state_set_completed(task.state);
      loaded_bytes_->fetch_add(task.bytes);
    } else {
      pf_load_state_set_error(task.state);
      failures_->fetch_add(1);
    }
    pf_load_state_close(task.state);
    {
      std::lock_guard<std::mutex> lk(q_mu_);
      --busy_;
    }
    idle_cv_.notify_all();
  }
}

// ===========================================================================
// Instances.
// ===========================================================================
struct GpuContext {
  std::mutex mu;
  std::unordered_map<std::string, pf_kv_layout> regs;
  std::shared_ptr<DeviceWorker> worker;
};

struct Instance {
  std::string id, ns;
  size_t num_layers = 0, tp_size = 0;
  std::mutex layers_mu;
  std::unordered_map<std::string, size_t> layer_ids;
  std::vector<std::string> layer_names;
  std::shared_mutex gpus_mu;
  std::map<int, std::shared_ptr<GpuContext>> gpus;

  size_t layer_id_or_create(const std::string& name) {
    std::lock_guard<std::mutex> lk(layers_mu);
    auto it = layer_ids.find(name);
    if (it != layer_ids.end()) return it->second;
    const size_t next = layer_names.size();
    layer_names.push_back(name);
    layer_ids[name] = next;
    return next;
  }
  bool layer_id(const std::string& name, size_t* out) {
    std::lock_guard<std::mutex> lk(layers_mu);
    auto it = layer_ids.find(name);
    if (it == layer_ids.end()) return false;
    *out = it->second;
    return true;
  }
  std::shared_ptr<GpuContext> gpu(int device) {
    std::shared_lock<std::shared_mutex> lk(gpus_mu);
    auto it = gpus.find(device);
    return it == gpus.end() ? nullptr : it->second;
  }
  // lib.rs:205-219.
  int slot_index(size_t layer, size_t tp_rank, size_t* out) const {
    if (layer >= num_layers)
      return fail(PF_ERR_INVALID_ARGUMENT, strf("invalid argument: layer_id %zu out of range (%zu layers)",
                                                layer, num_layers));
    if (tp_rank >= tp_size)
      return fail(PF_ERR_INVALID_ARGUMENT, strf("invalid argument: tp_rank %zu out of range (tp_size %zu)",
                                                tp_rank, tp_size));
    *out = layer * tp_size + tp_rank;
    return PF_OK;
  }
};

std::string block_key(const std::string& ns, const uint8_t* hash, size_t len) {
  std::string k;
  k.reserve(ns.size() + 1 + len);
  k.append(ns);
  k.push_back('\0');
  k.append(reinterpret_cast<const char*>(hash), len);
  return k;
}

}  // namespace pf

using namespace pf;

struct pf_allocator {
  std::unique_ptr<UnitAllocator> a;
};

struct pf_engine {
  std::shared_mutex mu;
  std::unordered_map<std::string, std::shared_ptr<Instance>> instances;
  std::shared_ptr<PinnedPool> pool;
  std::unique_ptr<BlockStore> store;
  // Saves and loads of long host runs (PF_MODE_AUTO) run staged, their
  // link traffic on the copy engines, leaving the device's other kernels at
  // their speed: beside a zero-copy save a bf16 GEMM in another process ran
  // at 1/29th of its speed, beside a zero-copy restore at 1/2.4th.  A staged
  // load lands its first layer as soon as the kernel's (its first layer is
  // sliced and copied while the rest is planned), and a staged save and
  // load at once share the link (94 GB/s) where a zero-copy restore starves
  // a staged save (59 GB/s).  Loads of short runs (a few blocks) take the
  // kernel.
  std::atomic<uint32_t> save_mode{PF_MODE_AUTO};
  std::atomic<uint32_t> load_mode{PF_MODE_AUTO};
  std::atomic<uint64_t> saved_bytes{0};
  std::atomic<uint64_t> loaded_bytes{0};
  std::atomic<uint64_t> load_failures{0};
  std::mutex disk_mu;
  std::unique_ptr<DiskTier> disk;  // declared after store: destroyed before it
  // Pre-eviction monitor (storage.rs:646-688), when configured.
  std::mutex policy_mu;  // serializes pf_engine_set_storage_policy
  std::thread pre_evict;
  std::mutex pre_mu;
  std::condition_variable pre_cv;
  bool pre_stop = false;
  std::atomic<uint64_t> pre_evicted{0};
};

namespace {

int get_instance(pf_engine* e, const char* id, std::shared_ptr<Instance>* out) {
  std::shared_lock<std::shared_mutex> lk(e->mu);
  auto it = e->instances.find(id);
  if (it == e->instances.end())
    return fail(PF_ERR_INSTANCE_MISSING, strf("instance %s not found", id));
  *out = it->second;
  return PF_OK;
}

std::vector<std::string> keys_of(const std::string& ns, const uint8_t* data, const uint64_t* offs,
                                 uint64_t n) {
  std::vector<std::string> keys(n);
  for (uint64_t i = 0; i < n; ++i)
    keys[i] = block_key(ns, data + offs[i], static_cast<size_t>(offs[i + 1] - offs[i]));
  return keys;
}

// keys_of into *keys, reusing its strings' storage (a caller's per-thread
// buffer: a load names its blocks' keys every step).
void keys_into(const std::string& ns, const uint8_t* data, const uint64_t* offs, uint64_t n,
               std::vector<std::string>* keys) {
  keys->resize(static_cast<size_t>(n));
  for (uint64_t i = 0; i < n; ++i) {
    std::string& k = (*keys)[i];
    k.assign(ns);
    k.push_back('\0');
    k.append(reinterpret_cast<const char*>(data + offs[i]),
             static_cast<size_t>(offs[i + 1] - offs[i]));
  }
}

// Host side of one planned layer save.
struct SavePlan {
  size_t slot = 0;
  size_t group = 0;                // index of the layer's hash list
  pf_kv_layout layout{};
  std::vector<int64_t> ids;        // kept block ids, in order
  std::vector<uint32_t> key_idx;   // kept hashes (indices into the list), in order
  std::vector<pf_block_xfer> blocks;
  std::shared_ptr<PoolAllocation> k_alloc, v_alloc;
  bool split = false;
};

// The LayerBlocks of one planned layer in one allocation, which also holds
// the pool regions; each block's handle shares the set's reference count.
struct LayerBlockSet {
  std::vector<LayerBlock> blocks;
  std::shared_ptr<PoolAllocation> k_alloc, v_alloc;
};

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// Allocator.
// ---------------------------------------------------------------------------
int pf_allocator_create(uint64_t total_bytes, uint64_t unit_size, pf_allocator** out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "null output");
  std::unique_ptr<UnitAllocator> a;
  if (int rc = UnitAllocator::create(total_bytes, unit_size, &a)) return rc;
  *out = new pf_allocator{std::move(a)};
  return PF_OK;
}

int pf_allocator_create_auto(uint64_t total_bytes, pf_allocator** out) {
  const uint64_t unit = total_bytes > kU32Max ? (total_bytes + kU32Max - 1) / kU32Max : 1;
  return pf_allocator_create(total_bytes, unit, out);
}

int pf_allocator_destroy(pf_allocator* a) {
  delete a;
  return PF_OK;
}

int pf_allocator_allocate(pf_allocator* a, uint64_t size_bytes, int* found, uint64_t* offset,
                          uint64_t* size) {
  bool f = false;
  uint64_t o = 0, s = 0;
  if (int rc = a->a->allocate(size_bytes, &f, &o, &s)) return rc;
  *found = f ? 1 : 0;
  if (offset) *offset = o;
  if (size) *size = s;
  return PF_OK;
}

int pf_allocator_free(pf_allocator* a, uint64_t offset) {
  a->a->free(offset);
  return PF_OK;
}

int pf_allocator_report(pf_allocator* a, uint64_t* total_bytes, uint64_t* free_bytes,
                        uint64_t* largest_free_bytes, uint64_t* unit_size) {
  if (total_bytes) *total_bytes = a->a->total_bytes();
  if (free_bytes) *free_bytes = a->a->free_bytes();
  if (largest_free_bytes) *largest_free_bytes = a->a->largest_free_bytes();
  if (unit_size) *unit_size = a->a->unit_size();
  return PF_OK;
}

// ---------------------------------------------------------------------------
// Engine.
// ---------------------------------------------------------------------------
int pf_engine_create(uint64_t pool_bytes, uint32_t pool_kind, uint32_t pinned_flags,
                     uint64_t unit_hint, pf_engine** out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "null output");
  if (pool_kind != PF_POOL_PINNED && pool_kind != PF_POOL_HOST)
    return fail(PF_ERR_INVALID_ARGUMENT, "unknown pool kind");
  std::shared_ptr<PinnedPool> pool;
  if (int rc = PinnedPool::create(pool_bytes, unit_hint, pool_kind == PF_POOL_PINNED, pinned_flags,
                                  &pool))
    return rc;
  auto* e = new pf_engine();
  e->pool = pool;
  e->store.reset(new BlockStore(pool));
  *out = e;
  return PF_OK;
}

namespace {

void stop_pre_evict(pf_engine* e) {
  if (!e->pre_evict.joinable()) return;
  {
    std::lock_guard<std::mutex> lk(e->pre_mu);
    e->pre_stop = true;
  }
  e->pre_cv.notify_all();
  e->pre_evict.join();
  e->pre_stop = false;
}

}  // namespace

int pf_engine_destroy(pf_engine* e) {
  if (!e) return PF_OK;
  stop_pre_evict(e);
  {
    std::unique_lock<std::shared_mutex> lk(e->mu);
    e->instances.clear();  // joins the workers after their queued loads
  }
  e->disk.reset();  // writes what is queued, then stops its threads
  delete e;
  return PF_OK;
}

// storage.rs:43-111, 346-398 and cache.rs:33-47: admission sized by the
// value-size hint, and the pre-eviction monitor's thread.
int pf_engine_set_storage_policy(pf_engine* e, int lfu_admission, uint64_t value_size_hint,
                                 int pre_evict, uint64_t threshold_bytes, uint64_t target_bytes,
                                 uint32_t interval_ms) {
  if (!e) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: null engine");
  if (pre_evict && interval_ms == 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: pre-eviction interval of 0 ms");
  std::lock_guard<std::mutex> policy(e->policy_mu);
  uint64_t used = 0, total = 0;
  e->pool->usage(&used, &total);
  const uint64_t per_value = value_size_hint ? value_size_hint : kLfuDefaultValueBytes;
  e->store->set_admission(lfu_admission ? std::max<uint64_t>(1, total / per_value) : 0,
                          std::random_device{}() ^ (uint64_t(std::random_device{}()) << 32));
  stop_pre_evict(e);
  if (pre_evict) {
    e->pre_evict = std::thread([e, threshold_bytes, target_bytes, interval_ms]() {
      std::unique_lock<std::mutex> lk(e->pre_mu);
      for (;;) {
        if (e->pre_cv.wait_for(lk, std::chrono::milliseconds(interval_ms),
                               [e] { return e->pre_stop; }))
          return;
        uint64_t used_now = 0, total_now = 0;
        e->pool->usage(&used_now, &total_now);
        const uint64_t free_now = total_now > used_now ? total_now - used_now : 0;
        if (free_now >= threshold_bytes) continue;
        const uint64_t need = target_bytes > free_now ? target_bytes - free_now : 0;
        lk.unlock();
        e->pre_evicted += e->store->evict_bytes(need, nullptr);
        lk.lock();
      }
    });
  }
  return PF_OK;
}

int pf_engine_set_modes(pf_engine* e, uint32_t save_mode, uint32_t load_mode) {
  if (save_mode > PF_MODE_AUTO || load_mode > PF_MODE_AUTO)
    return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: unknown transfer mode");
  e->save_mode = save_mode;
  e->load_mode = load_mode;
  return PF_OK;
}

// lib.rs:373-469.
int pf_engine_register_context_layer(pf_engine* e, const char* instance_id, const char* ns,
                                     int device_id, const char* layer_name, uint64_t data_ptr,
                                     uint64_t size_bytes, uint64_t num_blocks,
                                     uint64_t bytes_per_block, uint64_t kv_stride_bytes,
                                     uint64_t segments, uint64_t tp_rank, uint64_t tp_size,
                                     uint64_t num_layers) {
  const std::string layer(layer_name);
  if (bytes_per_block == 0 || num_blocks == 0 || segments == 0)
    return fail(PF_ERR_INVALID_ARGUMENT,
                "invalid argument: invalid KV cache layout for layer " + layer);
  if (segments > 1 && kv_stride_bytes == 0)
    return fail(PF_ERR_INVALID_ARGUMENT,
                "invalid argument: kv_stride_bytes must be > 0 when segments > 1 for layer " + layer);
  if (device_id < 0) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: device_id must be >= 0");
  pf_kv_layout layout{};
  if (pf_layout_init(data_ptr, size_bytes, num_blocks, bytes_per_block, kv_stride_bytes, segments,
                     &layout))
    return fail(PF_ERR_INVALID_ARGUMENT,
                std::string("invalid argument: ") + pf_last_error() + " for layer " + layer);
  std::shared_ptr<Instance> inst;
  {
    std::unique_lock<std::shared_mutex> lk(e->mu);
    auto it = e->instances.find(instance_id);
    if (it != e->instances.end()) {
      inst = it->second;
      if (inst->num_layers != num_layers || inst->tp_size != tp_size)
        return fail(PF_ERR_TOPOLOGY_MISMATCH,
                    strf("topology mismatch: instance %s exists with layers=%zu, tp=%zu; "
                         "requested layers=%llu, tp=%llu",
                         instance_id, inst->num_layers, inst->tp_size,
                         (unsigned long long)num_layers, (unsigned long long)tp_size));
    } else {
      inst = std::make_shared<Instance>();
      inst->id = instance_id;
      inst->ns = ns;
      inst->num_layers = num_layers;
      inst->tp_size = tp_size;
      e->instances[instance_id] = inst;
    }
  }
  // ensure_gpu (lib.rs:221-252): one worker per (instance, device).
  std::shared_ptr<GpuContext> gpu;
  {
    std::unique_lock<std::shared_mutex> lk(inst->gpus_mu);
    auto it = inst->gpus.find(device_id);
    if (it == inst->gpus.end()) {
      auto g = std::make_shared<GpuContext>();
      if (int rc = DeviceWorker::create(device_id, e->pool->device_backed(), &g->worker,
                                        &e->loaded_bytes, &e->load_failures))
        return rc;
      it = inst->gpus.emplace(device_id, g).first;
    }
    gpu = it->second;
  }
  inst->layer_id_or_create(layer);
  std::lock_guard<std::mutex> lk(gpu->mu);
  gpu->regs[layer] = layout;
  return PF_OK;
}

int pf_engine_unregister_instance(pf_engine* e, const char* instance_id) {
  std::shared_ptr<Instance> removed;
  {
    std::unique_lock<std::shared_mutex> lk(e->mu);
    auto it = e->instances.find(instance_id);
    if (it == e->instances.end())
      return fail(PF_ERR_INSTANCE_MISSING, strf("instance %s not found", instance_id));
    removed = std::move(it->second);
    e->instances.erase(it);
  }
  // Queued loads still read the instance's layer tensors: let them finish
  // before the caller may release that memory. The workers themselves stop
  // when the last reference to the instance drops.
  std::vector<std::shared_ptr<DeviceWorker>> workers;
  {
    std::shared_lock<std::shared_mutex> g(removed->gpus_mu);
    for (auto& gk : removed->gpus) workers.push_back(gk.second->worker);
  }
  for (auto& w : workers) w->wait_idle();
  return PF_OK;
}

// lib.rs:803-838.
int pf_engine_count_prefix_hit_blocks(pf_engine* e, const char* instance_id,
                                      const uint8_t* hash_data, const uint64_t* hash_offsets,
                                      uint64_t n, uint64_t* hits) {
  std::shared_ptr<Instance> inst;
  if (int rc = get_instance(e, instance_id, &inst)) return rc;
  uint64_t h = 0;
  for (uint64_t i = 0; i < n; ++i) {
    if (!e->store->cache_contains(block_key(inst->ns, hash_data + hash_offsets[i],
                                            static_cast<size_t>(hash_offsets[i + 1] - hash_offsets[i]))))
      break;
    ++h;
  }
  *hits = h;
  return PF_OK;
}

// lib.rs:497-782.
int pf_engine_batch_save(pf_engine* e, const char* instance_id, uint64_t tp_rank, int device_id,
                         const pf_save_layer* layers, uint32_t num_layers) {
  const auto t_start = std::chrono::steady_clock::now();
  std::shared_ptr<Instance> inst;
  if (int rc = get_instance(e, instance_id, &inst)) return rc;
  auto gpu = inst->gpu(device_id);
  if (!gpu)
    return fail(PF_ERR_WORKER_MISSING,
                strf("device %d not found in instance %s", device_id, instance_id));
  const size_t total_slots = inst->num_layers * inst->tp_size;
  // Pass 1: every layer's registration and slot, and its hash list.  The
  // layers of a batch normally share one list, so keys are built once per
  // distinct list and the store is consulted once per key, not per layer.
  struct KeyGroup {
    const uint8_t* data;
    const uint64_t* offs;
    uint64_t n;
    std::vector<std::string> keys;
    std::vector<size_t> plans;  // the layers that use it
  };
  std::vector<KeyGroup> groups;
  std::vector<SavePlan> plans(num_layers);
  for (uint32_t li = 0; li < num_layers; ++li) {
    const pf_save_layer& sl = layers[li];
    const std::string name(sl.layer_name);
    size_t layer_id = 0;
    if (!inst->layer_id(name, &layer_id))
      return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: layer " + name + " unknown");
    SavePlan& plan = plans[li];
    {
      std::lock_guard<std::mutex> lk(gpu->mu);
      auto it = gpu->regs.find(name);
      if (it == gpu->regs.end())
        return fail(PF_ERR_INVALID_ARGUMENT,
                    "invalid argument: layer " + name + " not registered on device");
      plan.layout = it->second;
    }
    if (int rc = inst->slot_index(layer_id, tp_rank, &plan.slot)) return rc;
    for (uint64_t i = 0; i < sl.num_blocks; ++i)
      if (sl.block_ids[i] >= 0 && static_cast<uint64_t>(sl.block_ids[i]) >= plan.layout.num_blocks)
        return fail(PF_ERR_INVALID_ARGUMENT,
                    strf("invalid argument: block %d out of range for layer %s (%llu blocks "
                         "registered)",
                         sl.block_ids[i], name.c_str(),
                         (unsigned long long)plan.layout.num_blocks));
    // Same list: the same buffers, or (callers that copy per layer, such as
    // the gRPC service) equal offsets and bytes.
    auto same_list = [&](const KeyGroup& kg) {
      if (kg.n != sl.num_blocks) return false;
      if (kg.data == sl.hash_data && kg.offs == sl.hash_offsets) return true;
      const size_t n = static_cast<size_t>(sl.num_blocks);
      return std::memcmp(kg.offs, sl.hash_offsets, (n + 1) * sizeof(uint64_t)) == 0 &&
             std::memcmp(kg.data + kg.offs[0], sl.hash_data + sl.hash_offsets[0],
                         static_cast<size_t>(sl.hash_offsets[n] - sl.hash_offsets[0])) == 0;
    };
    size_t g = 0;
    while (g < groups.size() && !same_list(groups[g])) ++g;
    if (g == groups.size())
      groups.push_back(KeyGroup{sl.hash_data, sl.hash_offsets, sl.num_blocks,
                                keys_of(inst->ns, sl.hash_data, sl.hash_offsets, sl.num_blocks),
                                {}});
    groups[g].plans.push_back(li);
    plan.group = g;
  }
  // Pass 2: filtering and dedup (lib.rs:590-621): each layer's kept block
  // ids, in order.
  for (const KeyGroup& g : groups) {
    std::vector<size_t> slots;
    for (size_t li : g.plans) slots.push_back(plans[li].slot);
    std::vector<std::vector<char>> keep;
    e->store->filter_slots(g.keys, slots, &keep);
    for (size_t j = 0; j < g.plans.size(); ++j) {
      SavePlan& plan = plans[g.plans[j]];
      const pf_save_layer& sl = layers[g.plans[j]];
      for (uint64_t i = 0; i < sl.num_blocks; ++i)
        if (sl.block_ids[i] >= 0 && keep[j][i]) {
          plan.ids.push_back(sl.block_ids[i]);
          plan.key_idx.push_back(static_cast<uint32_t>(i));
        }
    }
  }
  // The host regions in the reference's layout, one layer at a time.
  auto place = [&](SavePlan& plan) -> int {
    const pf_kv_layout& reg = plan.layout;
    const uint64_t n = plan.ids.size();
    plan.split = reg.segments == 2 && reg.kv_stride_bytes > reg.bytes_per_block;
    plan.blocks.resize(n);
    if (plan.split) {  // lib.rs:636-679
      const uint64_t seg = reg.bytes_per_block;
      plan.k_alloc = e->store->allocate(seg * n);
      if (!plan.k_alloc)
        return fail(PF_ERR_STORAGE,
                    "storage error: pinned pool exhausted while allocating K segment buffer");
      plan.v_alloc = e->store->allocate(seg * n);
      if (!plan.v_alloc)
        return fail(PF_ERR_STORAGE,
                    "storage error: pinned pool exhausted while allocating V segment buffer");
      for (uint64_t i = 0; i < n; ++i)
        plan.blocks[i] =
            pf_block_xfer{plan.ids[i], reinterpret_cast<uint64_t>(plan.k_alloc->ptr + i * seg),
                          reinterpret_cast<uint64_t>(plan.v_alloc->ptr + i * seg)};
    } else {  // lib.rs:706-747
      const uint64_t bs = reg.block_size_bytes;
      plan.k_alloc = e->store->allocate(bs * n);
      if (!plan.k_alloc)
        return fail(PF_ERR_STORAGE,
                    "storage error: pinned pool exhausted while allocating contiguous block "
                    "buffer");
      for (uint64_t i = 0; i < n; ++i)
        plan.blocks[i] =
            pf_block_xfer{plan.ids[i], reinterpret_cast<uint64_t>(plan.k_alloc->ptr + i * bs), 0};
    }
    return PF_OK;
  };
  // The layers with blocks to copy, in call order.
  std::vector<size_t> order;
  uint64_t chunks = 0, max_blocks = 0;
  for (size_t pi = 0; pi < plans.size(); ++pi) {
    const SavePlan& p = plans[pi];
    if (p.ids.empty()) continue;
    order.push_back(pi);
    const bool split = p.layout.segments == 2 && p.layout.kv_stride_bytes > p.layout.bytes_per_block;
    chunks += p.ids.size() * (split ? 2 : 1);
    max_blocks = std::max<uint64_t>(max_blocks, p.ids.size());
  }
  if (order.empty()) return PF_OK;
  // A large save is pipelined as loads are: the first layers' regions and
  // lists are made, their copy starts, and the rest are made meanwhile
  // (pool allocations, which may evict, and the block lists: about 0.1 ms
  // for the Llama prefix, off the copy's start).  The reference likewise
  // allocates each layer's regions just before that layer's copy
  // (lib.rs:636-747 inside the per-layer loop).
  uint32_t mode = e->save_mode.load();
  if (int rc = place(plans[order[0]])) return rc;
  if (mode == PF_MODE_AUTO) {  // the first layer's host runs decide (auto_mode)
    const SavePlan& p0 = plans[order[0]];
    const pf_layer_xfer lx{p0.layout, p0.blocks.data(), p0.blocks.size()};
    mode = gpu->worker->resolve_save_mode(PF_MODE_AUTO, &lx, 1);
  }
  const uint32_t nl = static_cast<uint32_t>(order.size());
  uint32_t head = nl;
  if ((mode == PF_MODE_KERNEL || mode == PF_MODE_STAGED) && pipeline_head_layers(nl, chunks) > 0) {
    // As many leading layers as it takes for their copy to outlast making
    // the rest (about 10 ns per later block entry, in which the link moves
    // about 500 bytes): one layer for the Llama prefix.
    constexpr uint64_t kHeadBytesPerLaterEntry = 500;
    uint64_t later_entries = 0, head_bytes = 0;
    for (size_t pi : order) later_entries += plans[pi].ids.size();
    for (head = 0; head + 1 < nl;) {
      const SavePlan& p = plans[order[head++]];
      head_bytes += p.ids.size() * p.layout.block_size_bytes;
      later_entries -= p.ids.size();
      if (head_bytes >= later_entries * kHeadBytesPerLaterEntry) break;
    }
  }
  for (uint32_t k = 1; k < head; ++k)
    if (int rc = place(plans[order[k]])) return rc;
  std::vector<pf_layer_xfer> xl(nl);
  auto list = [&](uint32_t k) {
    const SavePlan& p = plans[order[k]];
    xl[k] = pf_layer_xfer{p.layout, p.blocks.data(), p.blocks.size()};
  };
  for (uint32_t k = 0; k < head; ++k) list(k);
  for (uint32_t k = head; k < nl; ++k) xl[k] = pf_layer_xfer{plans[order[k]].layout, nullptr, 0};
  // The later layers, made while the first ones copy.  A failure (the pool
  // exhausted) fails the call after the first layers' copy drained, with
  // nothing published, as a failure before any copy would.
  bool rest_made = head == nl;
  int rest_rc = PF_OK;
  std::string rest_error;
  PendingLayers pending;
  pending.head = head;
  pending.max_blocks = max_blocks;
  pending.ready = [&]() -> int {
    for (uint32_t k = head; k < nl; ++k) {
      if (int rc = place(plans[order[k]])) {
        rest_rc = rc;
        rest_error = pf_last_error();
        return rc;
      }
      list(k);
    }
    rest_made = true;
    return PF_OK;
  };
  // The LayerBlocks are built while the copy runs; they are published only
  // after it has completed (lib.rs:687-705, 755-770).
  std::vector<BlockStore::SlotEntries> entries(plans.size());
  struct GroupSeal {
    std::vector<size_t> slots;
    std::vector<BlockStore::SlotEntries> entries;
    BlockStore::Prepared prepared;
  };
  std::vector<GroupSeal> seals(groups.size());
  auto build_handles = [&] {
    for (size_t pi = 0; pi < plans.size(); ++pi) {
      const SavePlan& p = plans[pi];
      if (p.blocks.empty()) continue;
      const uint64_t seg = p.layout.bytes_per_block, bs = p.layout.block_size_bytes;
      auto set = std::make_shared<LayerBlockSet>();
      set->k_alloc = p.k_alloc;
      set->v_alloc = p.v_alloc;
      set->blocks.resize(p.key_idx.size());
      entries[pi].reserve(p.key_idx.size());
      for (size_t i = 0; i < p.key_idx.size(); ++i) {
        LayerBlock& lb = set->blocks[i];
        lb.size = bs;
        if (p.split) {
          lb.k_ptr = p.k_alloc->ptr + i * seg;
          lb.v_ptr = p.v_alloc->ptr + i * seg;
        } else {
          lb.k_ptr = p.k_alloc->ptr + i * bs;
        }
        entries[pi].emplace_back(p.key_idx[i], std::shared_ptr<LayerBlock>(set, &lb));
      }
    }
    // Per hash list, the slots it fills and, when they are all of its
    // blocks' slots, the complete blocks, ready to publish.
    for (size_t gi = 0; gi < groups.size(); ++gi) {
      GroupSeal& gs = seals[gi];
      for (size_t li : groups[gi].plans) {
        gs.slots.push_back(plans[li].slot);
        gs.entries.push_back(std::move(entries[li]));
      }
      gs.prepared = BlockStore::prepare_whole(gs.slots, gs.entries, total_slots);
      BlockStore::stage_nodes(groups[gi].keys, &gs.prepared);
    }
  };
  const auto t_planned = std::chrono::steady_clock::now();
  if (int rc = gpu->worker->save(xl, mode, build_handles, head < nl ? &pending : nullptr)) {
    if (rest_rc != PF_OK) return fail(rest_rc, rest_error);  // its own message
    return rc;
  }
  if (!rest_made)  // every transfer mode lists the later layers before it returns
    return fail(PF_ERR_STORAGE, "storage error: the later layers of a save were not planned");
  const auto t_copied = std::chrono::steady_clock::now();
  uint64_t bytes = 0;
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    for (size_t li : groups[gi].plans)
      bytes += plans[li].key_idx.size() * plans[li].layout.block_size_bytes;
    GroupSeal& gs = seals[gi];
    if (int rc = e->store->insert_slots(groups[gi].keys, gs.slots, gs.entries, total_slots,
                                        &gs.prepared))
      return fail(rc, std::string("storage error: ") + pf_last_error());
  }
  e->saved_bytes.fetch_add(bytes);
  if (tracing()) {
    const auto t_end = std::chrono::steady_clock::now();
    std::fprintf(stderr,
                 "[pegaflow] save instance=%s layers=%u bytes=%llu plan=%.0fus copy=%.0fus "
                 "publish=%.0fus total=%.0fus (%.2f GB/s)\n",
                 instance_id, num_layers, (unsigned long long)bytes, us_between(t_start, t_planned),
                 us_between(t_planned, t_copied), us_between(t_copied, t_end),
                 us_between(t_start, t_end), bytes / us_between(t_start, t_end) / 1e3);
  }
  return PF_OK;
}

// lib.rs:957-1069.
int pf_engine_batch_load(pf_engine* e, const char* instance_id, uint64_t tp_rank, int device_id,
                         const char* load_state_shm, const char* const* layer_names,
                         uint32_t num_layers, const int32_t* block_ids, const uint8_t* hash_data,
                         const uint64_t* hash_offsets, uint64_t n) {
  pf_load_state* state = nullptr;
  if (pf_load_state_attach(load_state_shm, &state))
    return fail(PF_ERR_LOAD_STATE, std::string("storage error: LoadState: ") + pf_last_error());
  std::shared_ptr<GpuContext> gpu;
  // A consumer's layer words are written even when nothing is copied, so
  // its device waits end; the LoadState says what happened.
  auto release_words = [&]() {
    LoadTask marks;
    marks.marks_only = true;
    (void)pf_load_state_layer_words(state, &marks.words, &marks.n_words);
    if (marks.n_words == 0 || !gpu) return;
    const std::string err = pf_last_error();
    (void)gpu->worker->submit(std::move(marks));
    set_error(err);
  };
  auto bail = [&](int code) {
    pf_load_state_set_error(state);
    release_words();
    pf_load_state_close(state);
    return code;
  };
  std::shared_ptr<Instance> inst;
  if (int rc = get_instance(e, instance_id, &inst)) return bail(rc);
  gpu = inst->gpu(device_id);
  if (!gpu)
    return bail(fail(PF_ERR_WORKER_MISSING,
                     strf("device %d not found in instance %s", device_id, instance_id)));
  LoadTask task;
  gpu->worker->take_spares(&task);
  const auto t_lookup = std::chrono::steady_clock::now();
  const long flt0 = tracing() ? thread_minor_faults() : 0;
  thread_local std::vector<std::string> keys;
  keys_into(inst->ns, hash_data, hash_offsets, n, &keys);
  if (e->store->lookup_many(keys, &task.keep))
    return bail(fail(PF_ERR_STORAGE, std::string("storage error: ") + pf_last_error()));
  const auto t_plan = std::chrono::steady_clock::now();
  // Every layer is resolved first (registration and slot), then the layers'
  // block lists are built block by block, so each sealed block's slot array
  // is read once, in order, rather than once per layer.
  struct LayerRef {
    pf_kv_layout reg;
    size_t slot;
    bool split;
  };
  std::vector<LayerRef> refs(num_layers);
  task.names.reserve(num_layers);
  for (uint32_t li = 0; li < num_layers; ++li) {
    std::string name(layer_names[li]);
    size_t layer_id = 0;
    if (!inst->layer_id(name, &layer_id))
      return bail(fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: layer " + name +
                                                    " unknown for instance " + instance_id));
    LayerRef& r = refs[li];
    {
      std::lock_guard<std::mutex> lk(gpu->mu);
      auto it = gpu->regs.find(name);
      if (it == gpu->regs.end())
        return bail(fail(PF_ERR_INVALID_ARGUMENT,
                         strf("invalid argument: layer %s not registered on device %d",
                              name.c_str(), device_id)));
      r.reg = it->second;
    }
    if (int rc = inst->slot_index(layer_id, tp_rank, &r.slot)) return bail(rc);
    r.split = r.reg.segments == 2 && r.reg.kv_stride_bytes > r.reg.bytes_per_block;
    task.names.push_back(std::move(name));
    task.layouts.push_back(r.reg);
  }
  const auto t_refs = std::chrono::steady_clock::now();
  const long flt1 = tracing() ? thread_minor_faults() : 0;
  // Block lists of layers [lo, hi) into out[0, hi - lo), built block by
  // block so that each sealed block's slot array is read once, in order.
  // Reads the task's sealed blocks and names through pointers that stay
  // valid when the task moves to the load thread.
  const std::shared_ptr<SealedBlock>* keep = task.keep.data();
  const std::string* names = task.names.data();
  auto build = [&](uint32_t lo, uint32_t hi, std::vector<pf_block_xfer>* out,
                   uint64_t* bytes) -> int {
    for (uint32_t li = lo; li < hi; ++li) {
      out[li - lo].clear();
      out[li - lo].reserve(static_cast<size_t>(n));
    }
    for (uint64_t j = 0; j < n; ++j) {
      if (block_ids[j] < 0) continue;
      const std::vector<SlotView>& views = keep[j]->views;
      for (uint32_t li = lo; li < hi; ++li) {
        const LayerRef& r = refs[li];
        if (r.slot >= views.size() || views[r.slot].size == 0) continue;
        const SlotView& lb = views[r.slot];
        if (lb.size != r.reg.block_size_bytes || (lb.v_ptr != nullptr) != r.split)
          return fail(PF_ERR_STORAGE,
                      strf("storage error: stored block at index %llu holds %llu %s bytes "
                           "for layer %s, which is registered with %llu %s bytes per block",
                           (unsigned long long)j, (unsigned long long)lb.size,
                           lb.v_ptr ? "split" : "contiguous", names[li].c_str(),
                           (unsigned long long)r.reg.block_size_bytes,
                           r.split ? "split" : "contiguous"));
        out[li - lo].push_back(pf_block_xfer{block_ids[j], reinterpret_cast<uint64_t>(lb.k_ptr),
                                             reinterpret_cast<uint64_t>(lb.v_ptr)});
        *bytes += lb.size;
      }
    }
    return PF_OK;
  };
  // A large kernel-mode or staged load is split: the lists of its first layers are
  // built and submitted, and this thread builds the rest while the load
  // thread copies those, so the first layers do not wait for the whole plan
  // (40-170 us for 640 blocks x 32 layers, varying with the core this thread
  // runs on).  The first part is the fewest leading layers whose copy
  // outlasts planning the rest: building the lists and the transfer's chunks
  // takes under 10 ns a block and layer, in which the host link moves about
  // 500 bytes.  For 640 Llama blocks that is one layer (0.74 ms of copy
  // against at most 0.25 ms of planning).  An error in the later layers
  // still fails the call and the LoadState, but the first layers may have
  // been copied by then.
  task.mode = e->load_mode.load();
  // Layer 0's list when built early (AUTO), kept as the task's.
  std::vector<pf_block_xfer> probe;
  uint64_t probe_bytes = 0;
  const bool probed = task.mode == PF_MODE_AUTO && num_layers > 0;
  if (probed) {
    // Blocks saved together lie alike in every layer: the first layer's
    // list decides, so a load resolved to the kernel mode is still split.
    if (int rc = build(0, 1, &probe, &probe_bytes)) return bail(rc);
    const pf_layer_xfer lx{refs[0].reg, probe.data(), probe.size()};
    task.mode = gpu->worker->resolve_load_mode(PF_MODE_AUTO, &lx, 1);
  }
  uint64_t chunks = 0;
  for (const LayerRef& r : refs) chunks += n * (r.split ? 2 : 1);
  uint32_t head = 0;
  if ((task.mode == PF_MODE_KERNEL || task.mode == PF_MODE_STAGED) &&
      pipeline_head_layers(num_layers, chunks) > 0) {
    constexpr uint64_t kHeadBytesPerLaterEntry = 500;
    uint64_t head_bytes = 0;
    for (head = 0; head + 1 < num_layers; ) {
      head_bytes += refs[head++].reg.block_size_bytes;
      if (head_bytes >= (num_layers - head) * kHeadBytesPerLaterEntry) break;
    }
  }
  task.blocks.resize(num_layers);
  uint32_t from = 0;
  if (probed) {
    task.blocks[0] = std::move(probe);
    task.bytes += probe_bytes;
    from = 1;
  }
  if (int rc = build(from, head ? head : num_layers, task.blocks.data() + from, &task.bytes))
    return bail(rc);
  bool any = false;
  for (uint32_t li = 0; li < (head ? head : num_layers); ++li)
    any = any || !task.blocks[li].empty();
  if (head && !any) {  // nothing in the first layers: built whole, not split
    if (int rc = build(head, num_layers, task.blocks.data() + head, &task.bytes))
      return bail(rc);
    for (uint32_t li = head; li < num_layers; ++li) any = any || !task.blocks[li].empty();
    head = 0;
  }
  const auto t_head = std::chrono::steady_clock::now();
  if (!any) {  // lib.rs:1055-1060
    pf_load_state_set_completed(state);
    release_words();
    pf_load_state_close(state);
    return PF_OK;
  }
  std::shared_ptr<LaterLayers> later;
  if (head) {
    later = std::make_shared<LaterLayers>();
    later->first = head;
    for (uint32_t li = head; li < num_layers; ++li)
      later->blocks.push_back(std::move(task.blocks[li]));
    task.blocks.resize(head);
    task.later = later;
  }
  task.state = state;
  task.submitted = std::chrono::steady_clock::now();
  if (int rc = gpu->worker->submit(std::move(task))) return bail(rc);
  // From here the load thread owns the LoadState and ends the load.
  int rc = PF_OK;
  if (later) {
    struct Publish {  // the load thread waits for this in every case
      LaterLayers& later;
      int rc = PF_ERR_STORAGE;
      std::string error = "storage error: the later layers of a load were not planned";
      ~Publish() { later.publish(rc, std::move(error)); }
    } publish{*later};
    publish.rc = rc = build(head, num_layers, later->blocks.data(), &later->bytes);
    publish.error = rc == PF_OK ? std::string() : std::string(pf_last_error());
  }
  if (tracing()) {
    const auto t_end = std::chrono::steady_clock::now();
    std::fprintf(stderr,
                 "[pegaflow] load plan instance=%s layers=%u blocks=%llu at=%.0fus lookup=%.0fus "
                 "plan=%.0fus (layers %.0fus, first %u) rest=%.0fus minor_faults=%ld+%ld\n",
                 instance_id, num_layers, (unsigned long long)n, mono_us(t_lookup),
                 us_between(t_lookup, t_plan), us_between(t_plan, t_head),
                 us_between(t_plan, t_refs), head ? head : num_layers,
                 us_between(t_head, t_end), flt1 - flt0, thread_minor_faults() - flt1);
  }
  return rc;
}

int pf_engine_stats_get(pf_engine* e, pf_engine_stats* out) {
  e->pool->usage(&out->pool_used_bytes, &out->pool_total_bytes);
  out->sealed_blocks = e->store->sealed_count();
  out->inflight_blocks = e->store->inflight_count();
  out->evicted_blocks = e->store->evictions();
  out->saved_bytes = e->saved_bytes.load();
  out->loaded_bytes = e->loaded_bytes.load();
  out->load_failures = e->load_failures.load();
  out->admission_rejections = e->store->admission_rejections();
  out->pre_evicted_blocks = e->pre_evicted.load();
  return PF_OK;
}

int pf_engine_enable_disk(pf_engine* e, const char* root, uint64_t quota_bytes,
                          uint32_t max_pack_blocks, uint32_t max_prefetch_tasks,
                          uint32_t io_threads) {
  if (!root) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: null disk root");
  std::lock_guard<std::mutex> lk(e->disk_mu);
  if (e->disk) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: disk tier already enabled");
  DiskConfig cfg;
  cfg.root = root;
  cfg.quota_bytes = quota_bytes;
  if (max_pack_blocks) cfg.max_pack_blocks = max_pack_blocks;
  if (max_prefetch_tasks) cfg.max_prefetch_tasks = max_prefetch_tasks;
  if (io_threads) cfg.io_threads = io_threads;
  if (int rc = DiskTier::open(cfg, e->store.get(), &e->disk)) return rc;
  DiskTier* d = e->disk.get();
  e->store->set_seal_hook(
      [d](const std::string& k, const std::shared_ptr<SealedBlock>& b) { d->on_seal(k, b); });
  return PF_OK;
}

int pf_engine_query_prefetch(pf_engine* e, const char* instance_id, const uint8_t* hash_data,
                             const uint64_t* hash_offsets, uint64_t n, pf_prefetch_status* out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: null output");
  *out = pf_prefetch_status{};
  if (!e->disk) {
    out->state = PF_PREFETCH_READY;
    return pf_engine_count_prefix_hit_blocks(e, instance_id, hash_data, hash_offsets, n,
                                             &out->hit_blocks);
  }
  std::shared_ptr<Instance> inst;
  if (int rc = get_instance(e, instance_id, &inst)) return rc;
  int state = 0;
  e->disk->query(keys_of(inst->ns, hash_data, hash_offsets, n), &state, &out->hit_blocks,
                 &out->loading_blocks, &out->missing_blocks);
  out->state = state;
  return PF_OK;
}

int pf_engine_disk_flush(pf_engine* e) {
  if (e->disk) e->disk->flush();
  return PF_OK;
}

int pf_engine_disk_wait_prefetch(pf_engine* e) {
  if (e->disk) e->disk->wait_prefetch();
  return PF_OK;
}

int pf_engine_disk_stats(pf_engine* e, pf_disk_stats* out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: null output");
  *out = pf_disk_stats{};
  if (!e->disk) return PF_OK;
  const DiskStats s = e->disk->stats();
  out->files = s.files;
  out->bytes = s.bytes;
  out->indexed_blocks = s.indexed_blocks;
  out->offloaded_blocks = s.offloaded_blocks;
  out->written_bytes = s.written_bytes;
  out->prefetched_blocks = s.prefetched_blocks;
  out->read_bytes = s.read_bytes;
  out->pending_blocks = s.pending_blocks;
  out->evicted_files = s.evicted_files;
  out->failures = s.failures;
  return PF_OK;
}

int pf_engine_read_block_slot(pf_engine* e, const char* ns, const uint8_t* hash,
                              uint64_t hash_len, uint64_t slot, uint8_t* dst, uint64_t dst_len,
                              uint64_t* k_bytes, uint64_t* v_bytes) {
  if (!ns || (!hash && hash_len)) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: null key");
  auto sb = e->store->peek(block_key(ns, hash, static_cast<size_t>(hash_len)));
  if (!sb)
    return fail(PF_ERR_STORAGE, strf("storage error: block not cached (namespace=%s, hash_len=%llu)",
                                     ns, (unsigned long long)hash_len));
  if (slot >= sb->slots.size() || !sb->slots[slot])
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("invalid argument: slot %llu out of range (%zu slots)",
                     (unsigned long long)slot, sb->slots.size()));
  const LayerBlock& lb = *sb->slots[slot];
  const uint64_t k = lb.v_ptr ? lb.size / 2 : lb.size, v = lb.v_ptr ? lb.size / 2 : 0;
  if (k_bytes) *k_bytes = k;
  if (v_bytes) *v_bytes = v;
  if (!dst) return PF_OK;
  if (dst_len < k + v)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("invalid argument: slot holds %llu bytes, buffer %llu",
                     (unsigned long long)(k + v), (unsigned long long)dst_len));
  std::memcpy(dst, lb.k_ptr, k);
  if (v) std::memcpy(dst + k, lb.v_ptr, v);
  return PF_OK;
}

int pf_engine_wait_idle(pf_engine* e) {
  std::vector<std::shared_ptr<DeviceWorker>> workers;
  {
    std::shared_lock<std::shared_mutex> lk(e->mu);
    for (auto& kv : e->instances) {
      std::shared_lock<std::shared_mutex> g(kv.second->gpus_mu);
      for (auto& gk : kv.second->gpus) workers.push_back(gk.second->worker);
    }
  }
  for (auto& w : workers) w->wait_idle();
  return PF_OK;
}

}  // extern "C"
