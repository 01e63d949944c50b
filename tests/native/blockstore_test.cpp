// blockstore_test.cpp — the block store's sealing rules, on the host (no GPU),
// built by tests/test_native.py from the library's own sources.
//
// A block seals when every one of its slots (layer x tensor-parallel rank)
// has arrived (storage.rs:160-193, 457-514): a slot already present keeps
// its first copy, a block sealed earlier is not replaced, and one call may
// bring a whole block at once.  Checked here through BlockStore directly:
//   1. a call bringing every slot of its blocks (slots in a permuted order);
//   2. a block partly in flight from an earlier call, completed by a call
//      that brings all slots (the earlier copies win);
//   3. a block sealed earlier, saved again (unchanged);
//   4. one key named twice in a call (the first occurrence seals);
//   5. a slot count that differs from the block's in flight (an error);
//   6. the engine's own publishing of a whole call, with the cache nodes
//      made ahead (prepare_whole + stage_nodes, as a save does while its
//      copy runs): a fresh key, a key sealed meanwhile, a key an earlier call
//      left in flight, a key named twice; then the recency order those
//      blocks took, read through eviction;
//   7. TinyLFU admission (cache.rs:71-95): a new key colder than the least
//      recently used entry is refused, one as warm is let in, lookup hits
//      warm a key, blocks read back from disk go through it too, and with
//      admission off every key enters;
//   8. eviction by bytes (storage.rs:610-644, the pre-eviction monitor's
//      step): least recently used blocks until their footprints reach the
//      request;
//   9. allocation racing a monitor thread's evictions: no allocation fails
//      while memory the monitor took out of the cache is still returning.
// Exit status 0 and "ok" on success; the first failed check is printed.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <thread>
#include <string>
#include <vector>

#include "pf_engine.h"

using namespace pf;

namespace {

int failures = 0;

void expect(bool cond, const char* what) {
  if (!cond) {
    std::printf("FAILED: %s\n", what);
    ++failures;
  }
}

// One layer block per (slot, key) with a recognisable address.
std::shared_ptr<LayerBlock> block(uint64_t tag) {
  auto b = std::make_shared<LayerBlock>();
  b->k_ptr = reinterpret_cast<uint8_t*>(tag);
  b->size = 64;
  return b;
}

uint64_t tag_of(const std::shared_ptr<LayerBlock>& b) {
  return b ? reinterpret_cast<uint64_t>(b->k_ptr) : 0;
}

// entries[j] for slot slots[j]: every key index in `idx`, tagged
// call * 1000 + slot * 10 + key index.
std::vector<BlockStore::SlotEntries> entries_for(const std::vector<size_t>& slots,
                                                 const std::vector<uint32_t>& idx, int call) {
  std::vector<BlockStore::SlotEntries> e(slots.size());
  for (size_t j = 0; j < slots.size(); ++j)
    for (uint32_t i : idx) e[j].emplace_back(i, block(call * 1000 + slots[j] * 10 + i + 1));
  return e;
}

}  // namespace

int main() {
  std::shared_ptr<PinnedPool> pool;
  if (PinnedPool::create(1 << 20, 0, false, 0, &pool)) {
    std::printf("FAILED: pool: %s\n", pf_last_error());
    return 1;
  }
  BlockStore store(pool);
  const size_t total = 4;
  // Keys as the engine builds them: namespace, a zero byte, the hash.
  auto key = [](int i) { return std::string("ns") + '\0' + "hash" + std::to_string(i); };
  const std::vector<std::string> keys = {key(0), key(1), key(2), key(3)};

  // 1. Every slot of keys 0 and 1 in one call, slots in a permuted order.
  {
    std::vector<size_t> slots = {2, 0, 3, 1};
    auto e = entries_for(slots, {0, 1}, 1);
    expect(store.insert_slots(keys, slots, e, total) == PF_OK, "whole call");
    for (uint32_t i : {0u, 1u}) {
      auto sb = store.peek(keys[i]);
      expect(sb && sb->slots.size() == total, "whole call seals its blocks");
      if (!sb) continue;
      for (size_t s = 0; s < total; ++s)
        expect(tag_of(sb->slots[s]) == 1000 + s * 10 + i + 1, "slot s holds the copy for slot s");
      expect(sb->footprint == total * 64, "footprint");
    }
    expect(store.inflight_count() == 0, "nothing left in flight");
  }
  // 2. Key 2: slots 0 and 1 first (in flight), then a call with all slots.
  {
    std::vector<size_t> half = {0, 1};
    auto e = entries_for(half, {2}, 2);
    expect(store.insert_slots(keys, half, e, total) == PF_OK, "partial call");
    expect(!store.peek(keys[2]) && store.inflight_count() == 1, "partial block stays in flight");
    std::vector<size_t> all = {0, 1, 2, 3};
    auto e2 = entries_for(all, {2}, 3);
    expect(store.insert_slots(keys, all, e2, total) == PF_OK, "completing call");
    auto sb = store.peek(keys[2]);
    expect(sb != nullptr && store.inflight_count() == 0, "completed block seals");
    if (sb) {
      expect(tag_of(sb->slots[0]) == 2000 + 0 + 3 && tag_of(sb->slots[1]) == 2000 + 10 + 3,
             "slots present in flight keep their first copy");
      expect(tag_of(sb->slots[2]) == 3000 + 20 + 3 && tag_of(sb->slots[3]) == 3000 + 30 + 3,
             "missing slots come from the completing call");
      expect(sb->footprint == total * 64, "footprint counts every slot once");
    }
  }
  // 3. Key 1 saved again: the sealed block is not replaced.
  {
    auto before = store.peek(keys[1]);
    std::vector<size_t> all = {0, 1, 2, 3};
    auto e = entries_for(all, {1}, 4);
    expect(store.insert_slots(keys, all, e, total) == PF_OK, "save of a sealed key");
    expect(store.peek(keys[1]) == before, "sealed block unchanged");
  }
  // 4. Key 3 named twice (indices 3 and 4 of the call's key list).
  {
    std::vector<std::string> dup = keys;
    dup.push_back(keys[3]);
    std::vector<size_t> all = {0, 1, 2, 3};
    auto e = entries_for(all, {3, 4}, 5);
    expect(store.insert_slots(dup, all, e, total) == PF_OK, "duplicate key");
    auto sb = store.peek(keys[3]);
    expect(sb && tag_of(sb->slots[0]) == 5000 + 0 + 3 + 1, "first occurrence seals");
    expect(store.sealed_count() == 4, "four keys sealed");
  }
  // 5. A block in flight with 4 slots, then a call that counts 5.
  {
    const std::vector<std::string> k5 = {key(5)};
    std::vector<size_t> one = {0};
    auto e = entries_for(one, {0}, 6);
    expect(store.insert_slots(k5, one, e, total) == PF_OK, "partial call (4 slots)");
    std::vector<size_t> other = {1};
    auto e2 = entries_for(other, {0}, 7);
    expect(store.insert_slots(k5, other, e2, total + 1) != PF_OK, "slot count mismatch refused");
    expect(std::string(pf_last_error()).find("slot count mismatch") != std::string::npos,
           "the reference's message");
  }
  // 6. Staged publishing.  Keys 10-13: 10 fresh, 11 sealed by another call
  //    after this one was prepared, 12 left in flight (slot 0) by an earlier
  //    call, and 10 named again as index 4.
  {
    std::vector<std::string> k6 = {key(10), key(11), key(12), key(13), key(10)};
    const std::vector<size_t> one = {0};
    auto early = entries_for(one, {2}, 8);
    expect(store.insert_slots(k6, one, early, total) == PF_OK, "earlier partial call");
    const std::vector<size_t> all = {3, 1, 0, 2};
    auto e = entries_for(all, {0, 1, 2, 3, 4}, 9);
    BlockStore::Prepared prep = BlockStore::prepare_whole(all, e, total);
    expect(prep.blocks.size() == 5, "five complete blocks prepared");
    BlockStore::stage_nodes(k6, &prep);
    expect(prep.nodes.size() == 4 && prep.order.size() == 4, "one node per distinct key");
    auto other = entries_for(all, {1}, 10);  // key 11 seals through another call
    expect(store.insert_slots(k6, all, other, total) == PF_OK, "another call seals key 11");
    auto sealed11 = store.peek(k6[1]);
    const uint64_t before = store.sealed_count();
    expect(store.insert_slots(k6, all, e, total, &prep) == PF_OK, "staged publish");
    expect(store.sealed_count() == before + 3, "keys 10, 12 and 13 sealed");
    expect(store.peek(k6[1]) == sealed11, "the block sealed meanwhile stays");
    auto b10 = store.peek(k6[0]);
    expect(b10 && tag_of(b10->slots[3]) == 9000 + 30 + 0 + 1, "a key named twice keeps its first");
    auto b12 = store.peek(k6[2]);
    expect(b12 && tag_of(b12->slots[0]) == 8000 + 0 + 2 + 1 &&
               tag_of(b12->slots[1]) == 9000 + 10 + 2 + 1,
           "the in-flight key keeps its earlier slot and takes the rest");
    expect(store.inflight_count() == 1, "only key 5 of check 5 is left in flight");
    expect(prep.nodes.empty() && prep.blocks.empty(), "the prepared call is consumed");
    // Recency: evicting all but three leaves the three most recent: key 12
    // (sealed through the in-flight path, last), then 13 and 10 (the staged
    // nodes, most recent first).
    const uint64_t n = store.sealed_count();
    expect(store.evict_lru(n - 3) == n - 3, "eviction");
    expect(store.peek(k6[2]) && store.peek(k6[3]) && store.peek(k6[0]),
           "the staged and completed blocks are the most recent");
    expect(store.evict_lru(1) == 1 && !store.peek(k6[0]) && store.peek(k6[3]),
           "key 10, staged first, is the older of the staged two");
  }
  // 7. Admission, on a store of its own.
  {
    BlockStore lfu(pool);
    lfu.set_admission(1000, 7);  // a wide sketch: no collisions among these keys
    std::vector<std::string> k7 = {key(20), key(21), key(22)};
    std::vector<size_t> all = {0, 1, 2, 3};
    auto seal = [&](uint32_t i, int call) {
      auto e = entries_for(all, {i}, call);
      return lfu.insert_slots(k7, all, e, total);
    };
    std::vector<std::shared_ptr<SealedBlock>> got;
    expect(seal(0, 20) == PF_OK && lfu.sealed_count() == 1, "the first key enters an empty cache");
    expect(lfu.lookup_many({k7[0]}, &got) == PF_OK && lfu.lookup_many({k7[0]}, &got) == PF_OK,
           "two hits");
    // Key 20 is the least recently used entry, recorded three times; key 21,
    // recorded once, is colder: refused, and a lookup of it misses.
    expect(seal(1, 21) == PF_OK && lfu.sealed_count() == 1 && lfu.admission_rejections() == 1,
           "a colder key is refused");
    expect(lfu.lookup_many({k7[1]}, &got) != PF_OK, "a refused key is not in the cache");
    expect(lfu.inflight_count() == 0, "a refused block does not stay in flight");
    // Offered again it is recorded again: twice is still colder, three
    // times as warm as key 20 (3): let in.
    expect(seal(1, 22) == PF_OK && lfu.sealed_count() == 1, "still colder");
    expect(seal(1, 23) == PF_OK && lfu.sealed_count() == 2 && lfu.admission_rejections() == 2,
           "as warm as the least recently used entry: let in");
    // A block read back from disk is offered the same way.  Key 20 is now
    // the least recently used entry (3 records); key 22 has none yet.
    auto sb = std::make_shared<SealedBlock>();
    sb->slots.resize(total);
    expect(!lfu.cache_insert(k7[2], sb) && lfu.admission_rejections() == 3,
           "a cold block from disk is refused");
    lfu.set_admission(0, 0);
    expect(lfu.cache_insert(k7[2], sb) && lfu.sealed_count() == 3, "admission off: it enters");
  }
  // 8. Eviction by bytes.  Every block of check 7's store layout holds four
  // 64-byte slots (256 bytes of footprint).
  {
    BlockStore ev(pool);
    std::vector<std::string> k8;
    for (int i = 0; i < 6; ++i) k8.push_back(key(30 + i));
    std::vector<size_t> all = {0, 1, 2, 3};
    auto e = entries_for(all, {0, 1, 2, 3, 4, 5}, 30);
    expect(ev.insert_slots(k8, all, e, total) == PF_OK && ev.sealed_count() == 6, "six blocks");
    uint64_t freed = 0;
    expect(ev.evict_bytes(600, &freed) == 3 && freed == 768, "three blocks free 768 >= 600 bytes");
    expect(!ev.peek(k8[0]) && !ev.peek(k8[2]) && ev.peek(k8[3]), "the oldest three went");
    expect(ev.evict_bytes(1 << 20, &freed) == 3 && freed == 768 && ev.sealed_count() == 0,
           "a request past the cache empties it");
    expect(ev.evict_bytes(0, &freed) == 0 && freed == 0, "nothing asked, nothing evicted");
  }
  // 9. Eviction racing allocation.  A saver thread fills a pool of its own
  // with sealed blocks (eight 8 KiB blocks sharing one 64 KiB allocation
  // per call), while a monitor thread, as the pre-eviction monitor does,
  // evicts whenever little is free.  Nothing but the cache and the saver's
  // own current allocation holds pool memory, so every allocation must
  // succeed, including one made while the monitor is still returning the
  // memory of blocks it has just taken out of the cache; and once the
  // cache is emptied, no memory may stay in use.  Run with admission off
  // and on (refused blocks must return their memory too).
  for (int lfu_on = 0; lfu_on < 2; ++lfu_on) {
    std::shared_ptr<PinnedPool> small;
    if (PinnedPool::create(1 << 20, 0, false, 0, &small)) {
      std::printf("FAILED: pool: %s\n", pf_last_error());
      return 1;
    }
    BlockStore race(small);
    if (lfu_on) race.set_admission(128, 9);
    std::atomic<bool> stop{false};
    std::atomic<uint64_t> failed{0}, calls{0}, monitor_evicted{0};
    std::thread monitor([&] {
      while (!stop.load()) {
        uint64_t used = 0, total_bytes = 0;
        small->usage(&used, &total_bytes);
        if (total_bytes - used < (128u << 10)) monitor_evicted += race.evict_bytes(~0ull, nullptr);
      }
    });
    std::vector<size_t> one = {0};
    std::vector<std::shared_ptr<SealedBlock>> hits;
    const auto until = std::chrono::steady_clock::now() + std::chrono::milliseconds(1000);
    for (uint32_t call = 0; std::chrono::steady_clock::now() < until; ++call) {
      auto a = race.allocate(64u << 10);
      if (!a) {
        ++failed;
        continue;
      }
      std::vector<std::string> keys;
      std::vector<BlockStore::SlotEntries> e(1);
      for (uint32_t i = 0; i < 8; ++i) {
        keys.push_back(key(1000000 + static_cast<int>(call * 8 + i)));
        auto b = std::make_shared<LayerBlock>();
        b->k_ptr = a->ptr + i * (8u << 10);
        b->size = 8u << 10;
        b->k_alloc = a;
        e[0].emplace_back(i, std::move(b));
      }
      a.reset();
      if (race.insert_slots(keys, one, e, 1) != PF_OK) ++failed;
      // Some hits, so admission has warm entries to weigh new keys against.
      if (call % 3 == 0) (void)race.lookup_many({keys[0]}, &hits);
      hits.clear();
      ++calls;
    }
    stop = true;
    monitor.join();
    race.evict_bytes(~0ull, nullptr);
    uint64_t used = 0, total_bytes = 0;
    small->usage(&used, &total_bytes);
    std::printf("eviction race (admission %s): %llu calls, %llu blocks evicted by the monitor, "
                "%llu refused, %llu failed, %llu bytes in use after evicting everything\n",
                lfu_on ? "on" : "off", (unsigned long long)calls.load(),
                (unsigned long long)monitor_evicted.load(),
                (unsigned long long)race.admission_rejections(),
                (unsigned long long)failed.load(), (unsigned long long)used);
    expect(calls.load() > 1000 && monitor_evicted.load() > 0, "the race ran");
    expect(!lfu_on || race.admission_rejections() > 0, "admission refused some blocks");
    expect(failed.load() == 0, "no allocation fails while evicted memory is returning");
    expect(used == 0, "every evicted or refused block returned its memory");
  }
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
