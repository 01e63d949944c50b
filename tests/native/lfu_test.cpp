// lfu_test.cpp — TinyLFU's sketch (pf_lfu.h) on the host: the reference's
// sizing (cache.rs:104-123, 232-238) in closed form, the count-min property
// against exact counts, halving at the window's end, saturation, and the
// share of new blocks the reference's default admission refuses under a
// save/load mix of KV blocks (printed).
// Exit status 0 and "ok" on success; the first failed checks are printed.
#include <array>
#include <cstdio>
#include <list>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "pf_lfu.h"

using namespace pf;

namespace {

int failures = 0;

void expect(bool cond, const std::string& what) {
  if (!cond && ++failures <= 20) std::printf("FAILED: %s\n", what.c_str());
}

}  // namespace

int main() {
  // Width ceil(e * n) (at least 16), depth ceil(log2 n) (at least 2).
  const uint64_t table[][3] = {{1, 16, 2}, {2, 16, 2}, {5, 16, 3}, {62, 169, 6},
                               {240, 653, 8}, {100000, 271829, 17}};
  for (const auto& t : table) {
    uint64_t w = 0, d = 0;
    TinyLfu::sizing(t[0], &w, &d);
    expect(w == t[1] && d == t[2], "sizing for " + std::to_string(t[0]) + " items: " +
                                       std::to_string(w) + " x " + std::to_string(d));
  }
  {
    TinyLfu s(240, 1);
    expect(s.width() == 653 && s.depth() == 8 && s.window() == 1920, "a 240-item sketch");
  }
  // Count-min: an estimate never falls below the true count, and in a wide
  // sketch it is exact for nearly every key (7,999 recordings, below the
  // 8,000-record window of 1,000 items).
  {
    TinyLfu s(1000, 42);
    std::mt19937_64 rng(3);
    std::unordered_map<std::string, int> truth;
    std::vector<std::string> keys;
    for (int i = 0; i < 2000; ++i) keys.push_back("ns" + std::string(1, '\0') + std::to_string(i));
    for (int r = 0; r < 7999; ++r) {
      const std::string& k = keys[rng() % keys.size()];
      ++truth[k];
      s.incr(k);
    }
    int exact = 0, under = 0;
    for (const auto& k : keys) {
      const int t = truth.count(k) ? truth[k] : 0;
      const int e = s.get(k);
      under += e < t;
      exact += e == t;
    }
    expect(under == 0, "no estimate below its count (" + std::to_string(under) + ")");
    expect(exact >= 1980, "estimates exact for " + std::to_string(exact) + " of 2000 keys");
  }
  // Halving: 4 items record a window of 32.  Recordings 1..32 count up; the
  // 33rd finds 32 recorded, halves every counter and then adds its own; the
  // count restarts from 0, so the 66th halves again.
  {
    TinyLfu s(4, 9);
    const std::string a = "a";
    for (int i = 0; i < 32; ++i) s.incr(a);
    expect(s.get(a) == 32, "32 recordings");
    expect(s.incr(a) == 17, "the 33rd recording halves, then adds");
    for (int i = 0; i < 32; ++i) s.incr(a);
    expect(s.get(a) == 49, "a full window more");
    expect(s.incr(a) == 25, "the next window's end halves again");
  }
  // Saturation at 255 (a window of 8,000 is not reached).
  {
    TinyLfu s(1000, 5);
    for (int i = 0; i < 300; ++i) s.incr("hot");
    expect(s.get("hot") == 255, "counters saturate at 255");
    expect(s.get("cold") == 0, "an unrecorded key reads 0 in a wide sketch");
  }
  // The reference's default admission (cache.rs:71-95, sized for 128 MiB
  // values) on a pool of 2 MiB blocks (a Llama-3.1-8B block of 32 layers):
  // batches of new blocks saved, and after every other batch one of the last
  // eight batches loaded (hits recorded, moved to most recent); the cache
  // evicts its least recently used block when full.  Printed: the share of
  // new blocks refused.
  for (const auto& c : std::vector<std::array<uint64_t, 2>>{{30, 640}, {8, 640}, {30, 64}}) {
    const uint64_t pool = c[0] << 30, blocks = pool / (2ull << 20), batch = c[1];
    TinyLfu s(pool / (128ull << 20), 11);
    std::list<uint64_t> lru;  // front = most recent
    std::unordered_map<uint64_t, std::list<uint64_t>::iterator> where;
    std::vector<std::vector<uint64_t>> saved;
    std::mt19937_64 rng(5);
    uint64_t next = 0, refused = 0, offered = 0;
    auto name = [](uint64_t k) { return "ns" + std::string(1, '\0') + std::to_string(k); };
    for (int b = 0; b < 200; ++b) {
      std::vector<uint64_t> keys;
      for (uint64_t i = 0; i < batch; ++i) {
        const uint64_t k = next++;
        keys.push_back(k);
        while (lru.size() >= blocks) {
          where.erase(lru.back());
          lru.pop_back();
        }
        ++offered;
        s.incr(name(k));
        if (!lru.empty() && s.get(name(k)) < s.get(name(lru.back()))) {
          ++refused;
          continue;
        }
        lru.push_front(k);
        where[k] = lru.begin();
      }
      saved.push_back(keys);
      if (b % 2 == 1) {
        const size_t lo = saved.size() > 8 ? saved.size() - 8 : 0;
        for (uint64_t k : saved[lo + rng() % (saved.size() - lo)]) {
          auto it = where.find(k);
          if (it == where.end()) continue;
          lru.splice(lru.begin(), lru, it->second);
          s.incr(name(k));
        }
      }
    }
    const double share = double(refused) / double(offered);
    std::printf("default admission, %llu GiB pool of 2 MiB blocks, batches of %llu: %.1f%% of "
                "new blocks refused\n",
                (unsigned long long)c[0], (unsigned long long)batch, 100.0 * share);
    expect(share > 0.02 && share < 0.6, "refused share " + std::to_string(share));
  }
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
