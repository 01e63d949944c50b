// pf_lfu.h — TinyLFU admission for the block store's cache (cache.rs:28-241),
// in a header of its own so its rules are tested on the host
// (tests/native/lfu_test.cpp).
//
// A count-min sketch of 8-bit saturating counters estimates how often each
// key was recorded; every `window` recordings all counters are halved.  The
// cache records a key on every insert attempt and on every lookup hit, and
// refuses a new key whose estimate is below that of its least recently used
// entry.  Sizing follows the reference: for `items` expected entries
// (capacity / value-size hint, 128 MiB by default: cache.rs:14, 36-47), a
// width of max(ceil(e * items), 16) counters, a depth of
// max(ceil(log2(items)), 2) rows (cache.rs:104-123, from the count-min
// bounds with error and failure probability 1/items) and a window of
// 8 * items (cache.rs:22, 232-238).  Each row hashes the key with a seed of
// its own; the reference draws its hashers at random per process, so which
// keys collide differs from run to run there as here.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

namespace pf {

class TinyLfu {
 public:
  static void sizing(uint64_t items, uint64_t* width, uint64_t* depth) {
    items = std::max<uint64_t>(items, 1);
    const double n = static_cast<double>(items);
    *width = std::max<uint64_t>(static_cast<uint64_t>(std::ceil(std::exp(1.0) * n)), 16);
    // ln(1/n) / ln(1/2) = log2(n); 0 for one item.
    const double d = std::ceil(std::log(1.0 / n) / std::log(0.5));
    *depth = std::max<uint64_t>(d > 0 ? static_cast<uint64_t>(d) : 0, 2);
  }

  TinyLfu(uint64_t items, uint64_t seed) {
    items = std::max<uint64_t>(items, 1);
    sizing(items, &width_, &depth_);
    window_ = 8 * items;
    counters_.assign(width_ * depth_, 0);
    seeds_.resize(depth_);
    uint64_t s = seed;
    for (uint64_t& r : seeds_) r = mix(s += 0x9E3779B97F4A7C15ull);
  }

  // Records one access of `key` (cache.rs:221-228): ages the sketch when the
  // window is full (the count of recordings before this one equals the
  // window, or passed twice the window), then adds one to the key's counter
  // in every row, saturating at 255.  Returns the key's new estimate.
  uint8_t incr(const std::string& key) {
    const uint64_t before = recorded_++;
    if (before == window_ || before > 2 * window_) {
      recorded_ = 0;
      for (uint8_t& c : counters_) c = static_cast<uint8_t>(c >> 1);
    }
    const uint64_t h = hash(key);
    uint8_t est = 255;
    for (uint64_t r = 0; r < depth_; ++r) {
      uint8_t& c = counters_[r * width_ + slot(h, r)];
      if (c < 255) ++c;
      est = std::min(est, c);
    }
    return est;
  }

  // The key's estimate: the least of its row counters (cache.rs:170-179).
  uint8_t get(const std::string& key) const {
    const uint64_t h = hash(key);
    uint8_t est = 255;
    for (uint64_t r = 0; r < depth_; ++r)
      est = std::min(est, counters_[r * width_ + slot(h, r)]);
    return est;
  }

  uint64_t width() const { return width_; }
  uint64_t depth() const { return depth_; }
  uint64_t window() const { return window_; }

 private:
  static uint64_t mix(uint64_t z) {  // splitmix64's finalizer
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  static uint64_t hash(const std::string& key) {  // FNV-1a, 64-bit
    uint64_t h = 0xCBF29CE484222325ull;
    for (unsigned char ch : key) {
      h ^= ch;
      h *= 0x100000001B3ull;
    }
    return h;
  }
  uint64_t slot(uint64_t h, uint64_t row) const { return mix(h ^ seeds_[row]) % width_; }

  uint64_t width_ = 16, depth_ = 2, window_ = 8;
  uint64_t recorded_ = 0;
  std::vector<uint8_t> counters_;
  std::vector<uint64_t> seeds_;
};

}  // namespace pf
