// stress_engine.cpp — concurrency stress of the engine's host side, built
// with ThreadSanitizer or AddressSanitizer+UBSan by tests/test_native.py.
//
// A host-memory pool engine (no GPU, no HIP call) with a disk tier over packed
// files written here: several threads query prefixes (starting prefetches that
// allocate from a pool small enough to evict constantly), count prefixes, read
// cached slots and check every byte, read statistics, register and
// unregister an instance, and turn TinyLFU admission and the pre-eviction
// monitor on and off, all at once.  Exit status 0 = every byte read back
// was right and the engine shut down cleanly; a sanitizer report fails the run
// through its own exit code.
#include <sys/stat.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "pegaflow_hip.h"

namespace {

constexpr int kFiles = 8;
constexpr int kBlocksPerFile = 32;
constexpr int kBlocks = kFiles * kBlocksPerFile;
constexpr int kSlots = 4;            // 2 layers x tp 2
constexpr uint64_t kSeg = 2048;      // bytes per K (or V) half
constexpr uint64_t kSlotBytes = 2 * kSeg;
constexpr uint64_t kBlockBytes = kSlots * kSlotBytes;

uint8_t byte_of(int block, int slot, uint64_t i) {
  uint64_t z = (uint64_t)block * 0x9E3779B97F4A7C15ull + (uint64_t)slot * 0xBF58476D1CE4E5B9ull + i;
  z ^= z >> 29;
  z *= 0x94D049BB133111EBull;
  return static_cast<uint8_t>(z >> 56);
}

std::string hash_of(int block) {
  std::string h(16, '\0');
  for (int i = 0; i < 16; ++i) h[i] = static_cast<char>((block * 131 + i * 7) & 0xff);
  return h;
}

std::string hex(const std::string& s) {
  static const char* d = "0123456789abcdef";
  std::string o;
  for (unsigned char c : s) {
    o.push_back(d[c >> 4]);
    o.push_back(d[c & 15]);
  }
  return o;
}

bool write_all(const std::string& path, const std::string& data) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) return false;
  const bool ok = std::fwrite(data.data(), 1, data.size(), f) == data.size();
  return std::fclose(f) == 0 && ok;
}

// Packed files in the disk tier's format, plus their sidecars.
bool write_files(const std::string& root) {
  const std::string dir = root + "/stress";
  ::mkdir(root.c_str(), 0755);
  ::mkdir(dir.c_str(), 0755);
  for (int f = 0; f < kFiles; ++f) {
    char uuid[64];
    std::snprintf(uuid, sizeof(uuid), "00000000-0000-4000-8000-%012d", f + 1);
    std::string data, side = std::string("{\"version\":1,\"namespace\":\"stress\",\"file\":\"") +
                             uuid + ".bin\",\"size\":" +
                             std::to_string(kBlocksPerFile * kBlockBytes) + ",\"blocks\":[";
    for (int j = 0; j < kBlocksPerFile; ++j) {
      const int b = f * kBlocksPerFile + j;
      for (int s = 0; s < kSlots; ++s)
        for (uint64_t i = 0; i < kSlotBytes; ++i) data.push_back(static_cast<char>(byte_of(b, s, i)));
      if (j) side += ",";
      side += "{\"hash\":\"" + hex(hash_of(b)) + "\",\"meta\":{\"file\":\"" + uuid +
              ".bin\",\"offset\":" + std::to_string(j * kBlockBytes) + ",\"slots\":[";
      for (int s = 0; s < kSlots; ++s)
        side += std::string(s ? "," : "") + "{\"is_split\":true,\"size\":" +
                std::to_string(kSlotBytes) + "}";
      side += "],\"total_slots\":" + std::to_string(kSlots) + "}}";
    }
    side += "]}";
    if (!write_all(dir + "/" + uuid + ".bin", data) || !write_all(dir + "/" + uuid + ".json", side))
      return false;
  }
  return true;
}

struct Hashes {
  std::vector<uint8_t> data;
  std::vector<uint64_t> offs{0};
  void add(const std::string& h) {
    data.insert(data.end(), h.begin(), h.end());
    offs.push_back(data.size());
  }
  uint64_t n() const { return offs.size() - 1; }
};

int reg(pf_engine* e, const char* inst) {
  for (int l = 0; l < 2; ++l) {
    const std::string name = "layer." + std::to_string(l);
    for (int r = 0; r < 2; ++r)
      if (int rc = pf_engine_register_context_layer(e, inst, "stress", 0, name.c_str(), 0x100000,
                                                    2 * 64 * kSeg, 64, kSeg, 64 * kSeg, 2, r, 2,
                                                    2))
        return rc;
  }
  return PF_OK;
}

}  // namespace

int main(int argc, char** argv) {
  const double seconds = argc > 2 ? std::atof(argv[2]) : 2.0;
  const std::string root = argc > 1 ? argv[1] : "/tmp/pf_stress";
  if (!write_files(root)) {
    std::fprintf(stderr, "cannot write packed files under %s\n", root.c_str());
    return 2;
  }
  pf_engine* e = nullptr;
  // 40 blocks fit: prefetching the 256 on disk evicts all the time.
  if (pf_engine_create(40 * kBlockBytes, PF_POOL_HOST, 0, 256, &e) ||
      pf_engine_enable_disk(e, root.c_str(), 1ull << 40, 16, 4, 3) || reg(e, "a") ||
      reg(e, "b")) {
    std::fprintf(stderr, "setup failed: %s\n", pf_last_error());
    return 2;
  }
  std::atomic<bool> stop{false};
  std::atomic<uint64_t> bad{0}, slot_reads{0}, queries{0};
  std::vector<std::thread> threads;
  auto until_stop = [&](auto body) {
    return [&, body]() mutable {
      while (!stop.load()) body();
    };
  };
  for (int t = 0; t < 3; ++t)  // prefix queries that start prefetches
    threads.emplace_back([&, t] {
      std::mt19937 rng(t + 1);
      while (!stop.load()) {
        Hashes hs;
        const int start = rng() % kBlocks, len = 1 + rng() % 48;
        for (int i = 0; i < len; ++i) hs.add(hash_of((start + i) % kBlocks));
        pf_prefetch_status st{};
        if (pf_engine_query_prefetch(e, t % 2 ? "a" : "b", hs.data.data(), hs.offs.data(), hs.n(),
                                     &st) == PF_OK)
          queries.fetch_add(1);
        if (st.hit_blocks + st.loading_blocks + st.missing_blocks > hs.n()) bad.fetch_add(1);
        if (rng() % 16 == 0) pf_engine_disk_wait_prefetch(e);
      }
    });
  threads.emplace_back(until_stop([&, rng = std::mt19937(99)]() mutable {  // prefix counts
    Hashes hs;
    for (int i = 0; i < 32; ++i) hs.add(hash_of((int)(rng() % kBlocks)));
    uint64_t hits = 0;
    if (pf_engine_count_prefix_hit_blocks(e, "a", hs.data.data(), hs.offs.data(), hs.n(), &hits) ==
            PF_OK &&
        hits > hs.n())
      bad.fetch_add(1);
  }));
  threads.emplace_back(until_stop([&, rng = std::mt19937(7)]() mutable {  // slot reads
    std::vector<uint8_t> buf(kSlotBytes);
    const int b = rng() % kBlocks, s = rng() % kSlots;
    const std::string h = hash_of(b);
    uint64_t k = 0, v = 0;
    if (pf_engine_read_block_slot(e, "stress", reinterpret_cast<const uint8_t*>(h.data()),
                                  h.size(), s, buf.data(), buf.size(), &k, &v) == PF_OK) {
      slot_reads.fetch_add(1);
      if (k != kSeg || v != kSeg) bad.fetch_add(1);
      for (uint64_t i = 0; i < kSlotBytes; ++i)
        if (buf[i] != byte_of(b, s, i)) {
          bad.fetch_add(1);
          break;
        }
    }
  }));
  threads.emplace_back(until_stop([&] {  // statistics
    pf_engine_stats es{};
    pf_disk_stats ds{};
    pf_engine_stats_get(e, &es);
    pf_engine_disk_stats(e, &ds);
    if (es.pool_used_bytes > es.pool_total_bytes) bad.fetch_add(1);
  }));
  threads.emplace_back(until_stop([&, on = false]() mutable {  // storage policy churn
    // TinyLFU admission and a 1 ms pre-eviction monitor (keeping 30 of the
    // 40 blocks' room free once fewer than 20 are), on and off in turn.
    on = !on;
    if (pf_engine_set_storage_policy(e, on, 4096, on, 20 * kBlockBytes, 30 * kBlockBytes, 1))
      bad.fetch_add(1);
    std::this_thread::sleep_for(std::chrono::milliseconds(3));
  }));
  threads.emplace_back(until_stop([&] {  // instance churn
    if (reg(e, "c") == PF_OK) {
      Hashes hs;
      hs.add(hash_of(3));
      pf_prefetch_status st{};
      pf_engine_query_prefetch(e, "c", hs.data.data(), hs.offs.data(), hs.n(), &st);
      pf_engine_unregister_instance(e, "c");
    }
  }));
  std::this_thread::sleep_for(std::chrono::duration<double>(seconds));
  stop.store(true);
  for (auto& t : threads) t.join();
  pf_engine_set_storage_policy(e, 0, 0, 0, 0, 0, 0);
  pf_engine_disk_wait_prefetch(e);
  pf_disk_stats ds{};
  pf_engine_disk_stats(e, &ds);
  pf_engine_stats es{};
  pf_engine_stats_get(e, &es);
  std::printf("queries %llu slot_reads %llu prefetched %llu failures %llu evicted %llu bad %llu\n",
              (unsigned long long)queries.load(), (unsigned long long)slot_reads.load(),
              (unsigned long long)ds.prefetched_blocks, (unsigned long long)ds.failures,
              (unsigned long long)es.evicted_blocks, (unsigned long long)bad.load());
  const bool ok = bad.load() == 0 && ds.pending_blocks == 0 && queries.load() > 0 &&
                  ds.prefetched_blocks > 0 && slot_reads.load() > 0;
  pf_engine_destroy(e);
  return ok ? 0 : 1;
}
