// bench_pinned_copy.cpp — single-block host->device copy latency, the
// measurement of the reference's criterion benchmark
// (pegaflow-core/benches/pinned_copy.rs): one KV block of 2 segments x
// 24 KiB from pinned host memory into a device layer, with
//   contiguous layout (kv_stride = 24 KiB):  one copy of the block | one copy
//                                            per segment
//   strided layout (kv_stride = 27 x 24 KiB): one copy per segment | one 2D
//                                            copy
// (pinned_copy.rs:6-8, 70-118, 134-168), each timed as a synchronous call.
// Added beside them: the same block through this library's transfer
// context in the kernel mode (pf_load_layers + pf_xfer_synchronize) and in
// the batched-DMA mode, so the per-call cost of every route is on one line.
//
// Prints one JSON object: per variant the median and p10/p90 microseconds
// per block and the median GB/s (block bytes / median time).
//
// Usage: bench_pinned_copy [iterations] [device]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

#include "../../include/pegaflow_hip.h"

namespace {

constexpr uint64_t kBytesPerBlock = 24 * 1024;  // pinned_copy.rs:6
constexpr uint64_t kSegments = 2;               // pinned_copy.rs:7
constexpr uint64_t kBlocksInLayer = 27;         // pinned_copy.rs:8

[[noreturn]] void die(const char* what, const char* detail) {
  std::fprintf(stderr, "bench_pinned_copy: %s failed: %s\n", what, detail);
  std::exit(1);
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) die(what, hipGetErrorString(e));
}

void pf_check(int rc, const char* what) {
  if (rc != PF_OK) die(what, pf_last_error());
}

// TransferFixture (pinned_copy.rs:10-68): a pinned host block filled with
// its byte index, and a device buffer holding the block's segments
// kv_stride bytes apart.
struct Fixture {
  uint64_t kv_stride;
  void* host = nullptr;
  uint64_t host_dev = 0;
  void* dev = nullptr;
  uint64_t dev_bytes = 0;
  pf_kv_layout layout{};

  explicit Fixture(uint64_t stride) : kv_stride(stride) {
    const uint64_t block = kBytesPerBlock * kSegments;
    pf_check(pf_pinned_allocate(block, PF_PINNED_DEFAULT, &host, &host_dev), "pf_pinned_allocate");
    auto* b = static_cast<uint8_t*>(host);
    for (uint64_t i = 0; i < block; ++i) b[i] = static_cast<uint8_t>(i & 0xFF);
    dev_bytes = kv_stride * (kSegments - 1) + kBytesPerBlock;
    hip_check(hipMalloc(&dev, dev_bytes), "hipMalloc");
    pf_check(pf_layout_init(reinterpret_cast<uint64_t>(dev), dev_bytes, 1, kBytesPerBlock,
                            kv_stride, kSegments, &layout),
             "pf_layout_init");
  }
  ~Fixture() {
    (void)hipFree(dev);
    (void)pf_pinned_free(host);
  }
  uint8_t* seg_host(uint64_t s) const { return static_cast<uint8_t*>(host) + s * kBytesPerBlock; }
  uint8_t* seg_dev(uint64_t s) const { return static_cast<uint8_t*>(dev) + s * kv_stride; }

  // copy_single (pinned_copy.rs:70-82).
  void copy_single() const {
    hip_check(hipMemcpy(dev, host, kBytesPerBlock * kSegments, hipMemcpyHostToDevice),
              "hipMemcpy(single)");
  }
  // copy_segments (pinned_copy.rs:84-94).
  void copy_segments() const {
    for (uint64_t s = 0; s < kSegments; ++s)
      hip_check(hipMemcpy(seg_dev(s), seg_host(s), kBytesPerBlock, hipMemcpyHostToDevice),
                "hipMemcpy(segment)");
  }
  // copy_with_memcpy2d (pinned_copy.rs:96-118).
  void copy_2d() const {
    hip_check(hipMemcpy2D(dev, kv_stride, host, kBytesPerBlock, kBytesPerBlock, kSegments,
                          hipMemcpyHostToDevice),
              "hipMemcpy2D");
  }
  // The block through a transfer context: block 0, K half then V half.
  void copy_xfer(pf_xfer* x, uint32_t mode) const {
    pf_block_xfer b{0, reinterpret_cast<uint64_t>(seg_host(0)),
                    reinterpret_cast<uint64_t>(seg_host(1))};
    pf_layer_xfer l{layout, &b, 1};
    pf_check(pf_load_layers(x, &l, 1, mode, nullptr), "pf_load_layers");
    pf_check(pf_xfer_synchronize(x), "pf_xfer_synchronize");
  }
  // Every byte of the block arrived in place.
  bool check() const {
    std::vector<uint8_t> got(kBytesPerBlock);
    for (uint64_t s = 0; s < kSegments; ++s) {
      hip_check(hipMemcpy(got.data(), seg_dev(s), kBytesPerBlock, hipMemcpyDeviceToHost),
                "hipMemcpy(check)");
      for (uint64_t i = 0; i < kBytesPerBlock; ++i)
        if (got[i] != seg_host(s)[i]) return false;
    }
    return true;
  }
};

struct Result {
  std::string name;
  double p10, p50, p90, gbps;
  bool exact;
};

Result measure(const std::string& name, int iters, const Fixture& f,
               const std::function<void()>& fn) {
  (void)hipMemset(f.dev, 0, f.dev_bytes);
  for (int i = 0; i < std::max(10, iters / 20); ++i) fn();  // warm-up
  std::vector<double> us(iters);
  for (int i = 0; i < iters; ++i) {
    const auto t0 = std::chrono::steady_clock::now();
    fn();
    us[i] = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0)
                .count();
  }
  std::sort(us.begin(), us.end());
  const double p50 = us[iters / 2];
  return {name, us[iters / 10], p50, us[iters * 9 / 10],
          (kBytesPerBlock * kSegments) / (p50 * 1e3), f.check()};
}

}  // namespace

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::max(100, std::atoi(argv[1])) : 2000;
  const int device = argc > 2 ? std::atoi(argv[2]) : 0;
  pf_check(pf_init(device), "pf_init");
  pf_xfer* x = nullptr;
  pf_check(pf_xfer_create(device, 0, &x), "pf_xfer_create");
  std::vector<Result> out;
  {
    Fixture f(kBytesPerBlock);  // pinned_contiguous group (pinned_copy.rs:134-151)
    out.push_back(measure("contiguous/single_memcpy", iters, f, [&] { f.copy_single(); }));
    out.push_back(measure("contiguous/loop_segments", iters, f, [&] { f.copy_segments(); }));
    out.push_back(measure("contiguous/kernel", iters, f, [&] { f.copy_xfer(x, PF_MODE_KERNEL); }));
  }
  {
    Fixture f(kBytesPerBlock * kBlocksInLayer);  // pinned_strided group (153-168)
    out.push_back(measure("strided/loop_segments", iters, f, [&] { f.copy_segments(); }));
    out.push_back(measure("strided/memcpy2d", iters, f, [&] { f.copy_2d(); }));
    out.push_back(measure("strided/kernel", iters, f, [&] { f.copy_xfer(x, PF_MODE_KERNEL); }));
    out.push_back(measure("strided/dma_batched", iters, f,
                          [&] { f.copy_xfer(x, PF_MODE_DMA_BATCHED); }));
  }
  pf_check(pf_xfer_destroy(x), "pf_xfer_destroy");
  std::printf("{\"block_bytes\": %llu, \"segment_bytes\": %llu, \"iterations\": %d, \"variants\": {",
              (unsigned long long)(kBytesPerBlock * kSegments),
              (unsigned long long)kBytesPerBlock, iters);
  for (size_t i = 0; i < out.size(); ++i) {
    const Result& r = out[i];
    std::printf("%s\"%s\": {\"us_p10\": %.2f, \"us_median\": %.2f, \"us_p90\": %.2f, "
                "\"gbps\": %.3f, \"bit_exact\": %s}",
                i ? ", " : "", r.name.c_str(), r.p10, r.p50, r.p90, r.gbps,
                r.exact ? "true" : "false");
  }
  std::printf("}}\n");
  for (const Result& r : out)
    if (!r.exact) return 2;
  return 0;
}
