// bench_copy_engines.cpp — host-link bandwidth of each copy engine (SDMA) of
// a device, per direction: one copy of 1 GiB between pinned host memory and
// device memory on each engine (hsa_amd_memory_async_copy_on_engine), best
// of 3.  The engines differ several-fold on MI355X; the staged mode's copies
// use the engines pf_copy_engines reports (the runtime's preferred ones).
//
// Prints one JSON object: the preferred engine masks, the library's engines,
// and per direction the GB/s of each engine (null where unavailable).
//
// Usage: bench_copy_engines [device]
#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../include/pegaflow_hip.h"

namespace {

[[noreturn]] void die(const char* what, const std::string& detail) {
  std::fprintf(stderr, "bench_copy_engines: %s failed: %s\n", what, detail.c_str());
  std::exit(1);
}

struct Agents {
  uint32_t bdf = 0, domain = 0;
  hsa_agent_t gpu{}, cpu{};
  bool gpu_found = false, cpu_found = false;
};

hsa_status_t visit(hsa_agent_t a, void* arg) {
  Agents* s = static_cast<Agents*>(arg);
  hsa_device_type_t t;
  if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if (t == HSA_DEVICE_TYPE_CPU && !s->cpu_found) {
    s->cpu = a;
    s->cpu_found = true;
  }
  uint32_t bdf = 0, domain = 0;
  if (t == HSA_DEVICE_TYPE_GPU && !s->gpu_found &&
      hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID), &bdf) ==
          HSA_STATUS_SUCCESS &&
      hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_DOMAIN), &domain) ==
          HSA_STATUS_SUCCESS &&
      bdf == s->bdf && domain == s->domain) {
    s->gpu = a;
    s->gpu_found = true;
  }
  return HSA_STATUS_SUCCESS;
}

// One copy on `engine`, waited for (at most 10 s); seconds, or < 0 on failure.
double timed_copy(const Agents& ag, bool d2h, void* host, void* dev, size_t bytes,
                  uint32_t engine, hsa_signal_t sig) {
  hsa_signal_store_screlease(sig, 1);
  const auto t0 = std::chrono::steady_clock::now();
  const hsa_status_t r =
      d2h ? hsa_amd_memory_async_copy_on_engine(host, ag.cpu, dev, ag.gpu, bytes, 0, nullptr, sig,
                                                static_cast<hsa_amd_sdma_engine_id_t>(engine),
                                                false)
          : hsa_amd_memory_async_copy_on_engine(dev, ag.gpu, host, ag.cpu, bytes, 0, nullptr, sig,
                                                static_cast<hsa_amd_sdma_engine_id_t>(engine),
                                                false);
  if (r != HSA_STATUS_SUCCESS) return -1;
  while (hsa_signal_wait_scacquire(sig, HSA_SIGNAL_CONDITION_EQ, 0, 10000000,
                                   HSA_WAIT_STATE_BLOCKED) != 0) {
    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(10))
      die("copy", "no completion within 10 s");
  }
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace

int main(int argc, char** argv) {
  const int device = argc > 1 ? std::atoi(argv[1]) : 0;
  if (pf_init(device) != PF_OK) die("pf_init", pf_last_error());
  char bus[64] = {0};
  if (hipDeviceGetPCIBusId(bus, sizeof(bus), device) != hipSuccess) die("pci id", "hip");
  Agents ag;
  unsigned dom = 0, b = 0, dv = 0, fn = 0;
  if (std::sscanf(bus, "%x:%x:%x.%x", &dom, &b, &dv, &fn) != 4) die("pci id", bus);
  ag.bdf = (b << 8) | (dv << 3) | fn;
  ag.domain = dom;
  if (hsa_init() != HSA_STATUS_SUCCESS) die("hsa_init", "");
  hsa_iterate_agents(visit, &ag);
  if (!ag.gpu_found || !ag.cpu_found) die("agents", "device not found");
  uint32_t avail[2] = {0, 0}, pref[2] = {0, 0}, lib[2] = {0, 0};
  hsa_amd_memory_copy_engine_status(ag.cpu, ag.gpu, &avail[0]);
  hsa_amd_memory_copy_engine_status(ag.gpu, ag.cpu, &avail[1]);
  hsa_amd_memory_get_preferred_copy_engine(ag.cpu, ag.gpu, &pref[0]);
  hsa_amd_memory_get_preferred_copy_engine(ag.gpu, ag.cpu, &pref[1]);
  if (pf_copy_engines(device, &lib[0], &lib[1]) != PF_OK) die("pf_copy_engines", pf_last_error());
  const size_t bytes = 1ull << 30;
  void *host = nullptr, *dev = nullptr;
  if (hipHostMalloc(&host, bytes, hipHostMallocMapped | hipHostMallocPortable) != hipSuccess ||
      hipMalloc(&dev, bytes) != hipSuccess || hipMemset(dev, 7, bytes) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess)
    die("buffers", "hip");
  hsa_signal_t sig;
  if (hsa_signal_create(1, 0, nullptr, &sig) != HSA_STATUS_SUCCESS) die("signal", "");
  std::printf("{\"device\": \"%s\", \"bytes\": %zu, \"preferred\": {\"d2h\": %u, \"h2d\": %u}, "
              "\"library\": {\"d2h\": %u, \"h2d\": %u}",
              bus, bytes, pref[0], pref[1], lib[0], lib[1]);
  const char* names[2] = {"d2h_gbps", "h2d_gbps"};
  for (int dir = 0; dir < 2; ++dir) {
    std::printf(", \"%s\": [", names[dir]);
    for (int e = 0; e < 16; ++e) {
      const uint32_t id = 1u << e;
      double best = -1;
      if (avail[dir] & id)
        for (int rep = 0; rep < 3; ++rep) {
          const double t = timed_copy(ag, dir == 0, host, dev, bytes, id, sig);
          if (t > 0 && (best < 0 || t < best)) best = t;
        }
      if (best > 0)
        std::printf("%s%.2f", e ? ", " : "", bytes / best / 1e9);
      else
        std::printf("%snull", e ? ", " : "");
    }
    std::printf("]");
  }
  std::printf("}\n");
  hsa_signal_destroy(sig);
  (void)hipHostFree(host);
  (void)hipFree(dev);
  return 0;
}
