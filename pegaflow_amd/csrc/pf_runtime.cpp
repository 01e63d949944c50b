// pf_runtime.cpp — devices, streams, events, device memory and the pinned
// host pool backing (the roles of cudarc's CudaContext/CudaStream and of
// pegaflow-core/src/pinned_mem.rs in the reference).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>

#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include "pf_common.h"

namespace pf {

// ---------------------------------------------------------------------------
// Pinned allocation registry.
// ---------------------------------------------------------------------------
static std::mutex g_pinned_mu;
static std::map<uint64_t, uint64_t> g_pinned;  // base -> size

void pinned_register(uint64_t base, uint64_t size) {
  std::lock_guard<std::mutex> lk(g_pinned_mu);
  g_pinned[base] = size;
}

void pinned_unregister(uint64_t base) {
  std::lock_guard<std::mutex> lk(g_pinned_mu);
  g_pinned.erase(base);
}

bool pinned_lookup(uint64_t addr, uint64_t len, uint64_t* base, uint64_t* end) {
  std::lock_guard<std::mutex> lk(g_pinned_mu);
  auto it = g_pinned.upper_bound(addr);
  if (it == g_pinned.begin()) return false;
  --it;
  uint64_t b = it->first, e = it->first + it->second;
  if (addr < b || addr + len > e || addr + len < addr) return false;
  if (base) *base = b;
  if (end) *end = e;
  return true;
}

// Allocations mapped from another process with pf_ipc_open.
static std::mutex g_ipc_mu;
static std::map<uint64_t, uint64_t> g_ipc;  // base -> size

static bool ipc_lookup(uint64_t addr, uint64_t len, uint64_t* base, uint64_t* end) {
  std::lock_guard<std::mutex> lk(g_ipc_mu);
  auto it = g_ipc.upper_bound(addr);
  if (it == g_ipc.begin()) return false;
  --it;
  const uint64_t b = it->first, e = it->first + it->second;
  if (addr < b || addr + len > e || addr + len < addr) return false;
  *base = b;
  *end = e;
  return true;
}

bool RangeCache::contains(uint64_t a, uint64_t len) {
  const uint64_t e = a + len;
  if (e < a) return false;
  if (a >= last_b_ && e <= last_e_ && last_e_ > last_b_) return true;
  for (auto& r : ok_)
    if (a >= r.first && e <= r.second) {
      last_b_ = r.first;
      last_e_ = r.second;
      return true;
    }
  return false;
}

bool RangeCache::check(uint64_t a, uint64_t len) {
  if (a == 0 || a + len < a) return false;
  if (contains(a, len)) return true;
  uint64_t b = 0, e = 0;
  if (pinned_lookup(a, len, &b, &e) || ipc_lookup(a, len, &b, &e)) {
    ok_.push_back({b, e});
    last_b_ = b;
    last_e_ = e;
    return true;
  }
  hipPointerAttribute_t attr;
  hipError_t err = hipPointerGetAttributes(&attr, reinterpret_cast<void*>(a));
  if (err != hipSuccess) {
    (void)hipGetLastError();  // clear the sticky error of the probe
    return false;
  }
  if (attr.type != hipMemoryTypeDevice) return false;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  err = hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(a));
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  b = reinterpret_cast<uint64_t>(base);
  e = b + size;
  if (a < b || a + len > e) return false;
  ok_.push_back({b, e});
  last_b_ = b;
  last_e_ = e;
  return true;
}

static int check_range(uint64_t addr, uint64_t len, const char* what) {
  RangeCache rc;
  if (!rc.check(addr, len))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("%s: range [0x%llx, +%llu) is not inside one device or pinned "
                     "allocation",
                     what, (unsigned long long)addr, (unsigned long long)len));
  return PF_OK;
}

// Wall-clock rate per device (kHz), cached by pf_init.
static std::mutex g_dev_mu;
static std::map<int, int> g_wall_khz;

static int wall_clock_khz() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    auto it = g_wall_khz.find(dev);
    if (it != g_wall_khz.end()) return it->second;
  }
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    khz = 0;
  std::lock_guard<std::mutex> lk(g_dev_mu);
  g_wall_khz[dev] = khz;
  return khz;
}

// ---------------------------------------------------------------------------
// Static device scratch of pf_load_layers_noalloc.  Host code never uses the
// array's name as an address (in host code it names a host-side stand-in):
// hipGetSymbolAddress gives each device's own copy, and that address is what
// the entry point hands to copies and kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static std::map<int, std::unique_ptr<NoAllocScratch>> g_scratch;

int noalloc_scratch(int device, NoAllocScratch** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(device);
  if (it != g_scratch.end()) {
    *out = it->second.get();
    return PF_OK;
  }
  int prev = 0;
  PF_HIP(hipGetDevice(&prev));
  if (prev != device) PF_HIP(hipSetDevice(device));
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (prev != device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  if (!ptr) return fail(PF_ERR_INIT, "no device address for the scratch array");
  auto sc = std::make_unique<NoAllocScratch>();
  sc->base = reinterpret_cast<uint64_t>(ptr);
  // The array is zero when the code object is loaded, so the tile queue
  // starts empty, and every queued launch leaves it empty.
  *out = sc.get();
  g_scratch.emplace(device, std::move(sc));
  return PF_OK;
}

// ---------------------------------------------------------------------------
// Copy engines.
// ---------------------------------------------------------------------------
struct EngineDevice {
  bool ok = false;
  hsa_agent_t gpu{}, cpu{};
  // [0]: device to host, [1]: host to device; one or two engine id bits
  // each, alternated by the copies' lane.
  uint32_t engine[2][2] = {{0, 0}, {0, 0}};
};

static std::mutex g_engine_mu;
static std::map<int, EngineDevice> g_engines;

namespace {

struct AgentSearch {
  uint32_t bdf = 0, domain = 0;
  bool gpu_found = false, cpu_found = false;
  hsa_agent_t gpu{}, cpu{};
};

hsa_status_t visit_agent(hsa_agent_t a, void* arg) {
  AgentSearch* s = static_cast<AgentSearch*>(arg);
  hsa_device_type_t t;
  if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if (t == HSA_DEVICE_TYPE_CPU && !s->cpu_found) {
    s->cpu = a;
    s->cpu_found = true;
  }
  if (t == HSA_DEVICE_TYPE_GPU && !s->gpu_found) {
    uint32_t bdf = 0, domain = 0;
    if (hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID), &bdf) ==
            HSA_STATUS_SUCCESS &&
        hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_DOMAIN),
                           &domain) == HSA_STATUS_SUCCESS &&
        bdf == s->bdf && domain == s->domain) {
      s->gpu = a;
      s->gpu_found = true;
    }
  }
  return HSA_STATUS_SUCCESS;
}

uint32_t lowest_bit(uint32_t m) { return m & (~m + 1u); }

// The device's agents (matched by PCI address) and engine choice.
EngineDevice discover_engines(int device) {
  EngineDevice d;
  char bus[64] = {0};
  unsigned dom = 0, b = 0, dv = 0, fn = 0;
  if (hipDeviceGetPCIBusId(bus, sizeof(bus), device) != hipSuccess ||
      std::sscanf(bus, "%x:%x:%x.%x", &dom, &b, &dv, &fn) != 4) {
    (void)hipGetLastError();
    return d;
  }
  // HIP has initialized the HSA runtime already; this holds a reference of
  // the library's own (never released: engine copies may run until exit).
  if (hsa_init() != HSA_STATUS_SUCCESS) return d;
  AgentSearch s;
  s.bdf = (b << 8) | (dv << 3) | fn;
  s.domain = dom;
  if (hsa_iterate_agents(visit_agent, &s) != HSA_STATUS_SUCCESS || !s.gpu_found) return d;
  hsa_agent_t near{};
  if (hsa_agent_get_info(s.gpu, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_NEAREST_CPU),
                         &near) == HSA_STATUS_SUCCESS &&
      near.handle != 0) {
    s.cpu = near;
    s.cpu_found = true;
  }
  if (!s.cpu_found) return d;
  uint32_t d2h = 0, h2d = 0;
  if (hsa_amd_memory_get_preferred_copy_engine(s.cpu, s.gpu, &d2h) != HSA_STATUS_SUCCESS ||
      hsa_amd_memory_get_preferred_copy_engine(s.gpu, s.cpu, &h2d) != HSA_STATUS_SUCCESS ||
      d2h == 0 || h2d == 0)
    return d;
  uint32_t avail_d2h = 0, avail_h2d = 0;
  (void)hsa_amd_memory_copy_engine_status(s.cpu, s.gpu, &avail_d2h);
  (void)hsa_amd_memory_copy_engine_status(s.gpu, s.cpu, &avail_h2d);
  // The model's own copies (hipMemcpyAsync, in this process or in the
  // serving process beside it) run on the lowest engine of each preferred
  // set: measured on MI355X, a staged save on engine 1 slowed a 64 KiB
  // device-to-host hipMemcpyAsync every 0.5 ms 8.3x and fell to 26 GB/s
  // itself, and any staged copy on engine 0 slowed a 64 KiB host-to-device
  // one 6x; on engines 2 and 3 both stayed within 1.25x and the staged
  // copies at 56 GB/s.  So the staged copies take the fast engines the
  // runtime's copies do not use: engines 0-3 move 57 GB/s each way, the
  // others 7-51 GB/s.  One engine per direction, different for the two
  // directions, so a save and a load run at once.  A second engine per
  // direction was measured and dropped: two device-to-host engines saved
  // the Llama prefix at 45 GB/s against 56 on one, and with four engines
  // busy a save and a restore at once fell from 95 to 66 GB/s.
  constexpr uint32_t kFastEngines = 0xF;
  const uint32_t runtime_own = lowest_bit(d2h) | lowest_bit(h2d);
  const uint32_t spare = kFastEngines & ~runtime_own & avail_d2h & avail_h2d;
  uint32_t d0 = 0, h0 = 0;
  if (spare) {
    d0 = 1u << (31 - __builtin_clz(spare));  // the highest spare engine
    const uint32_t rest = spare & ~d0;
    h0 = rest ? lowest_bit(rest) : d0;
  } else {
    // No spare fast engine: the preferred ones, different where they allow.
    h0 = lowest_bit(h2d);
    const uint32_t d2h_rest = d2h & ~h0;
    d0 = lowest_bit(d2h_rest ? d2h_rest : d2h);
  }
  d.engine[0][0] = d.engine[0][1] = d0;
  d.engine[1][0] = d.engine[1][1] = h0;
  // PEGAFLOW_COPY_ENGINES="<d2h>,<h2d>" (engine id bit masks, one or two
  // bits each, e.g. "0x8,0x4") overrides the choice; masks the runtime does
  // not report available are ignored.
  if (const char* env = std::getenv("PEGAFLOW_COPY_ENGINES")) {
    unsigned long m[2] = {0, 0};
    char* end = nullptr;
    m[0] = std::strtoul(env, &end, 0);
    if (end && *end == ',') m[1] = std::strtoul(end + 1, &end, 0);
    const uint32_t avail[2] = {avail_d2h, avail_h2d};
    for (int dir = 0; dir < 2; ++dir) {
      const uint32_t mask = static_cast<uint32_t>(m[dir]);
      if (mask == 0 || (mask & ~avail[dir]) || __builtin_popcount(mask) > 2) continue;
      d.engine[dir][0] = lowest_bit(mask);
      d.engine[dir][1] = lowest_bit(mask & ~d.engine[dir][0]) ? lowest_bit(mask & ~d.engine[dir][0])
                                                              : d.engine[dir][0];
    }
  }
  d.gpu = s.gpu;
  d.cpu = s.cpu;
  d.ok = true;
  return d;
}

// The device's engines (discovered on first use), copied under the lock:
// pf_set_copy_engines may change the choice while copies are issued.
bool engines_of(int device, EngineDevice* out) {
  std::lock_guard<std::mutex> lk(g_engine_mu);
  auto it = g_engines.find(device);
  if (it == g_engines.end()) it = g_engines.emplace(device, discover_engines(device)).first;
  if (!it->second.ok) return false;
  *out = it->second;
  return true;
}

hsa_signal_t sig_of(const EngineSignal* s) { return hsa_signal_t{s->handle}; }

}  // namespace

bool engine_copies_available(int device) {
  EngineDevice d;
  return engines_of(device, &d);
}

bool engine_ids(int device, uint32_t* d2h, uint32_t* h2d) {
  EngineDevice d;
  const bool ok = engines_of(device, &d);
  *d2h = ok ? (d.engine[0][0] | d.engine[0][1]) : 0;
  *h2d = ok ? (d.engine[1][0] | d.engine[1][1]) : 0;
  return ok;
}

int set_engine_ids(int device, uint32_t d2h, uint32_t h2d) {
  EngineDevice d;
  if (!engines_of(device, &d))
    return fail(PF_ERR_UNSUPPORTED, "the device's copy engines are not known");
  uint32_t avail[2] = {0, 0};
  (void)hsa_amd_memory_copy_engine_status(d.cpu, d.gpu, &avail[0]);
  (void)hsa_amd_memory_copy_engine_status(d.gpu, d.cpu, &avail[1]);
  const uint32_t mask[2] = {d2h, h2d};
  for (int dir = 0; dir < 2; ++dir) {
    const uint32_t m = mask[dir];
    if (m == 0) continue;
    if (__builtin_popcount(m) > 2)
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("copy engine mask 0x%x: one or two engine bits per direction", m));
    if (m & ~avail[dir])
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("copy engine mask 0x%x: the runtime reports only 0x%x available %s", m,
                       avail[dir], dir == 0 ? "device to host" : "host to device"));
  }
  std::lock_guard<std::mutex> lk(g_engine_mu);
  EngineDevice& e = g_engines[device];
  for (int dir = 0; dir < 2; ++dir) {
    const uint32_t m = mask[dir];
    if (m == 0) continue;
    const uint32_t a = lowest_bit(m), b = lowest_bit(m & ~a);
    e.engine[dir][0] = a;
    e.engine[dir][1] = b ? b : a;
  }
  return PF_OK;
}

int engine_signal_create(EngineSignal* s) {
  hsa_signal_t h{};
  if (hsa_signal_create(0, 0, nullptr, &h) != HSA_STATUS_SUCCESS)
    return fail(PF_ERR_HIP, "hsa_signal_create failed");
  s->handle = h.handle;
  return PF_OK;
}

void engine_signal_destroy(EngineSignal* s) {
  if (s->handle) (void)hsa_signal_destroy(sig_of(s));
  s->handle = 0;
}

void engine_signal_add(EngineSignal* s, int64_t n) { hsa_signal_add_screlease(sig_of(s), n); }

int engine_copy(int device, bool d2h, uint64_t dst, uint64_t src, uint64_t bytes,
                EngineSignal* s, unsigned lane) {
  EngineDevice d;
  hsa_status_t r = HSA_STATUS_ERROR;
  if (engines_of(device, &d)) {
    const hsa_agent_t dst_agent = d2h ? d.cpu : d.gpu;
    const hsa_agent_t src_agent = d2h ? d.gpu : d.cpu;
    r = hsa_amd_memory_async_copy_on_engine(
        reinterpret_cast<void*>(dst), dst_agent, reinterpret_cast<const void*>(src), src_agent,
        bytes, 0, nullptr, sig_of(s),
        static_cast<hsa_amd_sdma_engine_id_t>(d.engine[d2h ? 0 : 1][lane & 1]), false);
  }
  if (r != HSA_STATUS_SUCCESS) {
    hsa_signal_subtract_screlease(sig_of(s), 1);
    return fail(PF_ERR_HIP, strf("copy engine refused a %s copy of %llu bytes (%d)",
                                 d2h ? "device-to-host" : "host-to-device",
                                 (unsigned long long)bytes, static_cast<int>(r)));
  }
  return PF_OK;
}

int engine_signal_wait(EngineSignal* s, bool spin) {
  const hsa_signal_t h = sig_of(s);
  if (spin) {
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t i = 1; hsa_signal_load_scacquire(h) != 0; ++i) {
      if ((i & 1023) == 0 &&
          std::chrono::steady_clock::now() - t0 > std::chrono::seconds(kEngineWaitSeconds))
        return fail(PF_ERR_HIP,
                    strf("copy engine copies not done after %d s", kEngineWaitSeconds));
    }
    return PF_OK;
  }
  // Each wait is bounded to about 0.1 s (in system timestamp ticks) so the
  // deadline below is checked.
  static const uint64_t hint = [] {
    uint64_t hz = 0;
    if (hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &hz) != HSA_STATUS_SUCCESS ||
        hz == 0)
      hz = 1000000000ull;
    return hz / 10;
  }();
  const auto t0 = std::chrono::steady_clock::now();
  while (hsa_signal_wait_scacquire(h, HSA_SIGNAL_CONDITION_EQ, 0, hint,
                                   HSA_WAIT_STATE_BLOCKED) != 0) {
    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(kEngineWaitSeconds))
      return fail(PF_ERR_HIP, strf("copy engine copies not done after %d s", kEngineWaitSeconds));
  }
  return PF_OK;
}

int ipc_events_supported(std::string* why) {
  static std::once_flag once;
  static int supported = -1;
  static std::string reason;
  std::call_once(once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
      (void)hipGetLastError();
      return;
    }
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventInterprocess);
    if (r == hipSuccess) {
      hipIpcEventHandle_t h;
      std::memset(&h, 0, sizeof(h));
      r = hipIpcGetEventHandle(&h, e);
      (void)hipEventDestroy(e);
    }
    (void)hipGetLastError();
    supported = r == hipSuccess ? 1 : 0;
    if (r != hipSuccess) reason = strf("hipIpcGetEventHandle: %s", hipGetErrorString(r));
  });
  if (why) *why = reason;
  return supported;
}

// An interprocess event this runtime cannot export would leave its consumer
// waiting on a handle that never arrives; the event is refused instead.
int refuse_ipc_events() {
  std::string why;
  if (ipc_events_supported(&why) != 0) return PF_OK;
  return fail(PF_ERR_UNSUPPORTED,
              "interprocess events are not supported by this runtime (" + why +
                  "); wait on layer words instead (pf_load_state_create_layered_words)");
}

}  // namespace pf

using namespace pf;

extern "C" {

int pf_get_device_count(int* count) {
  PF_HIP(hipGetDeviceCount(count));
  return PF_OK;
}

int pf_init(int device) {
  if (device < 0) return fail(PF_ERR_INVALID_ARGUMENT, "device_id must be >= 0");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device >= n)
    return fail(PF_ERR_INIT, strf("device %d not present (%d devices)", device, n));
  PF_HIP(hipSetDevice(device));
  if (wall_clock_khz() <= 0)
    return fail(PF_ERR_INIT, "hipDeviceAttributeWallClockRate unavailable");
  NoAllocScratch* sc = nullptr;
  return noalloc_scratch(device, &sc);
}

int pf_device_pci_bus_id(int device, char* buf, int len) {
  if (!buf || len < 13) return fail(PF_ERR_INVALID_ARGUMENT, "buffer too small for a PCI id");
  PF_HIP(hipDeviceGetPCIBusId(buf, len, device));
  for (int i = 0; i < len && buf[i]; ++i)
    if (buf[i] >= 'A' && buf[i] <= 'F') buf[i] = static_cast<char>(buf[i] - 'A' + 'a');
  return PF_OK;
}

int pf_set_device(int device) {
  PF_HIP(hipSetDevice(device));
  return PF_OK;
}

int pf_get_device(int* device) {
  PF_HIP(hipGetDevice(device));
  return PF_OK;
}

int pf_device_synchronize(void) {
  PF_HIP(hipDeviceSynchronize());
  return PF_OK;
}

int pf_stream_create(pf_stream* out) {
  hipStream_t s = nullptr;
  PF_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = s;
  return PF_OK;
}

int pf_stream_destroy(pf_stream stream) {
  PF_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return PF_OK;
}

int pf_stream_synchronize(pf_stream stream) {
  PF_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return PF_OK;
}

int pf_stream_wait_event(pf_stream stream, pf_event event) {
  PF_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream),
                            static_cast<hipEvent_t>(event), 0));
  return PF_OK;
}

int pf_event_create(pf_event* out) {
  hipEvent_t e = nullptr;
  PF_HIP(hipEventCreate(&e));
  *out = e;
  return PF_OK;
}

int pf_event_destroy(pf_event event) {
  PF_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return PF_OK;
}

int pf_event_record(pf_event event, pf_stream stream) {
  PF_HIP(hipEventRecord(static_cast<hipEvent_t>(event),
                        static_cast<hipStream_t>(stream)));
  return PF_OK;
}

int pf_event_synchronize(pf_event event) {
  PF_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return PF_OK;
}

int pf_event_query(pf_event event, int* done) {
  hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
  if (e == hipSuccess) {
    *done = 1;
    return PF_OK;
  }
  if (e == hipErrorNotReady) {
    *done = 0;
    return PF_OK;
  }
  return hip_fail(e, "hipEventQuery");
}

int pf_event_elapsed_ms(pf_event start, pf_event end, float* ms) {
  PF_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                             static_cast<hipEvent_t>(end)));
  return PF_OK;
}

int pf_device_malloc(uint64_t size, uint64_t* out_dev_ptr) {
  if (size == 0) return fail(PF_ERR_ZERO_SIZE, "size must be greater than zero");
  void* p = nullptr;
  PF_HIP(hipMalloc(&p, size));
  *out_dev_ptr = reinterpret_cast<uint64_t>(p);
  return PF_OK;
}

int pf_device_free(uint64_t dev_ptr) {
  PF_HIP(hipFree(reinterpret_cast<void*>(dev_ptr)));
  return PF_OK;
}

int pf_memcpy_h2d(uint64_t dst_dev, const void* src, uint64_t size) {
  PF_HIP(hipMemcpy(reinterpret_cast<void*>(dst_dev), src, size,
                   hipMemcpyHostToDevice));
  return PF_OK;
}

int pf_memcpy_d2h(void* dst, uint64_t src_dev, uint64_t size) {
  PF_HIP(hipMemcpy(dst, reinterpret_cast<const void*>(src_dev), size,
                   hipMemcpyDeviceToHost));
  return PF_OK;
}

int pf_memcpy_d2d(uint64_t dst_dev, uint64_t src_dev, uint64_t size) {
  PF_HIP(hipMemcpy(reinterpret_cast<void*>(dst_dev),
                   reinterpret_cast<const void*>(src_dev), size,
                   hipMemcpyDeviceToDevice));
  return PF_OK;
}

int pf_memset_d8(uint64_t dst_dev, uint8_t value, uint64_t size) {
  PF_HIP(hipMemset(reinterpret_cast<void*>(dst_dev), value, size));
  return PF_OK;
}

int pf_memcpy_async(uint64_t dst, uint64_t src, uint64_t size, pf_stream stream) {
  PF_HIP(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), size,
                        hipMemcpyDefault, static_cast<hipStream_t>(stream)));
  return PF_OK;
}

int pf_mem_get_info(uint64_t* free_bytes, uint64_t* total_bytes) {
  size_t f = 0, t = 0;
  PF_HIP(hipMemGetInfo(&f, &t));
  *free_bytes = f;
  *total_bytes = t;
  return PF_OK;
}

// PinnedMemory::allocate (pinned_mem.rs:128-164).  The reference asks CUDA for
// write-combined memory; HIP does not implement that flag, so the pool is
// ordinary pinned memory, always mapped so the transfer kernels can reach it.
int pf_pinned_allocate(uint64_t size, uint32_t flags, void** host_ptr,
                       uint64_t* dev_ptr) {
  if (size == 0) return fail(PF_ERR_ZERO_SIZE, "size must be greater than zero");
  if (!host_ptr) return fail(PF_ERR_INVALID_ARGUMENT, "null host_ptr");
  if ((flags & PF_PINNED_COHERENT) && (flags & PF_PINNED_NONCOHERENT))
    return fail(PF_ERR_INVALID_ARGUMENT, "coherent and non-coherent are exclusive");
  unsigned hip_flags = hipHostMallocMapped | hipHostMallocPortable;
  if (flags & PF_PINNED_COHERENT) hip_flags |= hipHostMallocCoherent;
  if (flags & PF_PINNED_NONCOHERENT) hip_flags |= hipHostMallocNonCoherent;
  if (flags & PF_PINNED_NUMA_USER) hip_flags |= hipHostMallocNumaUser;
  if (flags & PF_PINNED_WRITE_COMBINED) hip_flags |= hipHostMallocWriteCombined;
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, size, hip_flags);
  if (e != hipSuccess)
    return fail(PF_ERR_HIP, strf("hipHostMalloc failed: %s (%d)",
                                 hipGetErrorString(e), static_cast<int>(e)));
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return hip_fail(e, "hipHostGetDevicePointer");
  }
  if (d != p) {
    // The kernels address host memory through the host pointer itself; a
    // platform that maps it elsewhere is not supported.
    (void)hipHostFree(p);
    return fail(PF_ERR_UNSUPPORTED,
                "pinned memory is not mapped at its host address");
  }
  pinned_register(reinterpret_cast<uint64_t>(p), size);
  *host_ptr = p;
  if (dev_ptr) *dev_ptr = reinterpret_cast<uint64_t>(d);
  return PF_OK;
}

int pf_pinned_free(void* host_ptr) {
  if (!host_ptr) return PF_OK;
  pinned_unregister(reinterpret_cast<uint64_t>(host_ptr));
  PF_HIP(hipHostFree(host_ptr));
  return PF_OK;
}

int pf_host_device_pointer(const void* host_ptr, uint64_t* dev_ptr) {
  void* d = nullptr;
  PF_HIP(hipHostGetDevicePointer(&d, const_cast<void*>(host_ptr), 0));
  *dev_ptr = reinterpret_cast<uint64_t>(d);
  return PF_OK;
}

// ---------------------------------------------------------------------------
// Device-memory IPC.
// ---------------------------------------------------------------------------
int pf_ipc_export(uint64_t dev_ptr, uint8_t* handle, uint64_t* alloc_base,
                  uint64_t* alloc_size) {
  if (!handle) return fail(PF_ERR_INVALID_ARGUMENT, "null handle buffer");
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, reinterpret_cast<void*>(dev_ptr));
  if (e != hipSuccess || attr.type != hipMemoryTypeDevice) {
    (void)hipGetLastError();
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("0x%llx is not device memory", (unsigned long long)dev_ptr));
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  PF_HIP(hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(dev_ptr)));
  if (size >= PF_IPC_MAX_ALLOC_BYTES)
    return fail(PF_ERR_UNSUPPORTED,
                strf("allocation of %zu bytes is too large to share between processes "
                     "(limit %llu)",
                     size, (unsigned long long)PF_IPC_MAX_ALLOC_BYTES));
  hipIpcMemHandle_t h;
  PF_HIP(hipIpcGetMemHandle(&h, base));
  std::memcpy(handle, &h, PF_IPC_HANDLE_BYTES);
  if (alloc_base) *alloc_base = reinterpret_cast<uint64_t>(base);
  if (alloc_size) *alloc_size = size;
  return PF_OK;
}

int pf_ipc_open(const uint8_t* handle, uint64_t alloc_size, uint64_t* base) {
  if (!handle || !base) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  if (alloc_size == 0 || alloc_size >= PF_IPC_MAX_ALLOC_BYTES)
    return fail(PF_ERR_UNSUPPORTED,
                strf("shared allocation size %llu outside (0, %llu)",
                     (unsigned long long)alloc_size, (unsigned long long)PF_IPC_MAX_ALLOC_BYTES));
  hipIpcMemHandle_t h;
  std::memcpy(&h, handle, PF_IPC_HANDLE_BYTES);
  void* p = nullptr;
  PF_HIP(hipIpcOpenMemHandle(&p, h, hipIpcMemLazyEnablePeerAccess));
  // Trust the exporter's size only as far as the mapping goes.
  hipDeviceptr_t mb = nullptr;
  size_t ms = 0;
  if (hipMemGetAddressRange(&mb, &ms, p) == hipSuccess) {
    if (reinterpret_cast<uint64_t>(mb) != reinterpret_cast<uint64_t>(p) || ms < alloc_size) {
      (void)hipIpcCloseMemHandle(p);
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("shared allocation maps %zu bytes, %llu declared", ms,
                       (unsigned long long)alloc_size));
    }
  } else {
    (void)hipGetLastError();
  }
  {
    std::lock_guard<std::mutex> lk(g_ipc_mu);
    g_ipc[reinterpret_cast<uint64_t>(p)] = alloc_size;
  }
  *base = reinterpret_cast<uint64_t>(p);
  return PF_OK;
}

int pf_ipc_close(uint64_t base) {
  {
    std::lock_guard<std::mutex> lk(g_ipc_mu);
    g_ipc.erase(base);
  }
  PF_HIP(hipIpcCloseMemHandle(reinterpret_cast<void*>(base)));
  return PF_OK;
}

int pf_event_create_ipc(pf_event* out) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "null output");
  if (int rc = refuse_ipc_events()) return rc;
  hipEvent_t e = nullptr;
  PF_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventInterprocess));
  *out = e;
  return PF_OK;
}

int pf_ipc_event_export(pf_event event, uint8_t* handle) {
  if (!event || !handle) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  static_assert(sizeof(hipIpcEventHandle_t) >= PF_IPC_HANDLE_BYTES, "event handle size");
  hipIpcEventHandle_t h;
  std::memset(&h, 0, sizeof(h));
  PF_HIP(hipIpcGetEventHandle(&h, static_cast<hipEvent_t>(event)));
  std::memcpy(handle, &h, PF_IPC_HANDLE_BYTES);
  return PF_OK;
}

int pf_ipc_event_open(const uint8_t* handle, pf_event* out) {
  if (!handle || !out) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  hipIpcEventHandle_t h;
  std::memset(&h, 0, sizeof(h));
  std::memcpy(&h, handle, PF_IPC_HANDLE_BYTES);
  hipEvent_t e = nullptr;
  PF_HIP(hipIpcOpenEventHandle(&e, h));
  *out = e;
  return PF_OK;
}

// pinned_mem.rs:38-52: "Hugepagesize:       2048 kB" -> bytes.
uint64_t pf_huge_page_size(void) {
  std::ifstream f("/proc/meminfo");
  std::string line;
  while (std::getline(f, line)) {
    if (line.rfind("Hugepagesize:", 0) == 0) {
      std::istringstream ss(line);
      std::string key, unit;
      uint64_t kb = 0;
      if ((ss >> key >> kb >> unit) && unit == "kB") return kb * 1024;
      return 0;
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Synthetic data and verification.
// ---------------------------------------------------------------------------
int pf_fill_random(uint64_t dst_dev, uint64_t size_bytes, uint64_t seed,
                   uint64_t word_offset, pf_stream stream) {
  if (size_bytes % 8 != 0 || dst_dev % 8 != 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "fill needs 8-byte aligned size and address");
  if (size_bytes == 0) return PF_OK;
  if (int rc = check_range(dst_dev, size_bytes, "fill")) return rc;
  (void)hipGetLastError();
  PF_HIP(launch_fill_random(dst_dev, size_bytes, seed, word_offset,
                            static_cast<hipStream_t>(stream)));
  return PF_OK;
}

static int run_count_kernel(int which, uint64_t a, uint64_t b, uint64_t size,
                            uint64_t seed, uint64_t word_offset,
                            uint64_t* mismatches) {
  unsigned long long* d_count = nullptr;
  PF_HIP(hipMalloc(&d_count, sizeof(unsigned long long)));
  hipError_t e = hipMemset(d_count, 0, sizeof(unsigned long long));
  if (e == hipSuccess) {
    (void)hipGetLastError();
    e = which == 0 ? launch_verify_random(a, size, seed, word_offset, d_count, nullptr)
                   : launch_compare(a, b, size, d_count, nullptr);
  }
  unsigned long long h = 0;
  if (e == hipSuccess) e = hipMemcpy(&h, d_count, sizeof(h), hipMemcpyDeviceToHost);
  (void)hipFree(d_count);
  if (e != hipSuccess) return hip_fail(e, which == 0 ? "verify kernel" : "compare kernel");
  *mismatches = h;
  return PF_OK;
}

int pf_verify_random(uint64_t addr, uint64_t size_bytes, uint64_t seed,
                     uint64_t word_offset, uint64_t* mismatches) {
  if (size_bytes % 8 != 0 || addr % 8 != 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "verify needs 8-byte aligned size and address");
  if (size_bytes == 0) {
    *mismatches = 0;
    return PF_OK;
  }
  if (int rc = check_range(addr, size_bytes, "verify")) return rc;
  return run_count_kernel(0, addr, 0, size_bytes, seed, word_offset, mismatches);
}

int pf_verify_random_chunks(const uint64_t* addrs, const uint64_t* word_offsets,
                            uint64_t n, uint64_t chunk_bytes, uint64_t seed,
                            uint64_t* mismatches) {
  if (chunk_bytes % 8 != 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "verify needs an 8-byte multiple chunk size");
  for (uint64_t i = 0; i < n; ++i)
    if (addrs[i] % 8 != 0)
      return fail(PF_ERR_INVALID_ARGUMENT, "verify needs 8-byte aligned chunk addresses");
  *mismatches = 0;
  if (n == 0 || chunk_bytes == 0) return PF_OK;
  {
    RangeCache rc;
    for (uint64_t i = 0; i < n; ++i)
      if (!rc.check(addrs[i], chunk_bytes))
        return fail(PF_ERR_INVALID_ARGUMENT,
                    strf("verify: chunk %llu [0x%llx, +%llu) is not inside one device or "
                         "pinned allocation",
                         (unsigned long long)i, (unsigned long long)addrs[i],
                         (unsigned long long)chunk_bytes));
  }
  uint64_t* d = nullptr;
  unsigned long long* d_count = nullptr;
  PF_HIP(hipMalloc(&d, 2 * n * sizeof(uint64_t) + sizeof(unsigned long long)));
  d_count = reinterpret_cast<unsigned long long*>(d + 2 * n);
  hipError_t e = hipMemcpy(d, addrs, n * sizeof(uint64_t), hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(d + n, word_offsets, n * sizeof(uint64_t), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(d_count, 0, sizeof(unsigned long long));
  if (e == hipSuccess) {
    (void)hipGetLastError();
    e = launch_verify_random_chunks(d, d + n, n, chunk_bytes, seed, d_count, nullptr);
  }
  unsigned long long h = 0;
  if (e == hipSuccess) e = hipMemcpy(&h, d_count, sizeof(h), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "verify chunks kernel");
  *mismatches = h;
  return PF_OK;
}

int pf_compare(uint64_t a, uint64_t b, uint64_t size_bytes,
               uint64_t* mismatches) {
  if (size_bytes == 0) {
    *mismatches = 0;
    return PF_OK;
  }
  if (int rc = check_range(a, size_bytes, "compare")) return rc;
  if (int rc = check_range(b, size_bytes, "compare")) return rc;
  return run_count_kernel(1, a, b, size_bytes, 0, 0, mismatches);
}

int pf_stream_wait_word(pf_stream stream, uint64_t word, uint64_t value, uint32_t timeout_us,
                        uint64_t timed_out) {
  if ((word & 7u) != 0 || (timed_out & 3u) != 0)
    return fail(PF_ERR_INVALID_ARGUMENT, "wait word must be 8-byte aligned, timeout flag 4-byte");
  if (timeout_us > 60u * 1000u * 1000u)
    return fail(PF_ERR_INVALID_ARGUMENT, "wait timeout above 60 s");
  if (int rc = check_range(word, 8, "wait word")) return rc;
  if (timed_out)
    if (int rc = check_range(timed_out, 4, "wait timeout flag")) return rc;
  int khz = wall_clock_khz();
  if (khz <= 0) return fail(PF_ERR_INIT, "wall clock rate unknown (call pf_init)");
  const uint64_t ticks = static_cast<uint64_t>(timeout_us) * static_cast<uint64_t>(khz) / 1000;
  (void)hipGetLastError();
  PF_HIP(launch_wait_word(word, value, ticks, timed_out, static_cast<hipStream_t>(stream)));
  return PF_OK;
}

int pf_host_wait_word(const uint64_t* word, uint64_t value, uint64_t timeout_us, int* reached) {
  if (!word || !reached) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(timeout_us);
  for (uint32_t spins = 0;; ++spins) {
    if (__atomic_load_n(word, __ATOMIC_ACQUIRE) >= value) {
      *reached = 1;
      return PF_OK;
    }
    if (std::chrono::steady_clock::now() >= deadline) {
      *reached = 0;
      return PF_OK;
    }
    // Spin briefly (a layer lands every few hundred microseconds), then back off.
    if (spins > 2000) std::this_thread::sleep_for(std::chrono::microseconds(10));
  }
}

int pf_spin(pf_stream stream, uint32_t microseconds) {
  int khz = wall_clock_khz();
  if (khz <= 0) return fail(PF_ERR_INIT, "wall clock rate unknown (call pf_init)");
  uint64_t ticks = static_cast<uint64_t>(microseconds) * static_cast<uint64_t>(khz) / 1000;
  (void)hipGetLastError();
  PF_HIP(launch_spin(ticks, static_cast<hipStream_t>(stream)));
  return PF_OK;
}

}  // extern "C"

int pf_copy_engines(int device, uint32_t* d2h_engine, uint32_t* h2d_engine) {
  if (!d2h_engine || !h2d_engine) return pf::fail(PF_ERR_INVALID_ARGUMENT, "null output");
  if (int rc = pf_init(device)) return rc;
  (void)pf::engine_ids(device, d2h_engine, h2d_engine);
  return PF_OK;
}

int pf_set_copy_engines(int device, uint32_t d2h_engines, uint32_t h2d_engines) {
  if (int rc = pf_init(device)) return rc;
  return pf::set_engine_ids(device, d2h_engines, h2d_engines);
}
