// pf_load_state.cpp — LoadState, the cross-process completion word of an
// asynchronous load (the role of pegaflow-core/src/sync_state.rs).
//
// Mapping layout (native endian), identical to the reference for the first
// 32 bytes so either side can attach to the other's state:
//   [0, 8)    u64 offset of the record from the mapping start (8 when the
//             mapping is page aligned)                  sync_state.rs:27-30
//   offset:   u32 magic 0x50464C44 ('PFLD'), u32 version 1, i64 state
//             (0 pending, 1 success, -1 error)          sync_state.rs:19-43
//   mapping size 32 = 8 + sizeof(record) + alignof(record)  sync_state.rs:190-193
// Layered extension (absent from the reference), at byte 32:
//   u32 magic 0x50464C58 ('PFLX'), u32 num_layers, i64 layers_done
// so the per-layer completion of a layer-wise load is visible to a process
// that polls the shared memory, while a reader of the original record still
// attaches (it only requires the mapping to hold at least 32 bytes).
// Event block (optional, after the extension), at byte 48:
//   u32 magic 0x50464C45 ('PFLE'), u32 count, i64 events_recorded, then
//   count 64-byte interprocess event handles, one per layer; the loader
//   records layer l's event after layer l's copy and then publishes
//   events_recorded = count, after which a consumer can wait on the device.
//   Magic 0x50464C4C ('PFLL') marks the in-process variant: each 64-byte
//   slot holds the address of an event of the loader's own process in its
//   first 8 bytes (zeros after), recorded as it is.
// Words block (optional, instead of the event block), at byte 48:
//   u32 magic 0x50464C57 ('PFLW'), u32 count, u64 value, u32 kind,
//   u32 reserved, u64 address, u64 alloc_size, u64 offset, 64-byte IPC
//   memory handle (112 bytes): count 8-byte words of device memory, one per
//   layer, that the loader sets to value once that layer's bytes are in
//   place.  kind 0: the words are at offset in the allocation exported as
//   handle (alloc_size bytes); kind 1: at address in the loader's own
//   process.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/random.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <random>
#include <string>

#include "pf_common.h"

using namespace pf;

namespace {

constexpr uint32_t kMagic = 0x50464C44u;  // 'PFLD'
constexpr uint32_t kVersion = 1;
constexpr uint32_t kExtMagic = 0x50464C58u;  // 'PFLX'
constexpr size_t kMetaSize = 8;
constexpr size_t kRecordSize = 16;
constexpr size_t kRecordAlign = 8;
constexpr size_t kAllocSize = kMetaSize + kRecordSize + kRecordAlign;  // 32
constexpr size_t kExtOffset = kAllocSize;
constexpr size_t kExtSize = 16;
constexpr uint32_t kEvMagic = 0x50464C45u;       // 'PFLE'
constexpr uint32_t kEvLocalMagic = 0x50464C4Cu;  // 'PFLL'
constexpr size_t kEvOffset = kExtOffset + kExtSize;  // 48
constexpr size_t kEvSize = 16;
constexpr size_t kHandleBytes = PF_IPC_HANDLE_BYTES;
constexpr uint32_t kMaxEvents = 4096;

struct Record {
  uint32_t magic;
  uint32_t version;
  int64_t state;
};
static_assert(sizeof(Record) == kRecordSize, "record layout");

struct ExtRecord {
  uint32_t magic;
  uint32_t num_layers;
  int64_t layers_done;
};
static_assert(sizeof(ExtRecord) == kExtSize, "extension layout");

struct EvRecord {
  uint32_t magic;
  uint32_t count;
  int64_t recorded;
};
static_assert(sizeof(EvRecord) == kEvSize, "event block layout");

constexpr uint32_t kWordsMagic = 0x50464C57u;  // 'PFLW'
struct WordsRecord {
  uint32_t magic;
  uint32_t count;
  uint64_t value;
  uint32_t kind;
  uint32_t reserved;
  uint64_t address;
  uint64_t alloc_size;
  uint64_t offset;
  uint8_t handle[kHandleBytes];
};
static_assert(sizeof(WordsRecord) == 112, "words block layout");

std::string random_name() {
  // "pega_load_" + uuid-v4 in simple (32 lowercase hex) form (sync_state.rs:126).
  // getrandom: one system call (a std::random_device costs about 30 us to
  // construct, half the cost of creating a LoadState).
  uint8_t b[16];
  size_t got = 0;
  while (got < sizeof(b)) {
    const ssize_t r = getrandom(b + got, sizeof(b) - got, 0);
    if (r > 0) {
      got += static_cast<size_t>(r);
    } else if (r < 0 && errno != EINTR) {
      std::random_device rd;  // no getrandom: the library's own source
      for (; got < sizeof(b); ++got) b[got] = static_cast<uint8_t>(rd());
    }
  }
  b[6] = (b[6] & 0x0f) | 0x40;
  b[8] = (b[8] & 0x3f) | 0x80;
  static const char* hex = "0123456789abcdef";
  std::string s = "pega_load_";
  for (int i = 0; i < 16; ++i) {
    s.push_back(hex[b[i] >> 4]);
    s.push_back(hex[b[i] & 15]);
  }
  return s;
}

}  // namespace

struct pf_load_state {
  std::string name;
  uint8_t* map = nullptr;
  size_t len = 0;
  bool owner = false;
  Record* rec = nullptr;
  ExtRecord* ext = nullptr;
  EvRecord* ev = nullptr;
  bool ev_local = false;  // the event block holds in-process event addresses
  WordsRecord* words = nullptr;
};

namespace {

int create_state(uint32_t num_layers, bool layered, const uint8_t* handles,
                 const pf_layer_words* words, pf_load_state** out, bool local_events = false) {
  if (!out) return fail(PF_ERR_INVALID_ARGUMENT, "null output");
  if (handles && (num_layers == 0 || num_layers > kMaxEvents))
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("a LoadState carries 1..%u layer events, got %u", kMaxEvents, num_layers));
  if (words) {
    if (num_layers == 0 || num_layers > kMaxEvents)
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("a LoadState carries words for 1..%u layers, got %u", kMaxEvents,
                       num_layers));
    if (words->value == 0 || words->kind > PF_LAYER_WORDS_LOCAL || words->reserved != 0 ||
        (words->kind == PF_LAYER_WORDS_LOCAL ? (words->address & 7u) != 0
                                             : (words->offset & 7u) != 0 ||
                                                   words->alloc_size < words->offset ||
                                                   (words->alloc_size - words->offset) / 8 <
                                                       num_layers))
      return fail(PF_ERR_INVALID_ARGUMENT,
                  "layer words: value must be nonzero, words 8-byte aligned and inside the "
                  "allocation");
  }
  const size_t size = handles ? kEvOffset + kEvSize + num_layers * kHandleBytes
                      : words ? kEvOffset + sizeof(WordsRecord)
                      : layered ? kExtOffset + kExtSize : kAllocSize;
  std::string name;
  int fd = -1;
  for (int attempt = 0; attempt < 8 && fd < 0; ++attempt) {
    name = random_name();
    fd = shm_open(name.c_str(), O_CREAT | O_EXCL | O_RDWR, S_IRUSR | S_IWUSR);
    if (fd < 0 && errno != EEXIST) break;
  }
  if (fd < 0)
    return fail(PF_ERR_LOAD_STATE,
                strf("failed to create shared memory: %s", std::strerror(errno)));
  if (ftruncate(fd, static_cast<off_t>(size)) != 0) {
    int err = errno;
    close(fd);
    shm_unlink(name.c_str());
    return fail(PF_ERR_LOAD_STATE,
                strf("failed to create shared memory: %s", std::strerror(err)));
  }
  void* m = mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  close(fd);
  if (m == MAP_FAILED) {
    shm_unlink(name.c_str());
    return fail(PF_ERR_LOAD_STATE,
                strf("failed to create shared memory: %s", std::strerror(errno)));
  }
  uint8_t* base = static_cast<uint8_t*>(m);
  // init_new_mapping (sync_state.rs:201-242): align base+8 up to the record's
  // alignment and store the offset in the first 8 bytes.
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  const uintptr_t aligned = (b + kMetaSize + kRecordAlign - 1) & ~(uintptr_t)(kRecordAlign - 1);
  const uint64_t offset = aligned - b;
  std::memcpy(base, &offset, sizeof(offset));
  auto* st = new pf_load_state();
  st->name = name;
  st->map = base;
  st->len = size;
  st->owner = true;
  st->rec = reinterpret_cast<Record*>(base + offset);
  __atomic_store_n(&st->rec->magic, kMagic, __ATOMIC_RELEASE);
  __atomic_store_n(&st->rec->version, kVersion, __ATOMIC_RELEASE);
  __atomic_store_n(&st->rec->state, (int64_t)PF_LOAD_PENDING, __ATOMIC_RELEASE);
  if (layered) {
    st->ext = reinterpret_cast<ExtRecord*>(base + kExtOffset);
    __atomic_store_n(&st->ext->num_layers, num_layers, __ATOMIC_RELEASE);
    __atomic_store_n(&st->ext->layers_done, (int64_t)0, __ATOMIC_RELEASE);
    __atomic_store_n(&st->ext->magic, kExtMagic, __ATOMIC_RELEASE);
  }
  if (handles) {
    st->ev = reinterpret_cast<EvRecord*>(base + kEvOffset);
    std::memcpy(base + kEvOffset + kEvSize, handles, num_layers * kHandleBytes);
    __atomic_store_n(&st->ev->count, num_layers, __ATOMIC_RELEASE);
    __atomic_store_n(&st->ev->recorded, (int64_t)0, __ATOMIC_RELEASE);
    st->ev_local = local_events;
    __atomic_store_n(&st->ev->magic, local_events ? kEvLocalMagic : kEvMagic, __ATOMIC_RELEASE);
  }
  if (words) {
    st->words = reinterpret_cast<WordsRecord*>(base + kEvOffset);
    WordsRecord* w = st->words;
    w->count = num_layers;
    w->value = words->value;
    w->kind = words->kind;
    w->reserved = 0;
    w->address = words->address;
    w->alloc_size = words->alloc_size;
    w->offset = words->offset;
    std::memcpy(w->handle, words->handle, kHandleBytes);
    __atomic_store_n(&w->magic, kWordsMagic, __ATOMIC_RELEASE);
  }
  *out = st;
  return PF_OK;
}

}  // namespace

extern "C" {

int pf_load_state_create(pf_load_state** out) {
  return create_state(0, false, nullptr, nullptr, out);
}

int pf_load_state_create_layered(uint32_t num_layers, pf_load_state** out) {
  return create_state(num_layers, true, nullptr, nullptr, out);
}

int pf_load_state_create_layered_events(uint32_t num_layers, const uint8_t* event_handles,
                                        pf_load_state** out) {
  if (!event_handles) return fail(PF_ERR_INVALID_ARGUMENT, "null event handles");
  // Where this runtime cannot export interprocess events no loader could be
  // handed real ones: refused up front rather than at the loader's open.
  // Without a device the handles are opaque bytes, kept as given.
  std::string why;
  if (ipc_events_supported(&why) == 0)
    return fail(PF_ERR_UNSUPPORTED,
                "a LoadState of interprocess event handles: this runtime cannot export "
                "interprocess events (" + why + "); use layer words instead");
  return create_state(num_layers, true, event_handles, nullptr, out);
}

int pf_load_state_create_layered_local_events(uint32_t num_layers, const pf_event* events,
                                              pf_load_state** out) {
  if (!events) return fail(PF_ERR_INVALID_ARGUMENT, "null events");
  if (num_layers == 0 || num_layers > kMaxEvents)
    return fail(PF_ERR_INVALID_ARGUMENT,
                strf("a LoadState carries 1..%u layer events, got %u", kMaxEvents, num_layers));
  std::string slots(static_cast<size_t>(num_layers) * kHandleBytes, '\0');
  for (uint32_t l = 0; l < num_layers; ++l) {
    if (!events[l]) return fail(PF_ERR_INVALID_ARGUMENT, strf("null event for layer %u", l));
    const uint64_t a = reinterpret_cast<uint64_t>(events[l]);
    std::memcpy(&slots[static_cast<size_t>(l) * kHandleBytes], &a, sizeof(a));
  }
  return create_state(num_layers, true, reinterpret_cast<const uint8_t*>(slots.data()), nullptr,
                      out, true);
}

int pf_load_state_create_layered_words(uint32_t num_layers, const pf_layer_words* words,
                                       pf_load_state** out) {
  if (!words) return fail(PF_ERR_INVALID_ARGUMENT, "null layer words");
  return create_state(num_layers, true, nullptr, words, out);
}

// LoadState::attach + attach_mapping + validate_header (sync_state.rs:145-155,
// 244-292).
int pf_load_state_attach(const char* shm_name, pf_load_state** out) {
  if (!shm_name || !out) return fail(PF_ERR_INVALID_ARGUMENT, "null argument");
  int fd = shm_open(shm_name, O_RDWR, S_IRUSR);
  if (fd < 0)
    return fail(PF_ERR_LOAD_STATE,
                strf("failed to open shared memory: %s", std::strerror(errno)));
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    int err = errno;
    close(fd);
    return fail(PF_ERR_LOAD_STATE, strf("failed to open shared memory: %s", std::strerror(err)));
  }
  const size_t len = static_cast<size_t>(sb.st_size);
  if (len < kAllocSize) {
    close(fd);
    return fail(PF_ERR_LOAD_STATE,
                strf("shared memory too small (actual=%zu bytes, required=%zu bytes)", len,
                     kAllocSize));
  }
  void* m = mmap(nullptr, len, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  close(fd);
  if (m == MAP_FAILED)
    return fail(PF_ERR_LOAD_STATE,
                strf("failed to open shared memory: %s", std::strerror(errno)));
  uint8_t* base = static_cast<uint8_t*>(m);
  uint64_t offset = 0;
  std::memcpy(&offset, base, sizeof(offset));
  auto bail = [&](int code, const std::string& msg) {
    munmap(m, len);
    return fail(code, msg);
  };
  if (offset < kMetaSize)
    return bail(PF_ERR_LOAD_STATE,
                strf("invalid LoadState offset (offset=%llu, len=%zu) recorded in shared memory",
                     (unsigned long long)offset, len));
  if (offset > len || len - offset < kRecordSize)
    return bail(PF_ERR_LOAD_STATE,
                strf("shared memory too small (actual=%zu bytes, required=%llu bytes)", len,
                     (unsigned long long)(offset + kRecordSize)));
  if ((reinterpret_cast<uintptr_t>(base) + offset) % kRecordAlign != 0)
    return bail(PF_ERR_LOAD_STATE,
                strf("aligned pointer 0x%llx is not %zu-byte aligned",
                     (unsigned long long)(reinterpret_cast<uintptr_t>(base) + offset),
                     kRecordAlign));
  Record* rec = reinterpret_cast<Record*>(base + offset);
  const uint32_t magic = __atomic_load_n(&rec->magic, __ATOMIC_ACQUIRE);
  const uint32_t version = __atomic_load_n(&rec->version, __ATOMIC_ACQUIRE);
  if (magic != kMagic || version != kVersion)
    return bail(PF_ERR_LOAD_STATE,
                strf("invalid LoadState header (magic=0x%x, version=%u, expected magic=0x%x, "
                     "version=%u)",
                     magic, version, kMagic, kVersion));
  auto* st = new pf_load_state();
  st->name = shm_name;
  st->map = base;
  st->len = len;
  st->owner = false;
  st->rec = rec;
  if (len >= kExtOffset + kExtSize) {
    ExtRecord* ext = reinterpret_cast<ExtRecord*>(base + kExtOffset);
    if (__atomic_load_n(&ext->magic, __ATOMIC_ACQUIRE) == kExtMagic) st->ext = ext;
  }
  if (st->ext && len >= kEvOffset + kEvSize) {
    EvRecord* ev = reinterpret_cast<EvRecord*>(base + kEvOffset);
    const uint32_t count = __atomic_load_n(&ev->count, __ATOMIC_ACQUIRE);
    const uint32_t ev_magic = __atomic_load_n(&ev->magic, __ATOMIC_ACQUIRE);
    if ((ev_magic == kEvMagic || ev_magic == kEvLocalMagic) && count > 0 && count <= kMaxEvents &&
        len >= kEvOffset + kEvSize + count * kHandleBytes) {
      st->ev = ev;
      st->ev_local = ev_magic == kEvLocalMagic;
    }
  }
  if (st->ext && len >= kEvOffset + sizeof(WordsRecord)) {
    WordsRecord* w = reinterpret_cast<WordsRecord*>(base + kEvOffset);
    if (__atomic_load_n(&w->magic, __ATOMIC_ACQUIRE) == kWordsMagic && w->count > 0 &&
        w->count <= kMaxEvents && w->value != 0 && w->kind <= PF_LAYER_WORDS_LOCAL)
      st->words = w;
  }
  *out = st;
  return PF_OK;
}

int pf_load_state_close(pf_load_state* st) {
  if (!st) return PF_OK;
  if (st->map) munmap(st->map, st->len);
  if (st->owner) shm_unlink(st->name.c_str());
  delete st;
  return PF_OK;
}

const char* pf_load_state_name(const pf_load_state* st) { return st->name.c_str(); }

int64_t pf_load_state_get(const pf_load_state* st) {
  return __atomic_load_n(&st->rec->state, __ATOMIC_ACQUIRE);
}

void pf_load_state_set_completed(pf_load_state* st) {
  if (st->ext) {
    const int64_t n = static_cast<int64_t>(__atomic_load_n(&st->ext->num_layers, __ATOMIC_ACQUIRE));
    __atomic_store_n(&st->ext->layers_done, n, __ATOMIC_RELEASE);
  }
  __atomic_store_n(&st->rec->state, (int64_t)PF_LOAD_SUCCESS, __ATOMIC_RELEASE);
}

void pf_load_state_set_error(pf_load_state* st) {
  __atomic_store_n(&st->rec->state, (int64_t)PF_LOAD_ERROR, __ATOMIC_RELEASE);
}

uint32_t pf_load_state_num_layers(const pf_load_state* st) {
  return st->ext ? __atomic_load_n(&st->ext->num_layers, __ATOMIC_ACQUIRE) : 0;
}

int64_t pf_load_state_layers_done(const pf_load_state* st) {
  if (!st->ext) return pf_load_state_get(st) == PF_LOAD_SUCCESS ? 1 : 0;
  return __atomic_load_n(&st->ext->layers_done, __ATOMIC_ACQUIRE);
}

void pf_load_state_set_layers_done(pf_load_state* st, int64_t n) {
  if (st->ext) __atomic_store_n(&st->ext->layers_done, n, __ATOMIC_RELEASE);
}

const uint8_t* pf_load_state_event_handles(const pf_load_state* st, uint32_t* count) {
  if (!st->ev) {
    if (count) *count = 0;
    return nullptr;
  }
  if (count) *count = __atomic_load_n(&st->ev->count, __ATOMIC_ACQUIRE);
  return reinterpret_cast<const uint8_t*>(st->ev) + kEvSize;
}

int pf_load_state_events_local(const pf_load_state* st) { return st->ev && st->ev_local ? 1 : 0; }

int64_t pf_load_state_events_recorded(const pf_load_state* st) {
  return st->ev ? __atomic_load_n(&st->ev->recorded, __ATOMIC_ACQUIRE) : 0;
}

void pf_load_state_set_events_recorded(pf_load_state* st, int64_t n) {
  if (st->ev) __atomic_store_n(&st->ev->recorded, n, __ATOMIC_RELEASE);
}

int pf_load_state_layer_words(const pf_load_state* st, pf_layer_words* out, uint32_t* count) {
  if (!st->words) {
    if (count) *count = 0;
    return PF_OK;
  }
  if (out) {
    const WordsRecord* w = st->words;
    out->kind = w->kind;
    out->reserved = 0;
    out->value = w->value;
    out->address = w->address;
    out->alloc_size = w->alloc_size;
    out->offset = w->offset;
    std::memcpy(out->handle, w->handle, kHandleBytes);
  }
  if (count) *count = st->words->count;
  return PF_OK;
}

}  // extern "C"
