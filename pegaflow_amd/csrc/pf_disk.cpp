// pf_disk.cpp — the engine's disk tier (pegaflow-core/src/seal_offload.rs):
// packed block files written from the pinned pool by writer threads, a
// sidecar index per file (in place of Redis), a byte quota that drops the
// oldest files, and prefetch of a missed prefix back into the pinned pool by
// reader threads, after which loads take the ordinary restore path.
//
// File format (seal_offload.rs:379-448): blocks back to back; inside a
// block, its slots in slot order (layer * tp_size + tp_rank); inside a slot,
// the K half then the V half when the slot is split, else the whole slot.
// Differences: writes are gathered into pwritev calls and dropped from the
// page cache after fsync; reads of adjacent blocks are one preadv into their
// separate pool allocations; the namespace directory is hex-escaped when the
// namespace is not a plain file name.
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <sys/uio.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <chrono>
#include <random>

#include "pf_engine.h"

namespace pf {
namespace {

constexpr int kMaxIov = 1024;                // IOV_MAX on Linux
constexpr uint64_t kMaxReadRun = 256ull << 20;  // bytes per preadv run
constexpr uint64_t kReadJobBytes = 32ull << 20;  // bytes per reader job

std::string to_hex(const uint8_t* p, size_t n) {
  static const char* d = "0123456789abcdef";
  std::string s(2 * n, '0');
  for (size_t i = 0; i < n; ++i) {
    s[2 * i] = d[p[i] >> 4];
    s[2 * i + 1] = d[p[i] & 15];
  }
  return s;
}

bool from_hex(const std::string& s, std::string* out) {
  if (s.size() % 2) return false;
  out->resize(s.size() / 2);
  for (size_t i = 0; i < s.size(); i += 2) {
    int v = 0;
    for (int k = 0; k < 2; ++k) {
      const char c = s[i + k];
      int x = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : -1;
      if (x < 0) return false;
      v = v * 16 + x;
    }
    (*out)[i / 2] = static_cast<char>(v);
  }
  return true;
}

// Version-4 UUID in the hyphenated lower-case form the reference's file names use.
std::string uuid_v4() {
  static std::mutex mu;
  static std::mt19937_64 rng([] {
    std::random_device rd;
    return (static_cast<uint64_t>(rd()) << 32) ^ rd();
  }());
  uint8_t b[16];
  {
    std::lock_guard<std::mutex> lk(mu);
    const uint64_t a = rng(), c = rng();
    std::memcpy(b, &a, 8);
    std::memcpy(b + 8, &c, 8);
  }
  b[6] = static_cast<uint8_t>((b[6] & 0x0f) | 0x40);
  b[8] = static_cast<uint8_t>((b[8] & 0x3f) | 0x80);
  const std::string h = to_hex(b, 16);
  return h.substr(0, 8) + "-" + h.substr(8, 4) + "-" + h.substr(12, 4) + "-" + h.substr(16, 4) +
         "-" + h.substr(20, 12);
}

bool mkdirs(const std::string& path) {
  std::string cur;
  size_t i = 0;
  while (i <= path.size()) {
    const size_t j = path.find('/', i);
    cur = path.substr(0, j == std::string::npos ? path.size() : j);
    if (!cur.empty() && ::mkdir(cur.c_str(), 0755) != 0 && errno != EEXIST) return false;
    if (j == std::string::npos) break;
    i = j + 1;
  }
  struct stat sb;
  return ::stat(path.c_str(), &sb) == 0 && S_ISDIR(sb.st_mode);
}

// Full positional vectored I/O: retries short transfers and EINTR.
bool rw_all(bool write, int fd, std::vector<iovec> iov, uint64_t off) {
  size_t i = 0;
  while (i < iov.size()) {
    const int cnt = static_cast<int>(std::min<size_t>(kMaxIov, iov.size() - i));
    const ssize_t n = write ? ::pwritev(fd, &iov[i], cnt, static_cast<off_t>(off))
                            : ::preadv(fd, &iov[i], cnt, static_cast<off_t>(off));
    if (n < 0 && errno == EINTR) continue;
    if (n <= 0) return false;  // error, or end of file on a read
    off += static_cast<uint64_t>(n);
    size_t left = static_cast<size_t>(n);
    while (left > 0) {
      if (left >= iov[i].iov_len) {
        left -= iov[i].iov_len;
        ++i;
      } else {
        iov[i].iov_base = static_cast<uint8_t*>(iov[i].iov_base) + left;
        iov[i].iov_len -= left;
        left = 0;
      }
    }
    while (i < iov.size() && iov[i].iov_len == 0) ++i;
  }
  return true;
}

bool write_file(const std::string& path, const std::string& text) {
  const int fd = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (fd < 0) return false;
  std::vector<iovec> iov{{const_cast<char*>(text.data()), text.size()}};
  const bool ok = (text.empty() || rw_all(true, fd, iov, 0)) && ::fsync(fd) == 0;
  ::close(fd);
  return ok;
}

bool read_file(const std::string& path, std::string* out) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return false;
  struct stat sb;
  bool ok = ::fstat(fd, &sb) == 0 && sb.st_size >= 0 && sb.st_size < (64 << 20);
  if (ok) {
    out->resize(static_cast<size_t>(sb.st_size));
    std::vector<iovec> iov{{&(*out)[0], out->size()}};
    ok = out->empty() || rw_all(false, fd, iov, 0);
  }
  ::close(fd);
  return ok;
}

// ---------------------------------------------------------------------------
// JSON: the writer renders exactly what serde_json renders for BlockMeta;
// the reader accepts the subset the sidecars use (objects, arrays, strings,
// unsigned integers, booleans, null).
// ---------------------------------------------------------------------------
void json_str(std::string* o, const std::string& s) {
  o->push_back('"');
  for (unsigned char c : s) {
    switch (c) {
      case '"': *o += "\\\""; break;
      case '\\': *o += "\\\\"; break;
      case '\n': *o += "\\n"; break;
      case '\r': *o += "\\r"; break;
      case '\t': *o += "\\t"; break;
      case '\b': *o += "\\b"; break;
      case '\f': *o += "\\f"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", c);
          *o += buf;
        } else {
          o->push_back(static_cast<char>(c));
        }
    }
  }
  o->push_back('"');
}

struct JVal {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  bool b = false;
  uint64_t n = 0;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;
  const JVal* get(const char* k) const {
    for (const auto& kv : o)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char* p;
  const char* e;
  int depth = 0;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool lit(const char* w) {
    const size_t n = std::strlen(w);
    if (static_cast<size_t>(e - p) < n || std::memcmp(p, w, n) != 0) return false;
    p += n;
    return true;
  }
  bool str(std::string* out) {
    if (p >= e || *p != '"') return false;
    ++p;
    out->clear();
    while (p < e && *p != '"') {
      char c = *p++;
      if (c != '\\') {
        out->push_back(c);
        continue;
      }
      if (p >= e) return false;
      c = *p++;
      switch (c) {
        case '"': case '\\': case '/': out->push_back(c); break;
        case 'n': out->push_back('\n'); break;
        case 'r': out->push_back('\r'); break;
        case 't': out->push_back('\t'); break;
        case 'b': out->push_back('\b'); break;
        case 'f': out->push_back('\f'); break;
        case 'u': {
          if (e - p < 4) return false;
          unsigned v = 0;
          for (int i = 0; i < 4; ++i) {
            const char h = *p++;
            const int d = h >= '0' && h <= '9'   ? h - '0'
                          : h >= 'a' && h <= 'f' ? h - 'a' + 10
                          : h >= 'A' && h <= 'F' ? h - 'A' + 10
                                                 : -1;
            if (d < 0) return false;
            v = v * 16 + static_cast<unsigned>(d);
          }
          if (v < 0x80) {
            out->push_back(static_cast<char>(v));
          } else if (v < 0x800) {
            out->push_back(static_cast<char>(0xc0 | (v >> 6)));
            out->push_back(static_cast<char>(0x80 | (v & 0x3f)));
          } else {
            out->push_back(static_cast<char>(0xe0 | (v >> 12)));
            out->push_back(static_cast<char>(0x80 | ((v >> 6) & 0x3f)));
            out->push_back(static_cast<char>(0x80 | (v & 0x3f)));
          }
          break;
        }
        default: return false;
      }
    }
    if (p >= e) return false;
    ++p;
    return true;
  }
  bool val(JVal* v) {
    ws();
    if (p >= e || ++depth > 16) return false;
    bool ok = true;
    if (*p == '{') {
      v->kind = JVal::kObj;
      ++p;
      ws();
      if (p < e && *p == '}') {
        ++p;
      } else {
        for (;;) {
          std::string k;
          ws();
          JVal x;
          if (!str(&k)) return false;
          ws();
          if (p >= e || *p++ != ':') return false;
          if (!val(&x)) return false;
          v->o.emplace_back(std::move(k), std::move(x));
          ws();
          if (p < e && *p == ',') { ++p; continue; }
          if (p < e && *p == '}') { ++p; break; }
          return false;
        }
      }
    } else if (*p == '[') {
      v->kind = JVal::kArr;
      ++p;
      ws();
      if (p < e && *p == ']') {
        ++p;
      } else {
        for (;;) {
          JVal x;
          if (!val(&x)) return false;
          v->a.push_back(std::move(x));
          ws();
          if (p < e && *p == ',') { ++p; continue; }
          if (p < e && *p == ']') { ++p; break; }
          return false;
        }
      }
    } else if (*p == '"') {
      v->kind = JVal::kStr;
      ok = str(&v->s);
    } else if (*p >= '0' && *p <= '9') {
      v->kind = JVal::kNum;
      uint64_t n = 0;
      while (p < e && *p >= '0' && *p <= '9') {
        const uint64_t d = static_cast<uint64_t>(*p++ - '0');
        if (n > (UINT64_MAX - d) / 10) return false;
        n = n * 10 + d;
      }
      if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) return false;
      v->n = n;
    } else if (lit("true")) {
      v->kind = JVal::kBool;
      v->b = true;
    } else if (lit("false")) {
      v->kind = JVal::kBool;
    } else if (lit("null")) {
      v->kind = JVal::kNull;
    } else {
      return false;
    }
    --depth;
    return ok;
  }
};

bool parse_json(const std::string& text, JVal* out) {
  JParser jp{text.data(), text.data() + text.size()};
  if (!jp.val(out)) return false;
  jp.ws();
  return jp.p == jp.e;
}

bool get_u64(const JVal& o, const char* k, uint64_t* out) {
  const JVal* v = o.get(k);
  if (!v || v->kind != JVal::kNum) return false;
  *out = v->n;
  return true;
}

bool get_str(const JVal& o, const char* k, std::string* out) {
  const JVal* v = o.get(k);
  if (!v || v->kind != JVal::kStr) return false;
  *out = v->s;
  return true;
}

bool meta_from_json(const JVal& j, DiskBlockMeta* m) {
  if (j.kind != JVal::kObj || !get_str(j, "file", &m->file) || !get_u64(j, "offset", &m->offset) ||
      !get_u64(j, "total_slots", &m->total_slots))
    return false;
  const JVal* slots = j.get("slots");
  if (!slots || slots->kind != JVal::kArr) return false;
  m->slots.clear();
  for (const JVal& s : slots->a) {
    DiskSlotMeta sm;
    const JVal* split = s.kind == JVal::kObj ? s.get("is_split") : nullptr;
    if (!split || split->kind != JVal::kBool || !get_u64(s, "size", &sm.size)) return false;
    sm.is_split = split->b;
    if (sm.is_split && sm.size % 2) return false;
    m->slots.push_back(sm);
  }
  return true;
}

std::string ns_of(const std::string& key) { return key.substr(0, key.find('\0')); }
std::string hash_of(const std::string& key) {
  const size_t sep = key.find('\0');
  return sep == std::string::npos ? std::string() : key.substr(sep + 1);
}

std::shared_ptr<SealedBlock> rebuild(const std::shared_ptr<PoolAllocation>& alloc,
                                     const DiskBlockMeta& meta) {
  // rebuild_sealed_block, seal_offload.rs:869-909: every slot points into the
  // one allocation the block was read into.
  auto sb = std::make_shared<SealedBlock>();
  uint64_t off = 0;
  for (const DiskSlotMeta& sm : meta.slots) {
    auto lb = std::make_shared<LayerBlock>();
    lb->size = sm.size;
    lb->k_ptr = alloc->ptr + off;
    lb->k_alloc = alloc;
    if (sm.is_split) {
      lb->v_ptr = alloc->ptr + off + sm.size / 2;
      lb->v_alloc = alloc;
    }
    sb->slots.push_back(std::move(lb));
    off += sm.size;
  }
  sb->footprint = off;
  sb->index();
  return sb;
}

}  // namespace

std::string block_meta_json(const DiskBlockMeta& m) {
  std::string o = "{\"file\":";
  json_str(&o, m.file);
  o += ",\"offset\":" + std::to_string(m.offset) + ",\"slots\":[";
  for (size_t i = 0; i < m.slots.size(); ++i) {
    if (i) o.push_back(',');
    o += std::string("{\"is_split\":") + (m.slots[i].is_split ? "true" : "false") +
         ",\"size\":" + std::to_string(m.slots[i].size) + "}";
  }
  o += "],\"total_slots\":" + std::to_string(m.total_slots) + "}";
  return o;
}

std::string DiskTier::dir_name(const std::string& ns) {
  bool plain = !ns.empty() && ns != "." && ns != "..";
  for (unsigned char c : ns)
    plain = plain && (std::isalnum(c) || c == '.' || c == '_' || c == '-');
  return plain ? ns : "ns-" + to_hex(reinterpret_cast<const uint8_t*>(ns.data()), ns.size());
}

int DiskTier::open(const DiskConfig& cfg, BlockStore* store, std::unique_ptr<DiskTier>* out) {
  if (cfg.root.empty()) return fail(PF_ERR_INVALID_ARGUMENT, "invalid argument: empty disk root");
  if (cfg.max_pack_blocks == 0 || cfg.max_prefetch_tasks == 0 || cfg.io_threads == 0 ||
      cfg.io_threads > 64)
    return fail(PF_ERR_INVALID_ARGUMENT,
                "invalid argument: disk tier needs max_pack_blocks, max_prefetch_tasks >= 1 and "
                "1..64 io threads");
  if (!mkdirs(cfg.root))
    return fail(PF_ERR_STORAGE, strf("storage error: cannot create disk root %s: %s",
                                     cfg.root.c_str(), std::strerror(errno)));
  std::unique_ptr<DiskTier> d(new DiskTier());
  d->cfg_ = cfg;
  d->store_ = store;
  d->rescan();
  for (size_t i = 0; i < cfg.io_threads; ++i) {
    d->writers_.emplace_back([t = d.get()] { t->writer_loop(); });
    d->readers_.emplace_back([t = d.get()] { t->reader_loop(); });
  }
  *out = std::move(d);
  return PF_OK;
}

DiskTier::~DiskTier() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
    for (auto& job : read_q_)
      for (auto& b : job.blocks) pending_.erase(b.first);
    read_q_.clear();
  }
  write_cv_.notify_all();
  read_cv_.notify_all();
  for (auto& t : writers_)  // the writers drain the queue first
    if (t.joinable()) t.join();
  for (auto& t : readers_)
    if (t.joinable()) t.join();
}

void DiskTier::rescan() {
  struct Found {
    int64_t mtime;
    std::string ns_dir, uuid, ns;
    uint64_t size;
    std::vector<std::pair<std::string, DiskBlockMeta>> blocks;
  };
  std::vector<Found> found;
  DIR* root = ::opendir(cfg_.root.c_str());
  if (!root) return;
  while (dirent* de = ::readdir(root)) {
    const std::string nsd = de->d_name;
    if (nsd == "." || nsd == "..") continue;
    const std::string dir = cfg_.root + "/" + nsd;
    DIR* sub = ::opendir(dir.c_str());
    if (!sub) continue;
    while (dirent* fe = ::readdir(sub)) {
      const std::string name = fe->d_name;
      if (name.size() <= 5 || name.compare(name.size() - 5, 5, ".json") != 0) continue;
      const std::string uuid = name.substr(0, name.size() - 5);
      std::string text;
      JVal j;
      Found f;
      f.ns_dir = nsd;
      f.uuid = uuid;
      struct stat sb, bb;
      std::string file;
      uint64_t version = 0;
      bool ok = read_file(dir + "/" + name, &text) && parse_json(text, &j) &&
                j.kind == JVal::kObj && get_u64(j, "version", &version) && version == 1 &&
                get_str(j, "namespace", &f.ns) && get_str(j, "file", &file) &&
                file == uuid + ".bin" && get_u64(j, "size", &f.size) &&
                ::stat((dir + "/" + name).c_str(), &sb) == 0 &&
                ::stat((dir + "/" + file).c_str(), &bb) == 0 &&
                static_cast<uint64_t>(bb.st_size) == f.size;
      const JVal* blocks = ok ? j.get("blocks") : nullptr;
      ok = ok && blocks && blocks->kind == JVal::kArr;
      for (size_t i = 0; ok && i < blocks->a.size(); ++i) {
        const JVal& b = blocks->a[i];
        std::string hx, raw;
        DiskBlockMeta m;
        const JVal* mj = b.kind == JVal::kObj ? b.get("meta") : nullptr;
        ok = get_str(b, "hash", &hx) && from_hex(hx, &raw) && mj && meta_from_json(*mj, &m) &&
             m.file == file && m.offset + m.total_size() <= f.size;
        if (ok) f.blocks.emplace_back(f.ns + std::string(1, '\0') + raw, std::move(m));
      }
      if (!ok) {
        ++st_.failures;
        continue;
      }
      f.mtime = static_cast<int64_t>(sb.st_mtim.tv_sec) * 1000000000 + sb.st_mtim.tv_nsec;
      found.push_back(std::move(f));
    }
    ::closedir(sub);
  }
  ::closedir(root);
  std::sort(found.begin(), found.end(), [](const Found& a, const Found& b) {
    return a.mtime != b.mtime ? a.mtime < b.mtime : a.uuid < b.uuid;
  });
  std::lock_guard<std::mutex> lk(mu_);
  for (auto& f : found) {  // oldest first, so newer copies of a block win
    FileEntry fe{f.ns_dir, f.uuid, {}, f.size, next_seq_++};
    for (auto& b : f.blocks) {
      fe.keys.push_back(b.first);
      index_[b.first] = std::move(b.second);
    }
    by_age_[fe.seq] = f.uuid;
    usage_ += f.size;
    files_[f.uuid] = std::move(fe);
  }
  enforce_quota_locked();
}

void DiskTier::on_seal(const std::string& key, const std::shared_ptr<SealedBlock>& block) {
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (stop_ || index_.count(key)) return;  // already on disk
    write_q_.emplace_back(key, block);
    if (write_q_.size() % cfg_.max_pack_blocks != 0 && write_q_.size() != 1) return;
  }
  write_cv_.notify_one();  // on the first block, and whenever a file's worth is queued
}

void DiskTier::writer_loop() {
  for (;;) {
    std::vector<std::pair<std::string, std::weak_ptr<SealedBlock>>> batch;
    {
      std::unique_lock<std::mutex> lk(mu_);
      write_cv_.wait(lk, [this] { return stop_ || !write_q_.empty(); });
      if (write_q_.empty()) return;  // stopping, and drained
      // Seals arrive in bursts (a save seals its blocks together): linger
      // briefly so a burst fills whole files instead of a first tiny one.
      if (!stop_ && write_q_.size() < cfg_.max_pack_blocks)
        write_cv_.wait_for(lk, std::chrono::milliseconds(2), [this] {
          return stop_ || write_q_.size() >= cfg_.max_pack_blocks;
        });
      if (write_q_.empty()) continue;  // another writer took them
      while (!write_q_.empty() && batch.size() < cfg_.max_pack_blocks) {
        batch.push_back(std::move(write_q_.front()));
        write_q_.pop_front();
      }
      ++writing_;
    }
    // offload_loop, seal_offload.rs:235-365: drop blocks evicted meanwhile,
    // then one packed file per namespace.
    std::map<std::string, std::vector<std::pair<std::string, std::shared_ptr<SealedBlock>>>> by_ns;
    for (auto& kv : batch)
      if (auto b = kv.second.lock()) by_ns[ns_of(kv.first)].emplace_back(kv.first, std::move(b));
    for (auto& kv : by_ns)
      if (write_packed(kv.first, kv.second) != PF_OK) {
        std::lock_guard<std::mutex> lk(mu_);
        ++st_.failures;
      }
    {
      std::lock_guard<std::mutex> lk(mu_);
      --writing_;
    }
    idle_cv_.notify_all();
  }
}

int DiskTier::write_packed(
    const std::string& ns,
    const std::vector<std::pair<std::string, std::shared_ptr<SealedBlock>>>& blocks) {
  const std::string nsd = dir_name(ns);
  const std::string dir = cfg_.root + "/" + nsd;
  if (!mkdirs(dir)) return fail(PF_ERR_STORAGE, "storage error: cannot create " + dir);
  const std::string uuid = uuid_v4(), file = uuid + ".bin";
  const uint64_t total_slots = blocks.front().second->slots.size();
  std::vector<std::pair<std::string, DiskBlockMeta>> metas;
  std::vector<iovec> iov;
  uint64_t off = 0;
  for (const auto& kv : blocks) {
    const SealedBlock& sb = *kv.second;
    bool whole = true;
    for (const auto& s : sb.slots) whole = whole && s && s->k_ptr && (!s->v_ptr || s->size % 2 == 0);
    if (!whole) continue;
    DiskBlockMeta m;
    m.file = file;
    m.offset = off;
    m.total_slots = total_slots;
    for (const auto& s : sb.slots) {
      m.slots.push_back(DiskSlotMeta{s->v_ptr != nullptr, s->size});
      if (s->v_ptr) {
        iov.push_back(iovec{s->k_ptr, s->size / 2});
        iov.push_back(iovec{s->v_ptr, s->size / 2});
      } else {
        iov.push_back(iovec{s->k_ptr, s->size});
      }
    }
    off += m.total_size();
    metas.emplace_back(kv.first, std::move(m));
  }
  if (metas.empty()) return PF_OK;
  const std::string path = dir + "/" + file;
  const int fd = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (fd < 0) return fail(PF_ERR_STORAGE, "storage error: cannot create " + path);
  bool ok = rw_all(true, fd, iov, 0) && ::fsync(fd) == 0;
  if (ok) (void)::posix_fadvise(fd, 0, 0, POSIX_FADV_DONTNEED);  // written once, read rarely
  ::close(fd);
  std::string side = "{\"version\":1,\"namespace\":";
  json_str(&side, ns);
  side += ",\"file\":\"" + file + "\",\"size\":" + std::to_string(off) + ",\"blocks\":[";
  for (size_t i = 0; i < metas.size(); ++i) {
    if (i) side.push_back(',');
    const std::string h = hash_of(metas[i].first);
    side += "{\"hash\":\"" + to_hex(reinterpret_cast<const uint8_t*>(h.data()), h.size()) +
            "\",\"meta\":" + block_meta_json(metas[i].second) + "}";
  }
  side += "]}\n";
  const std::string side_path = dir + "/" + uuid + ".json";
  ok = ok && write_file(side_path + ".tmp", side) &&
       ::rename((side_path + ".tmp").c_str(), side_path.c_str()) == 0;
  if (!ok) {
    ::unlink((side_path + ".tmp").c_str());
    ::unlink(path.c_str());
    return fail(PF_ERR_STORAGE, "storage error: writing " + path + " failed");
  }
  std::lock_guard<std::mutex> lk(mu_);
  FileEntry fe{nsd, uuid, {}, off, next_seq_++};
  for (auto& kv : metas) {
    fe.keys.push_back(kv.first);
    index_[kv.first] = std::move(kv.second);
  }
  by_age_[fe.seq] = uuid;
  usage_ += off;
  st_.offloaded_blocks += metas.size();
  st_.written_bytes += off;
  files_[uuid] = std::move(fe);
  enforce_quota_locked();
  return PF_OK;
}

// check_quota / evict_oldest (seal_offload.rs:454-571): whole files, oldest
// first, until usage is within the quota.
void DiskTier::enforce_quota_locked() {
  while (usage_ > cfg_.quota_bytes && !by_age_.empty()) {
    const std::string uuid = by_age_.begin()->second;
    by_age_.erase(by_age_.begin());
    auto it = files_.find(uuid);
    if (it == files_.end()) continue;
    FileEntry fe = std::move(it->second);
    files_.erase(it);
    for (const auto& k : fe.keys) {
      auto ix = index_.find(k);
      if (ix != index_.end() && ix->second.file == uuid + ".bin") index_.erase(ix);
    }
    usage_ -= fe.size;
    ++st_.evicted_files;
    const std::string dir = cfg_.root + "/" + fe.ns_dir + "/";
    ::unlink((dir + uuid + ".json").c_str());  // the index entry goes first
    ::unlink((dir + uuid + ".bin").c_str());
  }
}

void DiskTier::query(const std::vector<std::string>& keys, int* state, uint64_t* ready,
                     uint64_t* loading, uint64_t* missing) {
  std::unique_lock<std::mutex> lk(mu_);
  uint64_t r = 0, l = 0;
  size_t miss = keys.size();
  for (size_t i = 0; i < keys.size(); ++i) {
    if (store_->cache_contains(keys[i])) {
      ++r;
    } else if (pending_.count(keys[i])) {
      ++l;
    } else {
      miss = i;
      break;
    }
  }
  *missing = 0;
  if (miss == keys.size()) {
    *state = l ? kPrefetchLoading : kPrefetchReady;
    *ready = r;
    *loading = l;
    return;
  }
  const uint64_t n = keys.size();
  if (active_tasks_ >= cfg_.max_prefetch_tasks) {  // lib.rs:896-903
    *state = kPrefetchPartialMiss;
    *ready = r;
    *loading = 0;
    *missing = n - r - l;
    return;
  }
  if (!index_.count(keys[miss])) {  // lib.rs:905-921
    *state = kPrefetchPartialMiss;
    *ready = r + l;
    *loading = 0;
    *missing = n - r - l;
    return;
  }
  // prefetch_blocks_inner (seal_offload.rs:683-780): the rest of the prefix
  // that is on disk, not cached and not being read, grouped by file.
  std::map<std::string, ReadJob> jobs;
  for (size_t i = miss; i < keys.size(); ++i) {
    const std::string& k = keys[i];
    if (pending_.count(k) || store_->cache_contains(k)) continue;
    auto ix = index_.find(k);
    if (ix == index_.end()) continue;
    const std::string uuid = ix->second.file.substr(0, ix->second.file.size() - 4);
    auto fe = files_.find(uuid);
    if (fe == files_.end()) continue;
    pending_[k] = 1;
    ReadJob& job = jobs[uuid];
    job.path = cfg_.root + "/" + fe->second.ns_dir + "/" + ix->second.file;
    job.blocks.emplace_back(k, ix->second);
  }
  if (!jobs.empty()) {
    // Each file's blocks, in offset order, are cut into jobs of about
    // kReadJobBytes so that every reader thread has work until the end.
    std::vector<ReadJob> parts;
    for (auto& kv : jobs) {
      auto& bl = kv.second.blocks;
      std::sort(bl.begin(), bl.end(),
                [](const auto& a, const auto& b) { return a.second.offset < b.second.offset; });
      ReadJob cur;
      uint64_t bytes = 0;
      for (auto& b : bl) {
        if (!cur.blocks.empty() && bytes >= kReadJobBytes) {
          cur.path = kv.second.path;
          parts.push_back(std::move(cur));
          cur = ReadJob();
          bytes = 0;
        }
        bytes += b.second.total_size();
        cur.blocks.push_back(std::move(b));
      }
      cur.path = kv.second.path;
      parts.push_back(std::move(cur));
    }
    ++active_tasks_;
    auto left = std::make_shared<std::atomic<size_t>>(parts.size());
    for (auto& job : parts) {
      job.parts_left = left;
      read_q_.push_back(std::move(job));
    }
  }
  *state = kPrefetchLoading;
  *ready = r;
  *loading = l + (n - miss);
  lk.unlock();
  read_cv_.notify_all();
}

void DiskTier::reader_loop() {
  for (;;) {
    ReadJob job;
    {
      std::unique_lock<std::mutex> lk(mu_);
      read_cv_.wait(lk, [this] { return stop_ || !read_q_.empty(); });
      if (stop_ || read_q_.empty()) {
        if (stop_) return;
        continue;
      }
      job = std::move(read_q_.front());
      read_q_.pop_front();
      ++reading_;
    }
    read_job(job);
    {
      std::lock_guard<std::mutex> lk(mu_);
      --reading_;
      if (job.parts_left && job.parts_left->fetch_sub(1) == 1) --active_tasks_;
    }
    idle_cv_.notify_all();
  }
}

// read_file_blocks (seal_offload.rs:790-867), with runs of adjacent blocks
// read by one preadv into their separate pool allocations.
void DiskTier::read_job(ReadJob& job) {
  auto& blocks = job.blocks;
  std::sort(blocks.begin(), blocks.end(),
            [](const auto& a, const auto& b) { return a.second.offset < b.second.offset; });
  auto done = [this](const std::string& key, bool failed) {
    std::lock_guard<std::mutex> lk(mu_);
    pending_.erase(key);
    if (failed) ++st_.failures;
  };
  const int fd = ::open(job.path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    for (auto& b : blocks) done(b.first, true);
    return;
  }
  (void)::posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
  size_t i = 0;
  while (i < blocks.size()) {
    const DiskBlockMeta& first = blocks[i].second;
    if (first.total_slots == 0 || first.total_size() == 0) {  // seal_offload.rs:808-815
      done(blocks[i].first, false);
      ++i;
      continue;
    }
    std::vector<std::shared_ptr<PoolAllocation>> allocs;
    std::vector<iovec> iov;
    uint64_t next = first.offset, bytes = 0;
    size_t j = i;
    while (j < blocks.size() && blocks[j].second.offset == next && bytes < kMaxReadRun) {
      const uint64_t size = blocks[j].second.total_size();
      if (size == 0 || blocks[j].second.total_slots == 0) break;
      auto a = store_->allocate(size);
      if (!a) break;
      iov.push_back(iovec{a->ptr, size});
      allocs.push_back(std::move(a));
      next += size;
      bytes += size;
      ++j;
    }
    if (allocs.empty()) {  // the pool cannot hold the block
      done(blocks[i].first, true);
      ++i;
      continue;
    }
    const bool ok = rw_all(false, fd, iov, first.offset);
    for (size_t k = 0; k < allocs.size(); ++k) {
      const auto& b = blocks[i + k];
      if (ok) {
        store_->cache_insert(b.first, rebuild(allocs[k], b.second));
        std::lock_guard<std::mutex> lk(mu_);
        ++st_.prefetched_blocks;
        st_.read_bytes += b.second.total_size();
      }
      done(b.first, !ok);
    }
    i += allocs.size();
  }
  ::close(fd);
}

void DiskTier::flush() {
  std::unique_lock<std::mutex> lk(mu_);
  idle_cv_.wait(lk, [this] { return write_q_.empty() && writing_ == 0; });
}

void DiskTier::wait_prefetch() {
  std::unique_lock<std::mutex> lk(mu_);
  idle_cv_.wait(lk, [this] { return read_q_.empty() && reading_ == 0; });
}

DiskStats DiskTier::stats() {
  std::lock_guard<std::mutex> lk(mu_);
  DiskStats s = st_;
  s.files = files_.size();
  s.bytes = usage_;
  s.indexed_blocks = index_.size();
  s.pending_blocks = pending_.size();
  return s;
}

}  // namespace pf
