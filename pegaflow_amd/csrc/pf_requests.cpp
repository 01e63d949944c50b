// pf_requests.cpp — the engine's own decoder of the Engine service's Load
// and Save request bytes (engine.proto LoadRequest / SaveRequest), served on
// the calling thread: the native gRPC server (pf_grpc.cpp) hands each Load
// and Save message to pf_engine_serve_request, which decodes it and calls
// the engine as the reference's service does (service.rs:184-250).  Every
// read is bounds-checked; a message that does not decode fails with
// PF_ERR_MALFORMED.

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "pf_common.h"

using namespace pf;

namespace {

// ---------------------------------------------------------------------------
// Protobuf wire reading (proto3): varints, length-delimited fields, fixed
// widths skipped.  Every read is bounds-checked against the message.
// ---------------------------------------------------------------------------
class Wire {
 public:
  Wire(const uint8_t* p, size_t n) : p_(p), end_(p + n) {}
  bool done() const { return p_ >= end_; }
  const uint8_t* pos() const { return p_; }
  bool varint(uint64_t* v) {
    uint64_t r = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p_ >= end_) return false;
      const uint8_t b = *p_++;
      r |= static_cast<uint64_t>(b & 0x7f) << shift;
      if (!(b & 0x80)) {
        *v = r;
        return true;
      }
    }
    return false;
  }
  bool tag(uint32_t* field, uint32_t* wt) {
    uint64_t t = 0;
    if (!varint(&t) || (t >> 3) == 0 || (t >> 3) > 0x1fffffff) return false;
    *field = static_cast<uint32_t>(t >> 3);
    *wt = static_cast<uint32_t>(t & 7);
    return true;
  }
  bool bytes(const uint8_t** p, size_t* n) {
    uint64_t len = 0;
    if (!varint(&len) || len > static_cast<uint64_t>(end_ - p_)) return false;
    *p = p_;
    *n = static_cast<size_t>(len);
    p_ += len;
    return true;
  }
  bool skip(uint32_t wt) {
    uint64_t v = 0;
    const uint8_t* p = nullptr;
    size_t n = 0;
    switch (wt) {
      case 0: return varint(&v);
      case 1: return advance(8);
      case 2: return bytes(&p, &n);
      case 5: return advance(4);
      default: return false;
    }
  }

 private:
  bool advance(size_t n) {
    if (n > static_cast<size_t>(end_ - p_)) return false;
    p_ += n;
    return true;
  }
  const uint8_t* p_;
  const uint8_t* end_;
};

// A repeated int32 field: one varint (wire type 0) or a packed run (2).
bool read_int32s(Wire& w, uint32_t wt, std::vector<int32_t>* out) {
  uint64_t v = 0;
  if (wt == 0) {
    if (!w.varint(&v)) return false;
    out->push_back(static_cast<int32_t>(static_cast<uint32_t>(v)));
    return true;
  }
  if (wt != 2) return false;
  const uint8_t* p = nullptr;
  size_t n = 0;
  if (!w.bytes(&p, &n)) return false;
  out->reserve(out->size() + n);  // at least one byte per varint
  Wire packed(p, n);
  while (!packed.done()) {
    if (!packed.varint(&v)) return false;
    out->push_back(static_cast<int32_t>(static_cast<uint32_t>(v)));
  }
  return true;
}

// UTF-8 as RFC 3629 defines it: no overlong forms, no surrogates, nothing
// above U+10FFFF.  A proto3 string field must hold it (a decoder refuses the
// message otherwise, as prost and protobuf's own parsers do).
bool valid_utf8(const uint8_t* p, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    size_t len = 0;
    uint8_t lo = 0x80, hi = 0xBF;  // allowed range of the second byte
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3;
      if (c == 0xE0) lo = 0xA0;  // overlong
      if (c == 0xED) hi = 0x9F;  // surrogates
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4;
      if (c == 0xF0) lo = 0x90;  // overlong
      if (c == 0xF4) hi = 0x8F;  // above U+10FFFF
    } else {
      return false;
    }
    if (n - i < len || p[i + 1] < lo || p[i + 1] > hi) return false;
    for (size_t k = 2; k < len; ++k)
      if ((p[i + k] & 0xC0) != 0x80) return false;
    i += len;
  }
  return true;
}

bool read_string(Wire& w, uint32_t wt, std::string* out) {
  const uint8_t* p = nullptr;
  size_t n = 0;
  if (wt != 2 || !w.bytes(&p, &n) || !valid_utf8(p, n)) return false;
  out->assign(reinterpret_cast<const char*>(p), n);
  return true;
}

bool read_scalar(Wire& w, uint32_t wt, uint64_t* v) { return wt == 0 && w.varint(v); }

// Hash lists as the engine takes them: one byte buffer and n + 1 offsets.
struct Hashes {
  std::vector<uint8_t> data;
  std::vector<uint64_t> offs{0};
  size_t size() const { return offs.size() - 1; }
  bool add(Wire& w, uint32_t wt) {
    const uint8_t* p = nullptr;
    size_t n = 0;
    if (wt != 2 || !w.bytes(&p, &n)) return false;
    data.insert(data.end(), p, p + n);
    offs.push_back(data.size());
    return true;
  }
};

// engine.proto LoadRequest (fields as in pegaflow_amd/rpc/proto.py).
struct LoadReq {
  std::string instance_id, load_state_shm;
  uint64_t tp_rank = 0, device_id = 0;  // uint32 and int32 fields: truncated at use
  std::vector<std::string> layer_names;
  std::vector<int32_t> block_ids;
  Hashes hashes;
};

bool decode_load(const uint8_t* p, size_t n, LoadReq* r) {
  Wire w(p, n);
  uint32_t f = 0, wt = 0;
  while (!w.done()) {
    if (!w.tag(&f, &wt)) return false;
    bool ok = true;
    switch (f) {
      case 1: ok = read_string(w, wt, &r->instance_id); break;
      case 2: ok = read_scalar(w, wt, &r->tp_rank); break;
      case 3: ok = read_scalar(w, wt, &r->device_id); break;
      case 4: ok = read_string(w, wt, &r->load_state_shm); break;
      case 5: r->layer_names.emplace_back(); ok = read_string(w, wt, &r->layer_names.back()); break;
      case 6: ok = read_int32s(w, wt, &r->block_ids); break;
      case 7: ok = r->hashes.add(w, wt); break;
      default: ok = w.skip(wt); break;
    }
    if (!ok) return false;
  }
  return true;
}

// engine.proto SaveRequest and SaveLayer.  A connector's save names the
// same block ids and the same hashes in every layer (32 x 640 hashes for the
// Llama prefix: 0.7 ms to decode one by one), so a layer whose id or hash
// fields are byte for byte the previous layer's shares that layer's decoded
// list: one memcmp instead of a decode, and the engine then sees the very
// same arrays (its per-list work runs once).
struct Field {  // where one repeated field's entries lie in a SaveLayer
  const uint8_t* p = nullptr;
  size_t n = 0;       // bytes from the first entry's tag to the last's end
  size_t bytes = 0;   // bytes of all the entries
  bool adjacent = true;
  bool same_as(const Field& o) const {
    return adjacent && o.adjacent && n == o.n && (n == 0 || std::memcmp(p, o.p, n) == 0);
  }
  void note(const uint8_t* at, const uint8_t* end) {
    if (bytes == 0) p = at;
    else if (p + n != at) adjacent = false;
    n = static_cast<size_t>(end - p);
    bytes += static_cast<size_t>(end - at);
  }
};

struct SaveLayerReq {
  std::string layer_name;
  std::vector<int32_t> own_ids;
  Hashes own_hashes;
  Field ids_field, hashes_field;
  int ids_from = -1, hashes_from = -1;  // the layer whose lists these are (-1: own)
  // The message after a leading name field, and whether a name field
  // follows in it (then a later name wins, as protobuf's last-one-wins).
  const uint8_t* rest = nullptr;
  size_t rest_n = 0;
  bool name_in_rest = false;
};

bool decode_save_layer(const uint8_t* p, size_t n, const SaveLayerReq* prev, int prev_index,
                       SaveLayerReq* r) {
  uint32_t f = 0, wt = 0;
  // The name, which encoders write first; the rest of the message is
  // usually the previous layer's, byte for byte.
  r->rest = p;
  {
    Wire h(p, n);
    if (!h.done()) {
      if (!h.tag(&f, &wt)) return false;
      if (f == 1) {
        if (!read_string(h, wt, &r->layer_name)) return false;
        r->rest = h.pos();
      }
    }
  }
  r->rest_n = static_cast<size_t>(p + n - r->rest);
  if (prev && !prev->name_in_rest && prev->rest_n == r->rest_n &&
      std::memcmp(prev->rest, r->rest, r->rest_n) == 0) {
    r->ids_from = prev->ids_from >= 0 ? prev->ids_from : prev_index;
    r->hashes_from = prev->hashes_from >= 0 ? prev->hashes_from : prev_index;
    r->ids_field = prev->ids_field;  // the same bytes: compared by content
    r->hashes_field = prev->hashes_field;
    return true;
  }
  // Pass 1: where the id and hash fields lie.
  Wire w(r->rest, r->rest_n);
  while (!w.done()) {
    const uint8_t* at = w.pos();
    if (!w.tag(&f, &wt)) return false;
    bool ok = true;
    switch (f) {
      case 1:
        r->name_in_rest = true;
        ok = read_string(w, wt, &r->layer_name);
        break;
      case 2: {
        uint64_t v = 0;
        const uint8_t* q = nullptr;
        size_t m = 0;
        ok = wt == 0 ? w.varint(&v) : (wt == 2 && w.bytes(&q, &m));
        if (ok) r->ids_field.note(at, w.pos());
        break;
      }
      case 3: {
        const uint8_t* q = nullptr;
        size_t m = 0;
        ok = wt == 2 && w.bytes(&q, &m);
        if (ok) r->hashes_field.note(at, w.pos());
        break;
      }
      default: ok = w.skip(wt); break;
    }
    if (!ok) return false;
  }
  if (prev && r->ids_field.same_as(prev->ids_field))
    r->ids_from = prev->ids_from >= 0 ? prev->ids_from : prev_index;
  if (prev && r->hashes_field.same_as(prev->hashes_field))
    r->hashes_from = prev->hashes_from >= 0 ? prev->hashes_from : prev_index;
  const bool ids = r->ids_from < 0 && r->ids_field.bytes > 0;
  const bool hashes = r->hashes_from < 0 && r->hashes_field.bytes > 0;
  if (!ids && !hashes) return true;
  // Pass 2: the lists not shared.
  if (hashes) {
    r->own_hashes.data.reserve(r->hashes_field.bytes);
    r->own_hashes.offs.reserve(r->hashes_field.bytes / 2 + 1);  // >= 2 bytes per entry
  }
  Wire v(r->rest, r->rest_n);
  while (!v.done()) {
    if (!v.tag(&f, &wt)) return false;
    bool ok = true;
    if (f == 2 && ids) ok = read_int32s(v, wt, &r->own_ids);
    else if (f == 3 && hashes) ok = r->own_hashes.add(v, wt);
    else ok = v.skip(wt);
    if (!ok) return false;
  }
  return true;
}

struct SaveReq {
  std::string instance_id;
  uint64_t tp_rank = 0, device_id = 0;
  std::vector<SaveLayerReq> saves;
  const std::vector<int32_t>& ids(const SaveLayerReq& s) const {
    return s.ids_from < 0 ? s.own_ids : saves[static_cast<size_t>(s.ids_from)].own_ids;
  }
  const Hashes& hashes(const SaveLayerReq& s) const {
    return s.hashes_from < 0 ? s.own_hashes : saves[static_cast<size_t>(s.hashes_from)].own_hashes;
  }
};

bool decode_save(const uint8_t* p, size_t n, SaveReq* r) {
  Wire w(p, n);
  uint32_t f = 0, wt = 0;
  while (!w.done()) {
    if (!w.tag(&f, &wt)) return false;
    bool ok = true;
    const uint8_t* q = nullptr;
    size_t m = 0;
    switch (f) {
      case 1: ok = read_string(w, wt, &r->instance_id); break;
      case 2: ok = read_scalar(w, wt, &r->tp_rank); break;
      case 3: ok = read_scalar(w, wt, &r->device_id); break;
      case 4:
        ok = wt == 2 && w.bytes(&q, &m);
        if (ok) {
          const int prev = static_cast<int>(r->saves.size()) - 1;
          r->saves.emplace_back();
          ok = decode_save_layer(q, m, prev >= 0 ? &r->saves[static_cast<size_t>(prev)] : nullptr,
                                 prev, &r->saves.back());
        }
        break;
      default: ok = w.skip(wt); break;
    }
    if (!ok) return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Requests against the engine.  Results are (status, message) as the gRPC
// service would turn them into status codes.
// ---------------------------------------------------------------------------
int serve_load(pf_engine* e, const uint8_t* p, size_t n) {
  LoadReq r;
  if (!decode_load(p, n, &r)) return fail(PF_ERR_MALFORMED, "malformed LoadRequest");
  // lib.rs:1008-1043: every hash is looked up; ids pair with hashes up to
  // the shorter list (extra hashes get id -1, skipped; extra ids dropped).
  const size_t nh = r.hashes.size();
  r.block_ids.resize(nh, -1);
  std::vector<const char*> names;
  names.reserve(r.layer_names.size());
  for (const std::string& s : r.layer_names) names.push_back(s.c_str());
  return pf_engine_batch_load(e, r.instance_id.c_str(), static_cast<uint32_t>(r.tp_rank),
                              static_cast<int>(static_cast<int32_t>(r.device_id)),
                              r.load_state_shm.c_str(), names.data(),
                              static_cast<uint32_t>(names.size()), r.block_ids.data(),
                              r.hashes.data.data(), r.hashes.offs.data(), nh);
}

int serve_save(pf_engine* e, const uint8_t* p, size_t n) {
  SaveReq r;
  if (!decode_save(p, n, &r)) return fail(PF_ERR_MALFORMED, "malformed SaveRequest");
  std::vector<pf_save_layer> layers;
  layers.reserve(r.saves.size());
  for (const SaveLayerReq& s : r.saves) {
    const std::vector<int32_t>& ids = r.ids(s);
    const Hashes& hs = r.hashes(s);
    if (ids.size() != hs.size())  // lib.rs:563-569
      return fail(PF_ERR_INVALID_ARGUMENT,
                  strf("invalid argument: block_ids length %zu does not match block_hashes %zu",
                       ids.size(), hs.size()));
    layers.push_back(pf_save_layer{s.layer_name.c_str(), ids.data(), ids.size(),
                                   hs.data.data(), hs.offs.data()});
  }
  return pf_engine_batch_save(e, r.instance_id.c_str(), static_cast<uint32_t>(r.tp_rank),
                              static_cast<int>(static_cast<int32_t>(r.device_id)), layers.data(),
                              static_cast<uint32_t>(layers.size()));
}

}  // namespace

extern "C" {

int pf_engine_serve_request(pf_engine* engine, uint32_t method, const uint8_t* request,
                            uint64_t size) {
  if (!engine) return fail(PF_ERR_INVALID_ARGUMENT, "null engine");
  if (size > 0 && !request) return fail(PF_ERR_INVALID_ARGUMENT, "null request");
  clear_error();
  switch (method) {
    case PF_REQUEST_LOAD: return serve_load(engine, request, static_cast<size_t>(size));
    case PF_REQUEST_SAVE: return serve_save(engine, request, static_cast<size_t>(size));
    case PF_REQUEST_HEALTH: return PF_OK;
    default: return fail(PF_ERR_INVALID_ARGUMENT, strf("unknown method %u", method));
  }
}

}  // extern "C"
