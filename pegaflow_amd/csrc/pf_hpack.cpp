// pf_hpack.cpp — HPACK header-block decoding (RFC 7541) for the native gRPC
// server.  The static table and the Huffman code are the RFC's (Appendices
// A and B), as any HTTP/2 peer's are; the code is canonical, so it is built
// here from each symbol's code length.
#include "pf_hpack.h"

#include <algorithm>
#include <array>

namespace pf {

namespace {

// RFC 7541 Appendix A.
constexpr const char* kStatic[61][2] = {
    {":authority", ""},
    {":method", "GET"},
    {":method", "POST"},
    {":path", "/"},
    {":path", "/index.html"},
    {":scheme", "http"},
    {":scheme", "https"},
    {":status", "200"},
    {":status", "204"},
    {":status", "206"},
    {":status", "304"},
    {":status", "400"},
    {":status", "404"},
    {":status", "500"},
    {"accept-charset", ""},
    {"accept-encoding", "gzip, deflate"},
    {"accept-language", ""},
    {"accept-ranges", ""},
    {"accept", ""},
    {"access-control-allow-origin", ""},
    {"age", ""},
    {"allow", ""},
    {"authorization", ""},
    {"cache-control", ""},
    {"content-disposition", ""},
    {"content-encoding", ""},
    {"content-language", ""},
    {"content-length", ""},
    {"content-location", ""},
    {"content-range", ""},
    {"content-type", ""},
    {"cookie", ""},
    {"date", ""},
    {"etag", ""},
    {"expect", ""},
    {"expires", ""},
    {"from", ""},
    {"host", ""},
    {"if-match", ""},
    {"if-modified-since", ""},
    {"if-none-match", ""},
    {"if-range", ""},
    {"if-unmodified-since", ""},
    {"last-modified", ""},
    {"link", ""},
    {"location", ""},
    {"max-forwards", ""},
    {"proxy-authenticate", ""},
    {"proxy-authorization", ""},
    {"range", ""},
    {"referer", ""},
    {"refresh", ""},
    {"retry-after", ""},
    {"server", ""},
    {"set-cookie", ""},
    {"strict-transport-security", ""},
    {"transfer-encoding", ""},
    {"user-agent", ""},
    {"vary", ""},
    {"via", ""},
    {"www-authenticate", ""},
};

// Code lengths of the symbols decoded here (RFC 7541 Appendix B): NUL and
// printable ASCII, every code of at most 19 bits.  Other symbols have codes
// of 19 to 30 bits that follow these in the canonical order.
int code_length(int sym) {
  if (sym == 0) return 13;
  if (sym < 32 || sym > 126) return 0;
  switch (sym) {
    case '0': case '1': case '2': case 'a': case 'c': case 'e': case 'i': case 'o':
    case 's': case 't':
      return 5;
    case ' ': case '%': case '-': case '.': case '/': case '3': case '4': case '5':
    case '6': case '7': case '8': case '9': case '=': case 'A': case '_': case 'b':
    case 'd': case 'f': case 'g': case 'h': case 'l': case 'm': case 'n': case 'p':
    case 'r': case 'u':
      return 6;
    case '&': case '*': case ',': case ';': case 'X': case 'Z':
      return 8;
    case '!': case '"': case '(': case ')': case '?':
      return 10;
    case '\'': case '+': case '|':
      return 11;
    case '#': case '>':
      return 12;
    case '$': case '@': case '[': case ']': case '~':
      return 13;
    case '^': case '}':
      return 14;
    case '<': case '`': case '{':
      return 15;
    case '\\':
      return 19;
    default:  // ':', 'B'-'W', 'Y', 'j', 'k', 'q', 'v'-'z'
      return 7;
  }
}

// Canonical decoding tables: per code length, the first code, the number of
// codes and where their symbols start in `syms` (ordered by length, then
// symbol value).
struct Huffman {
  std::array<uint32_t, 32> first{}, count{}, index{};
  std::vector<uint8_t> syms;
  Huffman() {
    std::vector<std::pair<int, int>> order;  // (length, symbol)
    for (int s = 0; s < 256; ++s)
      if (int l = code_length(s)) order.push_back({l, s});
    std::sort(order.begin(), order.end());
    uint32_t code = 0;
    int prev = order.front().first;
    for (size_t i = 0; i < order.size(); ++i) {
      const int len = order[i].first;
      if (i > 0) code = (code + 1) << (len - prev);
      prev = len;
      if (count[len] == 0) {
        first[len] = code;
        index[len] = static_cast<uint32_t>(syms.size());
      }
      ++count[len];
      syms.push_back(static_cast<uint8_t>(order[i].second));
    }
  }
};

const Huffman& huffman() {
  static const Huffman h;
  return h;
}

bool literal(const uint8_t** p, const uint8_t* end, std::string* out) {
  if (*p >= end) return false;
  const bool huff = (**p & 0x80) != 0;
  uint64_t len = 0;
  if (!hpack_integer(p, end, 7, &len) || len > static_cast<uint64_t>(end - *p)) return false;
  const bool ok = huff ? hpack_huffman(*p, static_cast<size_t>(len), out)
                       : (out->assign(reinterpret_cast<const char*>(*p), static_cast<size_t>(len)),
                          true);
  *p += len;
  return ok;
}

constexpr size_t kEntryOverhead = 32;   // RFC 7541 4.1
constexpr size_t kMaxDecoded = 1 << 20;  // bytes of names and values per block

}  // namespace

bool hpack_integer(const uint8_t** p, const uint8_t* end, int prefix_bits, uint64_t* out) {
  if (*p >= end) return false;
  const uint64_t mask = (1u << prefix_bits) - 1;
  uint64_t v = **p & mask;
  ++*p;
  if (v < mask) {
    *out = v;
    return true;
  }
  for (int m = 0; m < 35; m += 7) {
    if (*p >= end) return false;
    const uint8_t b = **p;
    ++*p;
    v += static_cast<uint64_t>(b & 0x7f) << m;
    if (!(b & 0x80)) {
      *out = v;
      return true;
    }
  }
  return false;
}

bool hpack_huffman(const uint8_t* p, size_t n, std::string* out) {
  const Huffman& h = huffman();
  out->clear();
  uint32_t code = 0;
  int len = 0;
  for (size_t i = 0; i < n; ++i) {
    for (int bit = 7; bit >= 0; --bit) {
      code = (code << 1) | ((p[i] >> bit) & 1u);
      ++len;
      if (h.count[len] && code >= h.first[len] && code - h.first[len] < h.count[len]) {
        out->push_back(static_cast<char>(h.syms[h.index[len] + code - h.first[len]]));
        code = 0;
        len = 0;
      } else if (len >= 30) {
        return false;  // EOS, or a symbol without a code here
      }
    }
  }
  // Padding: fewer than 8 bits, all ones (the start of EOS).
  return len < 8 && code == (1u << len) - 1u;
}

bool HpackDecoder::field(size_t index, HeaderField* f, std::string* err) const {
  if (index >= 1 && index <= 61) {
    f->name = kStatic[index - 1][0];
    f->value = kStatic[index - 1][1];
    return true;
  }
  if (index >= 62 && index - 62 < dyn_.size()) {
    *f = dyn_[index - 62];
    return true;
  }
  *err = "header index " + std::to_string(index) + " out of range";
  return false;
}

void HpackDecoder::evict_to(size_t max) {
  while (size_ > max && !dyn_.empty()) {
    size_ -= dyn_.back().name.size() + dyn_.back().value.size() + kEntryOverhead;
    dyn_.pop_back();
  }
}

void HpackDecoder::add(HeaderField f) {
  const size_t es = f.name.size() + f.value.size() + kEntryOverhead;
  if (es > max_) {  // RFC 7541 4.4: the table ends up empty
    evict_to(0);
    return;
  }
  evict_to(max_ - es);
  size_ += es;
  dyn_.push_front(std::move(f));
}

bool HpackDecoder::decode(const uint8_t* p, size_t n, std::vector<HeaderField>* out,
                          std::string* err) {
  const uint8_t* end = p + n;
  size_t decoded = 0;
  while (p < end) {
    const uint8_t b = *p;
    HeaderField f;
    uint64_t idx = 0;
    if (b & 0x80) {  // indexed field
      if (!hpack_integer(&p, end, 7, &idx) || idx == 0) {
        *err = "bad indexed header field";
        return false;
      }
      if (!field(static_cast<size_t>(idx), &f, err)) return false;
    } else if ((b & 0xe0) == 0x20) {  // dynamic table size update
      if (!hpack_integer(&p, end, 5, &idx) || idx > limit_) {
        *err = "dynamic table size update above the limit";
        return false;
      }
      max_ = static_cast<size_t>(idx);
      evict_to(max_);
      continue;
    } else {  // literal: with incremental indexing (01), without (0000) or never indexed (0001)
      const bool indexing = (b & 0xc0) == 0x40;
      if (!hpack_integer(&p, end, indexing ? 6 : 4, &idx)) {
        *err = "bad literal header field";
        return false;
      }
      if (idx) {
        HeaderField named;
        if (!field(static_cast<size_t>(idx), &named, err)) return false;
        f.name = std::move(named.name);
      } else if (!literal(&p, end, &f.name)) {
        *err = "bad header name string";
        return false;
      }
      if (!literal(&p, end, &f.value)) {
        *err = "bad header value string";
        return false;
      }
      if (indexing) add(f);
    }
    decoded += f.name.size() + f.value.size();
    if (decoded > kMaxDecoded) {
      *err = "header block too large";
      return false;
    }
    out->push_back(std::move(f));
  }
  return true;
}

}  // namespace pf
