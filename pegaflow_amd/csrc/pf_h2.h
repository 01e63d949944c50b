// pf_h2.h — HTTP/2 framing and header-block encoding for the native gRPC
// server (pf_grpc.cpp): RFC 9113 frame layout and codes, HPACK integers and
// literals (RFC 7541 5.1, 5.2, 6.2, without Huffman coding or indexing), and
// gRPC's percent-encoding of grpc-message.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace pf {
namespace h2 {

// Frame types, flags, settings and error codes (RFC 9113 6, 7).
enum : uint8_t {
  kData = 0, kHeaders = 1, kPriority = 2, kRstStream = 3, kSettings = 4, kPushPromise = 5,
  kPing = 6, kGoaway = 7, kWindowUpdate = 8, kContinuation = 9
};
constexpr uint8_t kEndStream = 0x1, kAck = 0x1, kEndHeaders = 0x4, kPadded = 0x8,
                  kPriorityFlag = 0x20;
enum : uint32_t {
  kProtocolError = 1, kFlowControlError = 3, kFrameSizeError = 6, kRefusedStream = 7,
  kCompressionError = 9
};

constexpr const char kPreface[] = "PRI * HTTP/2.0\r\n\r\nSM\r\n\r\n";
constexpr size_t kPrefaceLen = sizeof(kPreface) - 1;

inline void put32(std::string* s, uint32_t v) {
  for (int sh = 24; sh >= 0; sh -= 8) s->push_back(static_cast<char>((v >> sh) & 0xff));
}

inline void frame(std::string* out, uint8_t type, uint8_t flags, uint32_t sid, const void* p,
                  size_t n) {
  out->push_back(static_cast<char>((n >> 16) & 0xff));
  out->push_back(static_cast<char>((n >> 8) & 0xff));
  out->push_back(static_cast<char>(n & 0xff));
  out->push_back(static_cast<char>(type));
  out->push_back(static_cast<char>(flags));
  put32(out, sid & 0x7fffffffu);
  out->append(static_cast<const char*>(p), n);
}

// HPACK integer with an N-bit prefix, the prefix's other bits `first`.
inline void hp_int(std::string* s, uint8_t first, int prefix, uint64_t v) {
  const uint64_t mask = (1u << prefix) - 1;
  if (v < mask) {
    s->push_back(static_cast<char>(first | v));
    return;
  }
  s->push_back(static_cast<char>(first | mask));
  v -= mask;
  while (v >= 0x80) {
    s->push_back(static_cast<char>((v & 0x7f) | 0x80));
    v >>= 7;
  }
  s->push_back(static_cast<char>(v));
}

inline void hp_string(std::string* s, const std::string& v) {
  hp_int(s, 0x00, 7, v.size());  // no Huffman coding
  s->append(v);
}

// Literal header field without indexing: by static name index, or new name.
inline void hp_field(std::string* s, uint32_t name_index, const std::string& value) {
  hp_int(s, 0x00, 4, name_index);
  hp_string(s, value);
}
inline void hp_field(std::string* s, const std::string& name, const std::string& value) {
  s->push_back(0x00);
  hp_string(s, name);
  hp_string(s, value);
}

// grpc-message: bytes outside 0x20-0x7e, and '%', percent-encoded.
inline std::string percent_encode(const std::string& m) {
  static const char* hexd = "0123456789ABCDEF";
  std::string out;
  for (unsigned char c : m) {
    if (c >= 0x20 && c <= 0x7e && c != '%') {
      out.push_back(static_cast<char>(c));
    } else {
      out.push_back('%');
      out.push_back(hexd[c >> 4]);
      out.push_back(hexd[c & 15]);
    }
  }
  return out;
}

}  // namespace h2
}  // namespace pf
