// pf_hpack.h — HPACK header-block decoding (RFC 7541) for the native gRPC
// server (pf_grpc.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <string>
#include <vector>

namespace pf {

struct HeaderField {
  std::string name, value;
};

// The decoding context of one HTTP/2 connection's header blocks: the static
// table (RFC 7541 Appendix A) and the connection's dynamic table.  Huffman-
// coded strings (Appendix B) decode for every symbol whose code is at most
// 19 bits long: all printable ASCII and NUL, which is what gRPC's request
// headers hold; a longer code fails the block.
class HpackDecoder {
 public:
  // Largest dynamic table size the peer may ask for (the SETTINGS_HEADER_
  // TABLE_SIZE this side advertised).
  explicit HpackDecoder(size_t limit = 4096) : max_(limit), limit_(limit) {}
  // Appends the block's fields to *out; false with *err on a malformed block
  // (the connection must then be closed: the table is no longer in step).
  bool decode(const uint8_t* p, size_t n, std::vector<HeaderField>* out, std::string* err);
  size_t table_size() const { return size_; }
  size_t table_entries() const { return dyn_.size(); }

 private:
  bool field(size_t index, HeaderField* f, std::string* err) const;
  void add(HeaderField f);
  void evict_to(size_t max);
  std::deque<HeaderField> dyn_;  // front: the newest entry (index 62)
  size_t size_ = 0, max_, limit_;
};

// RFC 7541 5.1: an integer with an N-bit prefix at *p; advances *p.
bool hpack_integer(const uint8_t** p, const uint8_t* end, int prefix_bits, uint64_t* out);
// RFC 7541 Appendix B: Huffman-decodes n bytes.
bool hpack_huffman(const uint8_t* p, size_t n, std::string* out);

}  // namespace pf
