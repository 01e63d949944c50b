// hpack_test.cpp — the native gRPC server's HPACK decoder (pf_hpack.cpp)
// against the worked examples of RFC 7541 Appendix C, on the host (no GPU),
// built by tests/test_native.py from the library's own sources:
//   C.1    integer representation (5-bit prefix: 10 and 1337; 8-bit: 42);
//   C.3    three requests without Huffman coding, one decoder, the dynamic
//          table's size after each;
//   C.4    the same requests with Huffman coding;
// plus malformed input: an index past the table, padding of 8 bits or more,
// a truncated string, a table size update above the limit.
// Exit status 0 and "ok" on success; the first failed check is printed.
#include <cstdio>
#include <string>
#include <vector>

#include "pf_hpack.h"

using namespace pf;

namespace {

int failures = 0;

void expect(bool cond, const std::string& what) {
  if (!cond) {
    std::printf("FAILED: %s\n", what.c_str());
    ++failures;
  }
}

std::vector<uint8_t> hex(const char* s) {
  std::vector<uint8_t> out;
  int hi = -1;
  for (; *s; ++s) {
    int v = -1;
    if (*s >= '0' && *s <= '9') v = *s - '0';
    if (*s >= 'a' && *s <= 'f') v = *s - 'a' + 10;
    if (v < 0) continue;
    if (hi < 0) {
      hi = v;
    } else {
      out.push_back(static_cast<uint8_t>(hi * 16 + v));
      hi = -1;
    }
  }
  return out;
}

std::string joined(const std::vector<HeaderField>& fs) {
  std::string s;
  for (const HeaderField& f : fs) s += f.name + ": " + f.value + "\n";
  return s;
}

void request(HpackDecoder& d, const char* block, const char* want, size_t table_size,
             const char* what) {
  const std::vector<uint8_t> b = hex(block);
  std::vector<HeaderField> out;
  std::string err;
  const bool ok = d.decode(b.data(), b.size(), &out, &err);
  expect(ok, std::string(what) + ": decode failed: " + err);
  expect(joined(out) == want, std::string(what) + ": got\n" + joined(out));
  expect(d.table_size() == table_size,
         std::string(what) + ": table size " + std::to_string(d.table_size()));
}

bool fails(const char* block) {
  HpackDecoder d;
  const std::vector<uint8_t> b = hex(block);
  std::vector<HeaderField> out;
  std::string err;
  return !d.decode(b.data(), b.size(), &out, &err);
}

}  // namespace

int main() {
  // C.1.
  {
    const uint8_t a[] = {0x0a}, b[] = {0x1f, 0x9a, 0x0a}, c[] = {0x2a};
    const uint8_t* p = a;
    uint64_t v = 0;
    expect(hpack_integer(&p, a + 1, 5, &v) && v == 10 && p == a + 1, "C.1.1: 10");
    p = b;
    expect(hpack_integer(&p, b + 3, 5, &v) && v == 1337 && p == b + 3, "C.1.2: 1337");
    p = c;
    expect(hpack_integer(&p, c + 1, 8, &v) && v == 42, "C.1.3: 42");
    p = b;
    expect(!hpack_integer(&p, b + 2, 5, &v), "truncated integer");
  }
  const char* r1 = ":method: GET\n:scheme: http\n:path: /\n:authority: www.example.com\n";
  const char* r2 =
      ":method: GET\n:scheme: http\n:path: /\n:authority: www.example.com\n"
      "cache-control: no-cache\n";
  const char* r3 =
      ":method: GET\n:scheme: https\n:path: /index.html\n:authority: www.example.com\n"
      "custom-key: custom-value\n";
  // C.3: without Huffman coding.
  {
    HpackDecoder d;
    request(d, "8286 8441 0f77 7777 2e65 7861 6d70 6c65 2e63 6f6d", r1, 57, "C.3.1");
    request(d, "8286 84be 5808 6e6f 2d63 6163 6865", r2, 110, "C.3.2");
    request(d,
            "8287 85bf 400a 6375 7374 6f6d 2d6b 6579 0c63 7573 746f 6d2d 7661 6c75 65",
            r3, 164, "C.3.3");
    expect(d.table_entries() == 3, "C.3: three dynamic entries");
  }
  // C.4: with Huffman coding.
  {
    HpackDecoder d;
    request(d, "8286 8441 8cf1 e3c2 e5f2 3a6b a0ab 90f4 ff", r1, 57, "C.4.1");
    request(d, "8286 84be 5886 a8eb 1064 9cbf", r2, 110, "C.4.2");
    request(d, "8287 85bf 4088 25a8 49e9 5ba9 7d7f 8925 a849 e95b b8e8 b4bf", r3, 164,
            "C.4.3");
  }
  // Huffman strings alone.
  {
    std::string s;
    const std::vector<uint8_t> www = hex("f1e3 c2e5 f23a 6ba0 ab90 f4ff");
    expect(hpack_huffman(www.data(), www.size(), &s) && s == "www.example.com",
           "Huffman www.example.com: " + s);
    const std::vector<uint8_t> nc = hex("a8eb 1064 9cbf");
    expect(hpack_huffman(nc.data(), nc.size(), &s) && s == "no-cache", "Huffman no-cache");
    const std::vector<uint8_t> pad = hex("a8eb 1064 9cbf ff");  // 8 more bits of padding
    expect(!hpack_huffman(pad.data(), pad.size(), &s), "Huffman padding of 8 bits");
    const std::vector<uint8_t> eos = hex("ffff ffff");  // EOS (30 ones) and more
    expect(!hpack_huffman(eos.data(), eos.size(), &s), "Huffman EOS");
  }
  // Malformed blocks.
  expect(fails("be"), "index 62 with an empty dynamic table");
  expect(fails("80"), "index 0");
  expect(fails("410f 7777"), "string shorter than its length");
  expect(fails("3fe2 1f"), "table size update above 4096");
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
