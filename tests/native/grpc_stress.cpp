// grpc_stress.cpp — the native gRPC server (pf_grpc.cpp) under concurrent
// clients, on the host (no GPU), built by tests/test_native.py from the
// library's own sources under ThreadSanitizer and AddressSanitizer+UBSan.
//
// A host-memory engine serves on 127.0.0.1; 4 client threads each open a
// connection (raw HTTP/2 frames, header blocks as HPACK literals) and send
// 50 rounds of 4 requests in flight at once: Health (served on the
// connection's thread) and Query (handed to the handler below on a worker
// thread, which answers through pf_grpc_reply), plus a PING per round.
// Every reply must arrive, in order per stream, with grpc-status 0 and the
// expected message bytes.  Then the server is stopped with the connections
// still open.  Exit status 0 and "ok" on success.
#include <arpa/inet.h>
#include <netinet/in.h>
#include <netinet/tcp.h>
#include <sys/socket.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <vector>

#include "pegaflow_hip.h"

namespace {

std::atomic<int> failures{0};
std::atomic<int> handled{0};
std::atomic<int> clients_done{0};

void expect(bool cond, const std::string& what) {
  if (!cond && failures.fetch_add(1) < 10) std::printf("FAILED: %s\n", what.c_str());
}

// The Query handler's reply: an arbitrary message body.
const uint8_t kQueryReply[] = {0x0a, 0x02, 0x08, 0x01, 0x10, 0x07};

void handler(void*, pf_grpc_call* call, const char* method, const uint8_t*, uint64_t size) {
  handled.fetch_add(1);
  if (std::strcmp(method, "Query") == 0 && size == 3)
    (void)pf_grpc_reply(call, 0, nullptr, kQueryReply, sizeof(kQueryReply));
  else
    (void)pf_grpc_reply(call, 3, "unexpected request", nullptr, 0);
}

void frame(std::string* out, uint8_t type, uint8_t flags, uint32_t sid, const std::string& p) {
  out->push_back(static_cast<char>((p.size() >> 16) & 0xff));
  out->push_back(static_cast<char>((p.size() >> 8) & 0xff));
  out->push_back(static_cast<char>(p.size() & 0xff));
  out->push_back(static_cast<char>(type));
  out->push_back(static_cast<char>(flags));
  for (int sh = 24; sh >= 0; sh -= 8) out->push_back(static_cast<char>((sid >> sh) & 0xff));
  out->append(p);
}

// Literal header field without indexing, new name (lengths below 127).
void literal(std::string* b, const std::string& name, const std::string& value) {
  b->push_back(0x00);
  b->push_back(static_cast<char>(name.size()));
  b->append(name);
  b->push_back(static_cast<char>(value.size()));
  b->append(value);
}

std::string request(uint32_t sid, const std::string& path, const std::string& msg) {
  std::string block;
  block.push_back(static_cast<char>(0x83));  // :method POST
  block.push_back(static_cast<char>(0x86));  // :scheme http
  literal(&block, ":path", path);
  literal(&block, "content-type", "application/grpc");
  literal(&block, "te", "trailers");
  std::string body;
  body.push_back(0);
  for (int sh = 24; sh >= 0; sh -= 8)
    body.push_back(static_cast<char>((msg.size() >> sh) & 0xff));
  body.append(msg);
  std::string out;
  frame(&out, 1, 0x4, sid, block);  // HEADERS, END_HEADERS
  frame(&out, 0, 0x1, sid, body);   // DATA, END_STREAM
  return out;
}

bool read_exact(int fd, void* p, size_t n) {
  char* q = static_cast<char*>(p);
  while (n > 0) {
    const ssize_t r = ::recv(fd, q, n, 0);
    if (r <= 0) return false;
    q += r;
    n -= static_cast<size_t>(r);
  }
  return true;
}

bool send_all(int fd, const std::string& s) {
  size_t off = 0;
  while (off < s.size()) {
    const ssize_t r = ::send(fd, s.data() + off, s.size() - off, MSG_NOSIGNAL);
    if (r <= 0) return false;
    off += static_cast<size_t>(r);
  }
  return true;
}

struct Reply {
  std::string data;
  bool ok_status = false, ended = false;
  int headers = 0;
};

void client(int port, int id) {
  const int fd = ::socket(AF_INET, SOCK_STREAM, 0);
  sockaddr_in a{};
  a.sin_family = AF_INET;
  a.sin_port = htons(static_cast<uint16_t>(port));
  a.sin_addr.s_addr = htonl(INADDR_LOOPBACK);
  if (::connect(fd, reinterpret_cast<sockaddr*>(&a), sizeof(a)) != 0) {
    expect(false, "connect");
    ::close(fd);
    return;
  }
  std::string hello = "PRI * HTTP/2.0\r\n\r\nSM\r\n\r\n";
  frame(&hello, 4, 0, 0, "");
  expect(send_all(fd, hello), "send preface");
  uint32_t sid = 1;
  for (int round = 0; round < 50 && failures.load() == 0; ++round) {
    std::map<uint32_t, Reply> want;  // stream -> reply; even streams Health, odd Query
    std::string out;
    for (int k = 0; k < 4; ++k) {
      const bool health = (k % 2) == 0;
      out += request(sid, health ? "/pegaflow.Engine/Health" : "/pegaflow.Engine/Query",
                     health ? std::string() : std::string("\x0a\x01x", 3));
      want[sid] = Reply();
      sid += 2;
    }
    frame(&out, 6, 0, 0, std::string("ping") + static_cast<char>(id) + "abc");
    expect(send_all(fd, out), "send requests");
    size_t ended = 0;
    bool pong = false;
    while (ended < want.size() || !pong) {
      uint8_t h[9];
      if (!read_exact(fd, h, 9)) {
        expect(false, "connection closed early");
        ::close(fd);
        return;
      }
      const uint32_t len = (uint32_t(h[0]) << 16) | (uint32_t(h[1]) << 8) | h[2];
      const uint32_t s = ((uint32_t(h[5]) & 0x7f) << 24) | (uint32_t(h[6]) << 16) |
                         (uint32_t(h[7]) << 8) | h[8];
      std::string p(len, '\0');
      if (len && !read_exact(fd, &p[0], len)) {
        expect(false, "short frame");
        ::close(fd);
        return;
      }
      if (h[3] == 4 && !(h[4] & 1)) {  // the server's SETTINGS: acknowledge
        std::string ack;
        frame(&ack, 4, 1, 0, "");
        expect(send_all(fd, ack), "send settings ack");
      } else if (h[3] == 6 && (h[4] & 1)) {
        expect(p == std::string("ping") + static_cast<char>(id) + "abc", "ping payload");
        pong = true;
      } else if (h[3] == 1 || h[3] == 0) {
        auto it = want.find(s);
        if (it == want.end()) {
          expect(false, "reply on an unknown stream");
          continue;
        }
        Reply& r = it->second;
        if (h[3] == 0) {
          r.data += p;
        } else {
          ++r.headers;
          // The trailers carry grpc-status as a literal with a new name.
          if (p.find(std::string("\x0bgrpc-status\x01" "0", 14)) != std::string::npos)
            r.ok_status = true;
        }
        if (h[4] & 1) {
          r.ended = true;
          ++ended;
        }
      }
    }
    for (auto& kv : want) {
      const bool health = ((kv.first - 1) / 2) % 2 == 0;
      const std::string body =
          health ? std::string("\x0a\x02\x08\x01", 4)
                 : std::string(reinterpret_cast<const char*>(kQueryReply), sizeof(kQueryReply));
      std::string framed(1, '\0');
      for (int sh = 24; sh >= 0; sh -= 8)
        framed.push_back(static_cast<char>((body.size() >> sh) & 0xff));
      framed += body;
      expect(kv.second.ok_status, "grpc-status 0 on stream " + std::to_string(kv.first));
      expect(kv.second.headers == 2, "headers then trailers on stream " + std::to_string(kv.first));
      expect(kv.second.data == framed, "message on stream " + std::to_string(kv.first));
    }
  }
  // Left open: the server's stop closes it.
  clients_done.fetch_add(1);
  char b;
  (void)::recv(fd, &b, 1, 0);
  ::close(fd);
}

}  // namespace

int main() {
  pf_engine* e = nullptr;
  if (pf_engine_create(64ull << 20, 1, PF_PINNED_DEFAULT, 0, &e) != PF_OK) {
    std::printf("FAILED: engine: %s\n", pf_last_error());
    return 1;
  }
  pf_grpc_server* srv = nullptr;
  if (pf_grpc_start(e, "127.0.0.1:0", handler, nullptr, &srv) != PF_OK) {
    std::printf("FAILED: start: %s\n", pf_last_error());
    return 1;
  }
  const int port = pf_grpc_port(srv);
  std::vector<std::thread> ts;
  for (int i = 0; i < 4; ++i) ts.emplace_back(client, port, i);
  // Stop once every client has its replies (they then wait on their sockets).
  const auto t0 = std::chrono::steady_clock::now();
  while (clients_done.load() < 4 && failures.load() == 0 &&
         std::chrono::steady_clock::now() - t0 < std::chrono::seconds(120))
    std::this_thread::sleep_for(std::chrono::milliseconds(5));
  expect(clients_done.load() == 4, "clients finished within 120 s");
  expect(pf_grpc_served(srv) == 4u * 50u * 4u, "requests served");
  pf_grpc_stop(srv);
  for (std::thread& t : ts) t.join();
  pf_engine_destroy(e);
  expect(handled.load() == 4 * 50 * 2, "handler calls: " + std::to_string(handled.load()));
  if (failures.load()) return 1;
  std::printf("ok\n");
  return 0;
}
