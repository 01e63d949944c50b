// pf_grpc.cpp — the Engine gRPC service (engine.proto) served natively, over
// HTTP/2 without TLS (h2c with prior knowledge, as an insecure gRPC channel
// connects).  The reference serves it from Rust (tonic, service.rs:133-405);
// a Python gRPC server took about 0.27 ms from a client's request to its
// handler, against 0.07 ms for the request to be on the server's socket.
//
// Load and Health are served on the connection's own thread, Save on a
// worker thread (it holds its caller for the whole copy), each through the
// engine's own decoder of the request bytes (pf_engine_serve_request).  The
// other RPCs (registration, queries, unregistration, shutdown) go to a
// handler supplied by the caller, on a worker thread.
//
// HTTP/2 (RFC 9113) as a gRPC server needs it: the connection preface and
// SETTINGS, header blocks in HEADERS + CONTINUATION frames (HPACK,
// pf_hpack.cpp), request bodies in DATA frames, PING replies, WINDOW_UPDATE
// in both directions, RST_STREAM and GOAWAY.  Replies are response headers,
// one DATA frame with the length-prefixed message and trailers carrying
// grpc-status, or trailers only for an error (the gRPC HTTP/2 protocol).
#include <arpa/inet.h>
#include <fcntl.h>
#include <netdb.h>
#include <netinet/in.h>
#include <netinet/tcp.h>
#include <poll.h>
#include <sys/socket.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "pf_common.h"
#include "pf_h2.h"
#include "pf_hpack.h"

using namespace pf;
using namespace pf::h2;

namespace {

// gRPC status codes (grpc/status.h).
enum : uint32_t {
  kOk = 0, kInvalidArgument = 3, kResourceExhausted = 8, kFailedPrecondition = 9,
  kUnimplemented = 12, kInternal = 13
};

constexpr uint32_t kMaxFrame = (1u << 24) - 1;  // SETTINGS_MAX_FRAME_SIZE we advertise
constexpr int64_t kMaxWindow = 0x7fffffff;       // our windows: as large as allowed
constexpr size_t kMaxHeaderBlock = 1 << 20;
constexpr uint32_t kMaxStreams = 1024;
// Request bytes one connection may hold at once, over all its streams (two
// of the largest requests); a stream that would pass it is answered
// RESOURCE_EXHAUSTED, as a single oversized request is.
constexpr uint64_t kMaxConnBuffered = 2ull * PF_REQUEST_MAX_BYTES + 10;
constexpr uint64_t kWindowRefill = 64ull << 20;  // connection window given back per
constexpr size_t kWorkers = 8;

const std::string kServicePrefix = "/pegaflow.Engine/";
// LoadResponse / SaveResponse / HealthResponse { status: ResponseStatus { ok: true } }.
const uint8_t kOkResponse[] = {0x0a, 0x02, 0x08, 0x01};

// service.rs:77-88.
uint32_t grpc_code(int rc) {
  switch (rc) {
    case PF_OK: return kOk;
    case PF_ERR_INVALID_ARGUMENT: return kInvalidArgument;
    case PF_ERR_INSTANCE_MISSING:
    case PF_ERR_WORKER_MISSING:
    case PF_ERR_TOPOLOGY_MISMATCH: return kFailedPrecondition;
    default: return kInternal;
  }
}

class Workers {
 public:
  explicit Workers(size_t n) {
    for (size_t i = 0; i < n; ++i) threads_.emplace_back([this] { loop(); });
  }
  ~Workers() { shutdown(); }
  void post(std::function<void()> job) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      jobs_.push_back(std::move(job));
    }
    cv_.notify_one();
  }
  // Runs the jobs already posted, then ends the threads.
  void shutdown() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (std::thread& t : threads_)
      if (t.joinable()) t.join();
    threads_.clear();
  }

 private:
  void loop() {
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      cv_.wait(lk, [this] { return stop_ || !jobs_.empty(); });
      if (jobs_.empty()) return;
      std::function<void()> job = std::move(jobs_.front());
      jobs_.pop_front();
      lk.unlock();
      job();
      lk.lock();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<std::function<void()>> jobs_;
  bool stop_ = false;
  std::vector<std::thread> threads_;
};

struct Server;

class Conn : public std::enable_shared_from_this<Conn> {
 public:
  Conn(Server* s, int fd) : srv_(s), fd_(fd) {}
  ~Conn() { ::close(fd_); }
  void start() {
    auto self = shared_from_this();
    thread_ = std::thread([self] { self->run(); });
  }
  void shutdown_socket() { (void)::shutdown(fd_, SHUT_RDWR); }
  void join() {
    if (thread_.joinable()) thread_.join();
  }
  bool done() const { return done_.load(); }
  // Sends the reply of stream sid (dropped if the peer reset the stream or
  // the connection is gone).  A message waits for the peer's flow-control
  // windows to allow it, unless may_wait is false (the connection's own
  // thread, which reads the window updates): then false, nothing sent.
  bool reply(uint32_t sid, uint32_t status, const std::string& message, const uint8_t* body,
             size_t n, bool may_wait = true);
  bool reply_rc(uint32_t sid, int rc, const std::string& message, bool may_wait = true) {
    if (rc == PF_OK) return reply(sid, kOk, "", kOkResponse, sizeof(kOkResponse), may_wait);
    return reply(sid, grpc_code(rc), message, nullptr, 0, may_wait);
  }

 private:
  struct Stream {
    std::string block;    // header block being assembled
    std::string path, content_type, encoding;
    std::string data;     // request body (length-prefixed messages)
    bool headers_done = false, end_after_block = false, rejected = false;
    std::chrono::steady_clock::time_point opened;  // its first HEADERS frame
  };
  void run();
  bool handle(uint8_t type, uint8_t flags, uint32_t sid, std::string& payload);
  bool headers_complete(uint32_t sid, Stream& st);
  void complete(uint32_t sid, Stream&& st);
  bool read_exact(void* p, size_t n);
  bool send_locked(const std::string& bytes);
  void send(const std::string& bytes) {
    std::lock_guard<std::mutex> lk(wmu_);
    (void)send_locked(bytes);
  }
  void goaway(uint32_t code) {
    std::string out, p;
    put32(&p, last_sid_);
    put32(&p, code);
    frame(&out, kGoaway, 0, 0, p.data(), p.size());
    send(out);
  }
  void rst(uint32_t sid, uint32_t code) {
    std::string out, p;
    put32(&p, code);
    frame(&out, kRstStream, 0, sid, p.data(), p.size());
    send(out);
  }

  Server* srv_;
  int fd_;
  std::thread thread_;
  std::atomic<bool> done_{false};
  // Writers (the reader, workers) under wmu_; send windows and the streams
  // awaiting a reply with theirs.
  std::mutex wmu_;
  std::condition_variable wcv_;
  bool closed_ = false;
  int64_t conn_window_ = 65535, peer_initial_ = 65535;
  uint32_t peer_max_frame_ = 16384;
  std::unordered_map<uint32_t, int64_t> live_;
  // Reader only.
  HpackDecoder hpack_;
  std::unordered_map<uint32_t, Stream> streams_;
  uint32_t last_sid_ = 0, continuation_of_ = 0;
  uint64_t consumed_ = 0;
  uint64_t buffered_ = 0;  // bytes of request bodies held in streams_
  // Drops a stream's body from the count (before the stream is erased or
  // its body handed on).
  void unbuffer(Stream& st) { buffered_ -= st.data.size(); }
};

}  // namespace

struct pf_grpc_call {
  std::shared_ptr<Conn> conn;
  uint32_t sid = 0;
  bool replied = false;
};

namespace {

struct Server {
  pf_engine* engine = nullptr;
  pf_grpc_handler fallback = nullptr;
  void* ctx = nullptr;
  int listen_fd = -1, wake[2] = {-1, -1};
  int port = 0;
  std::thread acceptor;
  std::unique_ptr<Workers> workers;
  std::mutex mu;
  std::vector<std::shared_ptr<Conn>> conns;
  std::atomic<uint64_t> served{0};

  void accept_loop();
  // `data`: the request's one length-prefixed message (5 bytes of prefix).
  void dispatch(const std::shared_ptr<Conn>& c, uint32_t sid, const std::string& path,
                std::string&& data, std::chrono::steady_clock::time_point opened);
};

// With PEGAFLOW_TRACE set: when a request's stream opened, its body was
// complete, its handling began, and its reply was sent (monotonic us).
void trace_request(const std::string& method, size_t bytes,
                   std::chrono::steady_clock::time_point opened,
                   std::chrono::steady_clock::time_point received,
                   std::chrono::steady_clock::time_point started) {
  std::fprintf(stderr,
               "[pegaflow] grpc request method=%s bytes=%zu opened=%.0fus received=%.0fus "
               "started=%.0fus replied=%.0fus\n",
               method.c_str(), bytes, mono_us(opened), mono_us(received), mono_us(started),
               mono_us(std::chrono::steady_clock::now()));
}

bool Conn::read_exact(void* p, size_t n) {
  char* q = static_cast<char*>(p);
  while (n > 0) {
    const ssize_t r = ::recv(fd_, q, n, 0);
    if (r > 0) {
      q += r;
      n -= static_cast<size_t>(r);
    } else if (r < 0 && errno == EINTR) {
      continue;
    } else {
      return false;
    }
  }
  return true;
}

bool Conn::send_locked(const std::string& bytes) {
  if (closed_) return false;
  size_t off = 0;
  while (off < bytes.size()) {
    const ssize_t r = ::send(fd_, bytes.data() + off, bytes.size() - off, MSG_NOSIGNAL);
    if (r > 0) {
      off += static_cast<size_t>(r);
    } else if (r < 0 && errno == EINTR) {
      continue;
    } else {
      closed_ = true;
      wcv_.notify_all();
      return false;
    }
  }
  return true;
}

bool Conn::reply(uint32_t sid, uint32_t status, const std::string& message, const uint8_t* body,
                 size_t n, bool may_wait) {
  std::string headers;
  headers.push_back(static_cast<char>(0x88));  // :status: 200 (static index 8)
  hp_field(&headers, 31, "application/grpc");  // content-type
  std::string trailers;
  hp_field(&trailers, "grpc-status", std::to_string(status));
  if (!message.empty()) hp_field(&trailers, "grpc-message", percent_encode(message));
  std::string out;
  std::unique_lock<std::mutex> lk(wmu_);
  if (status != kOk) {  // trailers only
    if (live_.erase(sid) == 0) return true;
    frame(&out, kHeaders, kEndHeaders | kEndStream, sid, (headers + trailers).data(),
          headers.size() + trailers.size());
    (void)send_locked(out);
    return true;
  }
  std::string msg;
  msg.push_back(0);  // not compressed
  put32(&msg, static_cast<uint32_t>(n));
  msg.append(reinterpret_cast<const char*>(body), n);
  const int64_t need = static_cast<int64_t>(msg.size());
  // The message goes out whole once both send windows allow it.
  for (;;) {
    auto it = live_.find(sid);
    if (closed_ || it == live_.end()) return true;
    if (conn_window_ >= need && it->second >= need) break;
    if (!may_wait) return false;
    wcv_.wait(lk);
  }
  live_.erase(sid);
  conn_window_ -= need;
  frame(&out, kHeaders, kEndHeaders, sid, headers.data(), headers.size());
  for (size_t off = 0; off < msg.size(); off += peer_max_frame_) {
    const size_t len = std::min<size_t>(peer_max_frame_, msg.size() - off);
    frame(&out, kData, 0, sid, msg.data() + off, len);
  }
  frame(&out, kHeaders, kEndHeaders | kEndStream, sid, trailers.data(), trailers.size());
  (void)send_locked(out);
  return true;
}

void Conn::run() {
  char pre[kPrefaceLen];
  if (read_exact(pre, sizeof(pre)) && std::memcmp(pre, kPreface, sizeof(pre)) == 0) {
    std::string out, s;
    const uint16_t ids[3] = {0x3, 0x4, 0x5};  // max streams, initial window, max frame
    const uint32_t vals[3] = {kMaxStreams, static_cast<uint32_t>(kMaxWindow), kMaxFrame};
    for (int i = 0; i < 3; ++i) {
      s.push_back(static_cast<char>(ids[i] >> 8));
      s.push_back(static_cast<char>(ids[i] & 0xff));
      put32(&s, vals[i]);
    }
    frame(&out, kSettings, 0, 0, s.data(), s.size());
    std::string inc;
    put32(&inc, static_cast<uint32_t>(kMaxWindow - 65535));
    frame(&out, kWindowUpdate, 0, 0, inc.data(), inc.size());
    send(out);
    std::string payload;
    for (;;) {
      uint8_t h[9];
      if (!read_exact(h, sizeof(h))) break;
      const uint32_t len = (uint32_t(h[0]) << 16) | (uint32_t(h[1]) << 8) | h[2];
      const uint32_t sid =
          ((uint32_t(h[5]) & 0x7f) << 24) | (uint32_t(h[6]) << 16) | (uint32_t(h[7]) << 8) | h[8];
      if (len > kMaxFrame) {
        goaway(kFrameSizeError);
        break;
      }
      payload.resize(len);
      if (len && !read_exact(&payload[0], len)) break;
      if (continuation_of_ && (h[3] != kContinuation || sid != continuation_of_)) {
        goaway(kProtocolError);
        break;
      }
      if (!handle(h[3], h[4], sid, payload)) break;
    }
  }
  {
    std::lock_guard<std::mutex> lk(wmu_);
    closed_ = true;
    live_.clear();
  }
  wcv_.notify_all();
  shutdown_socket();
  done_.store(true);
}

bool Conn::handle(uint8_t type, uint8_t flags, uint32_t sid, std::string& payload) {
  switch (type) {
    case kData: {
      if (sid == 0) {
        goaway(kProtocolError);
        return false;
      }
      // Flow control counts the whole frame; the connection window is given
      // back in large steps (each stream's is larger than any request).
      consumed_ += payload.size();
      if (consumed_ >= kWindowRefill) {
        std::string out, inc;
        put32(&inc, static_cast<uint32_t>(consumed_));
        frame(&out, kWindowUpdate, 0, 0, inc.data(), inc.size());
        send(out);
        consumed_ = 0;
      }
      size_t off = 0, n = payload.size();
      if (flags & kPadded) {
        if (n < 1 || uint8_t(payload[0]) >= n) {
          goaway(kProtocolError);
          return false;
        }
        off = 1;
        n -= 1 + uint8_t(payload[0]);
      }
      auto it = streams_.find(sid);
      if (it == streams_.end() || !it->second.headers_done) return true;  // reset or unknown
      Stream& st = it->second;
      if (!st.rejected) {
        if (st.data.size() + n > PF_REQUEST_MAX_BYTES + 5ull ||
            buffered_ + n > kMaxConnBuffered) {
          unbuffer(st);
          st.rejected = true;
          st.data.clear();
          st.data.shrink_to_fit();
        } else {
          st.data.append(payload, off, n);
          buffered_ += n;
        }
      }
      if (flags & kEndStream) {
        unbuffer(st);
        Stream done = std::move(st);
        streams_.erase(it);
        complete(sid, std::move(done));
      }
      return true;
    }
    case kHeaders: {
      if (sid == 0 || !(sid & 1)) {
        goaway(kProtocolError);
        return false;
      }
      size_t off = 0, n = payload.size();
      if (flags & kPadded) {
        if (n < 1 || uint8_t(payload[0]) >= n) {
          goaway(kProtocolError);
          return false;
        }
        off = 1;
        n -= 1 + uint8_t(payload[0]);
      }
      if (flags & kPriorityFlag) {
        if (n < 5) {
          goaway(kProtocolError);
          return false;
        }
        off += 5;
        n -= 5;
      }
      auto it = streams_.find(sid);
      if (it == streams_.end()) {
        if (sid <= last_sid_) {  // a stream already closed
          goaway(kProtocolError);
          return false;
        }
        last_sid_ = sid;
        it = streams_.emplace(sid, Stream()).first;
        if (tracing()) it->second.opened = std::chrono::steady_clock::now();
      }
      // A second block on a stream is the client's trailers: decoded (the
      // table must stay in step) and otherwise ignored.
      Stream& st = it->second;
      st.block.append(payload, off, n);
      if (st.block.size() > kMaxHeaderBlock) {
        goaway(kProtocolError);
        return false;
      }
      st.end_after_block = (flags & kEndStream) != 0;
      if (!(flags & kEndHeaders)) {
        continuation_of_ = sid;
        return true;
      }
      return headers_complete(sid, st);
    }
    case kContinuation: {
      auto it = streams_.find(sid);
      if (it == streams_.end() || continuation_of_ != sid) {
        goaway(kProtocolError);
        return false;
      }
      it->second.block.append(payload);
      if (it->second.block.size() > kMaxHeaderBlock) {
        goaway(kProtocolError);
        return false;
      }
      if (!(flags & kEndHeaders)) return true;
      continuation_of_ = 0;
      return headers_complete(sid, it->second);
    }
    case kSettings: {
      if (sid != 0 || ((flags & kAck) ? payload.size() != 0 : payload.size() % 6 != 0)) {
        goaway(kProtocolError);
        return false;
      }
      if (flags & kAck) return true;
      bool bad = false;
      {
        std::lock_guard<std::mutex> lk(wmu_);
        for (size_t i = 0; i + 6 <= payload.size() && !bad; i += 6) {
          const uint16_t id = (uint16_t(uint8_t(payload[i])) << 8) | uint8_t(payload[i + 1]);
          const uint32_t v = (uint32_t(uint8_t(payload[i + 2])) << 24) |
                             (uint32_t(uint8_t(payload[i + 3])) << 16) |
                             (uint32_t(uint8_t(payload[i + 4])) << 8) | uint8_t(payload[i + 5]);
          if (id == 0x4) {  // SETTINGS_INITIAL_WINDOW_SIZE: applies to open streams too
            if (v > uint32_t(kMaxWindow)) {
              bad = true;
              break;
            }
            const int64_t delta = int64_t(v) - peer_initial_;
            for (auto& kv : live_) kv.second += delta;
            peer_initial_ = v;
          } else if (id == 0x5 && v >= 16384 && v <= kMaxFrame) {
            peer_max_frame_ = v;
          }
        }
        wcv_.notify_all();
        if (!bad) {
          std::string out;
          frame(&out, kSettings, kAck, 0, nullptr, 0);
          (void)send_locked(out);
        }
      }
      if (bad) {
        goaway(kFlowControlError);
        return false;
      }
      return true;
    }
    case kPing: {
      if (sid != 0 || payload.size() != 8) {
        goaway(kProtocolError);
        return false;
      }
      if (!(flags & kAck)) {
        std::string out;
        frame(&out, kPing, kAck, 0, payload.data(), payload.size());
        send(out);
      }
      return true;
    }
    case kWindowUpdate: {
      if (payload.size() != 4) {
        goaway(kFrameSizeError);
        return false;
      }
      const int64_t inc = ((uint32_t(uint8_t(payload[0])) & 0x7f) << 24) |
                          (uint32_t(uint8_t(payload[1])) << 16) |
                          (uint32_t(uint8_t(payload[2])) << 8) | uint8_t(payload[3]);
      bool bad_window = false;
      // RFC 9113 6.9: an increment of 0, or one that takes a window past
      // 2^31-1, is an error (of the connection, or of the stream).
      if (sid == 0) {
        std::lock_guard<std::mutex> lk(wmu_);
        if (inc == 0 || conn_window_ + inc > kMaxWindow) {
          bad_window = true;
        } else {
          conn_window_ += inc;
          wcv_.notify_all();
        }
      } else {
        bool reset = false;
        {
          std::lock_guard<std::mutex> lk(wmu_);
          auto it = live_.find(sid);
          if (it != live_.end()) {
            if (inc == 0 || it->second + inc > kMaxWindow) {
              live_.erase(it);
              std::string out, p;
              put32(&p, inc == 0 ? kProtocolError : kFlowControlError);
              frame(&out, kRstStream, 0, sid, p.data(), p.size());
              (void)send_locked(out);
              reset = true;
            } else {
              it->second += inc;
            }
          }
          wcv_.notify_all();
        }
        if (reset) {
          auto st = streams_.find(sid);
          if (st != streams_.end()) {
            unbuffer(st->second);
            streams_.erase(st);
          }
        }
      }
      if (bad_window) {
        goaway(inc == 0 ? kProtocolError : kFlowControlError);
        return false;
      }
      return true;
    }
    case kRstStream: {
      if (auto st = streams_.find(sid); st != streams_.end()) {
        unbuffer(st->second);
        streams_.erase(st);
      }
      std::lock_guard<std::mutex> lk(wmu_);
      live_.erase(sid);
      wcv_.notify_all();
      return true;
    }
    case kGoaway:
      return false;
    case kPushPromise:
      goaway(kProtocolError);
      return false;
    default:  // PRIORITY and unknown frame types are ignored
      return true;
  }
}

bool Conn::headers_complete(uint32_t sid, Stream& st) {
  std::vector<HeaderField> fields;
  std::string err;
  if (!hpack_.decode(reinterpret_cast<const uint8_t*>(st.block.data()), st.block.size(),
                     &fields, &err)) {
    goaway(kCompressionError);
    return false;
  }
  st.block.clear();
  if (st.headers_done) {  // trailers
    if (st.end_after_block) {
      unbuffer(st);
      Stream done = std::move(st);
      streams_.erase(sid);
      complete(sid, std::move(done));
    }
    return true;
  }
  st.headers_done = true;
  for (const HeaderField& f : fields) {
    if (f.name == ":path") st.path = f.value;
    else if (f.name == "content-type") st.content_type = f.value;
    else if (f.name == "grpc-encoding") st.encoding = f.value;
  }
  {
    std::lock_guard<std::mutex> lk(wmu_);
    if (live_.size() >= kMaxStreams) {
      streams_.erase(sid);
      std::string out, p;
      put32(&p, kRefusedStream);
      frame(&out, kRstStream, 0, sid, p.data(), p.size());
      (void)send_locked(out);
      return true;
    }
    live_[sid] = peer_initial_;
  }
  if (st.end_after_block) {
    Stream done = std::move(st);
    streams_.erase(sid);
    complete(sid, std::move(done));
  }
  return true;
}

void Conn::complete(uint32_t sid, Stream&& st) {
  if (st.rejected) {
    reply(sid, kResourceExhausted,
          strf("Received message larger than max (limit %u bytes)", PF_REQUEST_MAX_BYTES), nullptr,
          0);
    return;
  }
  if (st.content_type.compare(0, 16, "application/grpc") != 0) {
    reply(sid, kInternal, "content-type is not application/grpc: " + st.content_type, nullptr,
          0);
    return;
  }
  if (!st.encoding.empty() && st.encoding != "identity") {
    reply(sid, kUnimplemented, "message encoding " + st.encoding + " is not supported", nullptr,
          0);
    return;
  }
  const std::string& d = st.data;
  if (d.size() < 5 || d[0] != 0 ||
      ((uint64_t(uint8_t(d[1])) << 24) | (uint64_t(uint8_t(d[2])) << 16) |
       (uint64_t(uint8_t(d[3])) << 8) | uint8_t(d[4])) + 5 != d.size()) {
    reply(sid, d.size() >= 5 && d[0] != 0 ? kUnimplemented : kInternal,
          d.size() >= 5 && d[0] != 0 ? "compressed messages are not supported"
                                     : "a unary request must carry one message",
          nullptr, 0);
    return;
  }
  srv_->dispatch(shared_from_this(), sid, st.path, std::move(st.data), st.opened);
}

void Server::dispatch(const std::shared_ptr<Conn>& c, uint32_t sid, const std::string& path,
                      std::string&& data, std::chrono::steady_clock::time_point opened) {
  served.fetch_add(1);
  const bool trace = tracing();
  const auto received = trace ? std::chrono::steady_clock::now() : opened;
  if (path.compare(0, kServicePrefix.size(), kServicePrefix) != 0) {
    c->reply(sid, kUnimplemented, "Method not found!", nullptr, 0);
    return;
  }
  const std::string method = path.substr(kServicePrefix.size());
  const auto* req = reinterpret_cast<const uint8_t*>(data.data()) + 5;
  const size_t size = data.size() - 5;
  if (method == "Load" || method == "Health") {
    const int rc = method == "Load" ? pf_engine_serve_request(engine, PF_REQUEST_LOAD, req, size)
                                    : PF_OK;
    std::string msg = rc == PF_OK ? std::string() : std::string(pf_last_error());
    // On the connection's thread the reply may not wait for window updates
    // (that thread reads them); a worker sends it if the windows are short.
    if (!c->reply_rc(sid, rc, msg, false))
      workers->post([c, sid, rc, msg] { c->reply_rc(sid, rc, msg); });
    if (trace) trace_request(method, size, opened, received, received);
    return;
  }
  auto job = std::make_shared<std::string>(std::move(data));
  if (method == "Save") {
    workers->post([this, c, sid, job, trace, opened, received] {
      const auto started = std::chrono::steady_clock::now();
      const int rc = pf_engine_serve_request(
          engine, PF_REQUEST_SAVE, reinterpret_cast<const uint8_t*>(job->data()) + 5,
          job->size() - 5);
      c->reply_rc(sid, rc, rc == PF_OK ? std::string() : std::string(pf_last_error()));
      if (trace) trace_request("Save", job->size() - 5, opened, received, started);
    });
    return;
  }
  if (!fallback) {
    c->reply(sid, kUnimplemented, "Method not found!", nullptr, 0);
    return;
  }
  workers->post([this, c, sid, job, method] {
    pf_grpc_call call;
    call.conn = c;
    call.sid = sid;
    fallback(ctx, &call, method.c_str(), reinterpret_cast<const uint8_t*>(job->data()) + 5,
             job->size() - 5);
    if (!call.replied) c->reply(sid, kInternal, "the handler sent no reply", nullptr, 0);
  });
}

void Server::accept_loop() {
  for (;;) {
    pollfd fds[2] = {{listen_fd, POLLIN, 0}, {wake[0], POLLIN, 0}};
    const int r = ::poll(fds, 2, -1);
    if (r < 0 && errno == EINTR) continue;
    if (r < 0 || (fds[1].revents & POLLIN)) return;
    if (!(fds[0].revents & POLLIN)) continue;
    const int fd = ::accept4(listen_fd, nullptr, nullptr, SOCK_CLOEXEC);
    if (fd < 0) continue;
    const int one = 1;
    (void)::setsockopt(fd, IPPROTO_TCP, TCP_NODELAY, &one, sizeof(one));
    auto c = std::make_shared<Conn>(this, fd);
    std::lock_guard<std::mutex> lk(mu);
    for (size_t i = 0; i < conns.size();) {  // connections that ended
      if (conns[i]->done()) {
        conns[i]->join();
        conns[i] = conns.back();
        conns.pop_back();
      } else {
        ++i;
      }
    }
    conns.push_back(c);
    c->start();
  }
}

// "host:port" (an IPv6 host in brackets); a listening socket on it.
int listen_on(const char* address, int* fd_out, int* port_out) {
  std::string a = address ? address : "";
  const size_t colon = a.rfind(':');
  if (colon == std::string::npos)
    return fail(PF_ERR_INVALID_ARGUMENT, "gRPC address must be host:port: " + a);
  std::string host = a.substr(0, colon), port = a.substr(colon + 1);
  if (host.size() >= 2 && host.front() == '[' && host.back() == ']')
    host = host.substr(1, host.size() - 2);
  addrinfo hints{};
  hints.ai_family = AF_UNSPEC;
  hints.ai_socktype = SOCK_STREAM;
  hints.ai_flags = AI_PASSIVE;
  addrinfo* res = nullptr;
  if (int e = ::getaddrinfo(host.empty() ? nullptr : host.c_str(), port.c_str(), &hints, &res))
    return fail(PF_ERR_INVALID_ARGUMENT, "cannot resolve " + a + ": " + gai_strerror(e));
  int fd = -1;
  std::string why = "no address";
  for (addrinfo* ai = res; ai && fd < 0; ai = ai->ai_next) {
    fd = ::socket(ai->ai_family, ai->ai_socktype | SOCK_CLOEXEC, ai->ai_protocol);
    if (fd < 0) continue;
    const int one = 1;
    (void)::setsockopt(fd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof(one));
    if (::bind(fd, ai->ai_addr, ai->ai_addrlen) != 0 || ::listen(fd, 128) != 0) {
      why = std::strerror(errno);
      ::close(fd);
      fd = -1;
    }
  }
  ::freeaddrinfo(res);
  if (fd < 0) return fail(PF_ERR_STORAGE, "failed to bind " + a + ": " + why);
  sockaddr_storage ss{};
  socklen_t sl = sizeof(ss);
  (void)::getsockname(fd, reinterpret_cast<sockaddr*>(&ss), &sl);
  *port_out = ss.ss_family == AF_INET6
                  ? ntohs(reinterpret_cast<sockaddr_in6*>(&ss)->sin6_port)
                  : ntohs(reinterpret_cast<sockaddr_in*>(&ss)->sin_port);
  *fd_out = fd;
  return PF_OK;
}

}  // namespace

struct pf_grpc_server {
  Server s;
};

extern "C" {

int pf_grpc_start(pf_engine* engine, const char* address, pf_grpc_handler fallback, void* ctx,
                  pf_grpc_server** out) {
  clear_error();
  if (!engine || !out) return fail(PF_ERR_INVALID_ARGUMENT, "null engine or out pointer");
  *out = nullptr;
  std::unique_ptr<pf_grpc_server> g(new pf_grpc_server());
  Server& s = g->s;
  s.engine = engine;
  s.fallback = fallback;
  s.ctx = ctx;
  if (int rc = listen_on(address, &s.listen_fd, &s.port)) return rc;
  if (::pipe2(s.wake, O_CLOEXEC) != 0) {
    ::close(s.listen_fd);
    return fail(PF_ERR_STORAGE, std::string("pipe failed: ") + std::strerror(errno));
  }
  s.workers.reset(new Workers(kWorkers));
  s.acceptor = std::thread([p = &s] { p->accept_loop(); });
  *out = g.release();
  return PF_OK;
}

int pf_grpc_port(const pf_grpc_server* g) { return g ? g->s.port : 0; }

uint64_t pf_grpc_served(const pf_grpc_server* g) { return g ? g->s.served.load() : 0; }

int pf_grpc_reply(pf_grpc_call* call, uint32_t status, const char* message,
                  const uint8_t* response, uint64_t size) {
  if (!call) return fail(PF_ERR_INVALID_ARGUMENT, "null call");
  if (call->replied) return fail(PF_ERR_INVALID_ARGUMENT, "call already answered");
  if (size > 0 && !response) return fail(PF_ERR_INVALID_ARGUMENT, "null response bytes");
  call->replied = true;
  call->conn->reply(call->sid, status, message ? message : "", response,
                    static_cast<size_t>(size));
  return PF_OK;
}

int pf_grpc_stop(pf_grpc_server* g) {
  if (!g) return PF_OK;
  Server& s = g->s;
  const char b = 1;
  (void)!::write(s.wake[1], &b, 1);
  if (s.acceptor.joinable()) s.acceptor.join();
  ::close(s.listen_fd);
  std::vector<std::shared_ptr<Conn>> conns;
  {
    std::lock_guard<std::mutex> lk(s.mu);
    conns.swap(s.conns);
  }
  for (auto& c : conns) c->shutdown_socket();
  for (auto& c : conns) c->join();
  s.workers->shutdown();
  ::close(s.wake[0]);
  ::close(s.wake[1]);
  delete g;
  return PF_OK;
}

}  // extern "C"
