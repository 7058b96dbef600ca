#include "http.h"

#include <arpa/inet.h>
#include <netdb.h>
#include <netinet/in.h>
#include <sys/socket.h>
#include <sys/time.h>
#include <unistd.h>

#include <chrono>
#include <thread>
#include <cctype>
#include <cerrno>
#include <cstring>
#include <stdexcept>

namespace malkin_hip::http {

namespace {

constexpr size_t kMaxHeader = 64 << 10;
constexpr size_t kMaxBody = 64 << 20;
constexpr int kTimeoutS = 600;

const char* reason(int status) {
  switch (status) {
    case 200: return "OK";
    case 400: return "Bad Request";
    case 404: return "Not Found";
    case 405: return "Method Not Allowed";
    case 413: return "Payload Too Large";
    case 500: return "Internal Server Error";
    case 503: return "Service Unavailable";
    default: return "Status";
  }
}

std::string lower(std::string s) {
  for (char& c : s) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
  return s;
}

std::string trim(const std::string& s) {
  size_t a = 0, b = s.size();
  while (a < b && (s[a] == ' ' || s[a] == '\t')) ++a;
  while (b > a && (s[b - 1] == ' ' || s[b - 1] == '\t' || s[b - 1] == '\r')) --b;
  return s.substr(a, b - a);
}

// Reads the request head and body. Returns 0, or an HTTP status for a malformed / oversized request.
int read_request(int fd, Request& rq) {
  std::string buf;
  char tmp[8192];
  size_t head_end = std::string::npos;
  while (head_end == std::string::npos) {
    const ssize_t r = ::recv(fd, tmp, sizeof tmp, 0);
    if (r <= 0) return -1;
    buf.append(tmp, static_cast<size_t>(r));
    head_end = buf.find("\r\n\r\n");
    if (head_end == std::string::npos && buf.size() > kMaxHeader) return 413;
  }
  const std::string head = buf.substr(0, head_end);
  std::string rest = buf.substr(head_end + 4);
  size_t eol = head.find("\r\n");
  const std::string line = head.substr(0, eol);
  const size_t sp1 = line.find(' '), sp2 = line.rfind(' ');
  if (sp1 == std::string::npos || sp2 == sp1) return 400;
  rq.method = line.substr(0, sp1);
  rq.path = line.substr(sp1 + 1, sp2 - sp1 - 1);
  if (const size_t q = rq.path.find('?'); q != std::string::npos) rq.path.resize(q);
  while (eol != std::string::npos) {
    const size_t next = head.find("\r\n", eol + 2);
    const std::string h = head.substr(eol + 2, next == std::string::npos ? std::string::npos : next - eol - 2);
    eol = next;
    const size_t colon = h.find(':');
    if (colon == std::string::npos) continue;
    rq.headers[lower(trim(h.substr(0, colon)))] = trim(h.substr(colon + 1));
  }
  if (rq.headers.count("transfer-encoding")) return 400;  // chunked request bodies are not accepted
  size_t len = 0;
  if (auto it = rq.headers.find("content-length"); it != rq.headers.end()) {
    char* end = nullptr;
    errno = 0;
    const unsigned long long v = std::strtoull(it->second.c_str(), &end, 10);
    if (errno != 0 || end == it->second.c_str() || *end != '\0') return 400;
    if (v > kMaxBody) return 413;
    len = static_cast<size_t>(v);
  }
  while (rest.size() < len) {
    const ssize_t r = ::recv(fd, tmp, sizeof tmp, 0);
    if (r <= 0) return -1;
    rest.append(tmp, static_cast<size_t>(r));
  }
  rest.resize(len);
  rq.body = std::move(rest);
  return 0;
}

}  // namespace

bool Writer::write_all(const std::string& s) {
  size_t off = 0;
  while (ok_ && off < s.size()) {
    const ssize_t w = ::send(fd_, s.data() + off, s.size() - off, MSG_NOSIGNAL);
    if (w <= 0) {
      if (w < 0 && errno == EINTR) continue;
      ok_ = false;
      break;
    }
    off += static_cast<size_t>(w);
  }
  return ok_;
}

bool Writer::send(int status, const std::string& content_type, const std::string& body) {
  std::string h = "HTTP/1.1 " + std::to_string(status) + " " + reason(status) + "\r\nContent-Type: " + content_type +
                  "\r\nContent-Length: " + std::to_string(body.size()) + "\r\nConnection: close\r\n\r\n";
  return write_all(h) && write_all(body);
}

bool Writer::begin_stream(const std::string& content_type) {
  return write_all("HTTP/1.1 200 OK\r\nContent-Type: " + content_type +
                   "\r\nCache-Control: no-cache\r\nTransfer-Encoding: chunked\r\nConnection: close\r\n\r\n");
}

bool Writer::chunk(const std::string& data) {
  if (data.empty()) return ok_;
  char len[32];
  std::snprintf(len, sizeof len, "%zx\r\n", data.size());
  return write_all(len) && write_all(data) && write_all("\r\n");
}

bool Writer::end_stream() { return write_all("0\r\n\r\n"); }

Server::~Server() { stop(); }

int Server::bind(const std::string& host, int port) {
  addrinfo hints{}, *res = nullptr;
  hints.ai_family = AF_UNSPEC;
  hints.ai_socktype = SOCK_STREAM;
  hints.ai_flags = AI_PASSIVE | AI_NUMERICSERV;
  const std::string svc = std::to_string(port);
  if (const int rc = ::getaddrinfo(host.empty() ? nullptr : host.c_str(), svc.c_str(), &hints, &res); rc != 0)
    throw std::runtime_error("http: cannot resolve " + host + ": " + gai_strerror(rc));
  int fd = -1;
  for (addrinfo* a = res; a; a = a->ai_next) {
    fd = ::socket(a->ai_family, a->ai_socktype, a->ai_protocol);
    if (fd < 0) continue;
    const int one = 1;
    ::setsockopt(fd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof one);
    if (::bind(fd, a->ai_addr, a->ai_addrlen) == 0 && ::listen(fd, 64) == 0) break;
    ::close(fd);
    fd = -1;
  }
  ::freeaddrinfo(res);
  if (fd < 0) throw std::runtime_error("http: cannot listen on " + host + ":" + svc);
  sockaddr_storage ss{};
  socklen_t sl = sizeof ss;
  ::getsockname(fd, reinterpret_cast<sockaddr*>(&ss), &sl);
  listen_fd_ = fd;
  stopping_ = false;
  return ntohs(ss.ss_family == AF_INET6 ? reinterpret_cast<sockaddr_in6*>(&ss)->sin6_port
                                        : reinterpret_cast<sockaddr_in*>(&ss)->sin_port);
}

void Server::refuse(int fd) {
  timeval tv{1, 0};
  ::setsockopt(fd, SOL_SOCKET, SO_SNDTIMEO, &tv, sizeof tv);
  Writer w(fd);
  w.send(503, "application/json", "{\"error\":{\"message\":\"too many connections\",\"type\":\"server_error\"}}");
  ::shutdown(fd, SHUT_RDWR);
  ::close(fd);
}

// The accept loop. Out of descriptors or memory (EMFILE, ENFILE, ENOBUFS, ENOMEM) it retries after a pause; other
// errors end it (after stop(), the listener's shutdown is one).
void Server::serve() {
  while (!stopping_) {
    const int fd = ::accept(listen_fd_, nullptr, nullptr);
    if (fd < 0) {
      if (stopping_) break;
      if (errno == EINTR || errno == ECONNABORTED) continue;
      if (errno == EMFILE || errno == ENFILE || errno == ENOBUFS || errno == ENOMEM) {
        std::this_thread::sleep_for(std::chrono::milliseconds(50));
        continue;
      }
      break;
    }
    timeval tv{kTimeoutS, 0};
    ::setsockopt(fd, SOL_SOCKET, SO_RCVTIMEO, &tv, sizeof tv);
    ::setsockopt(fd, SOL_SOCKET, SO_SNDTIMEO, &tv, sizeof tv);
    bool full;
    {
      std::lock_guard<std::mutex> lk(m_);
      full = live_ >= kMaxConnections || stopping_;
      if (!full) {
        ++live_;
        clients_.insert(fd);
      }
    }
    if (full) {
      refuse(fd);
      continue;
    }
    try {
      std::thread([this, fd] { connection(fd); }).detach();
    } catch (const std::exception&) {  // no thread: refused like a connection past the cap
      {
        std::lock_guard<std::mutex> lk(m_);
        clients_.erase(fd);
        if (--live_ == 0) idle_.notify_all();
      }
      refuse(fd);
    }
  }
}

void Server::start() {
  accept_thread_ = std::thread([this] { serve(); });
}

void Server::connection(int fd) {
  try {
    Request rq;
    const int rc = read_request(fd, rq);
    Writer w(fd);
    if (rc > 0)
      w.send(rc, "application/json", std::string("{\"error\":{\"message\":\"") + reason(rc) +
                                          "\",\"type\":\"invalid_request_error\"}}");
    else if (rc == 0)
      handler_(rq, w);
  } catch (...) {
  }
  std::lock_guard<std::mutex> lk(m_);
  clients_.erase(fd);  // before the close, so that stop() never shuts down a reused descriptor
  ::shutdown(fd, SHUT_RDWR);
  ::close(fd);
  if (--live_ == 0) idle_.notify_all();
}

void Server::stop() {
  if (listen_fd_ >= 0) {
    stopping_ = true;
    ::shutdown(listen_fd_, SHUT_RDWR);
    if (accept_thread_.joinable()) accept_thread_.join();
    ::close(listen_fd_);
    listen_fd_ = -1;
  }
  std::unique_lock<std::mutex> lk(m_);
  for (const int fd : clients_) ::shutdown(fd, SHUT_RDWR);  // a pending recv or send returns at once
  idle_.wait(lk, [this] { return live_ == 0; });
}

}  // namespace malkin_hip::http
