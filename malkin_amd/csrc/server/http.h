// A minimal HTTP/1.1 server over POSIX sockets for the token API: one request per connection (Connection: close),
// a thread per connection, bodies by Content-Length (at most 64 MiB), responses with a Content-Length or as a
// chunked stream (server-sent events). Read and write time out after 600 s, as the reference's server sets them.
#pragma once

#include <atomic>
#include <condition_variable>
#include <functional>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <thread>

namespace malkin_hip::http {

struct Request {
  std::string method, path;  // path without the query string
  std::map<std::string, std::string> headers;  // lower-case names
  std::string body;
};

// Writes one response on a connection. Every call returns false once the peer is gone.
class Writer {
 public:
  explicit Writer(int fd) : fd_(fd) {}
  bool send(int status, const std::string& content_type, const std::string& body);
  bool begin_stream(const std::string& content_type);  // 200, Transfer-Encoding: chunked
  bool chunk(const std::string& data);
  bool end_stream();

 private:
  bool write_all(const std::string& s);
  int fd_;
  bool ok_ = true;
};

using Handler = std::function<void(const Request&, Writer&)>;

class Server {
 public:
  explicit Server(Handler h) : handler_(std::move(h)) {}
  ~Server();
  Server(const Server&) = delete;
  Server& operator=(const Server&) = delete;

  // Binds host:port (port 0: any free port); returns the bound port. Throws std::runtime_error.
  int bind(const std::string& host, int port);
  void serve();  // the accept loop, until stop()
  void start();  // serve() on a thread of its own
  void stop();   // closes the listener, shuts the open connections down, waits for their threads

  static constexpr int kMaxConnections = 256;  // open connections; beyond it a client gets 503 at once

 private:
  void connection(int fd);
  void refuse(int fd);  // 503 on the accept thread, then close

  Handler handler_;
  int listen_fd_ = -1;
  std::atomic<bool> stopping_{false};
  std::thread accept_thread_;
  std::mutex m_;
  std::condition_variable idle_;
  int live_ = 0;            // connection threads running (detached; stop() waits for none)
  std::set<int> clients_;   // their sockets, shut down by stop()
};

}  // namespace malkin_hip::http
