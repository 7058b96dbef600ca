// The HTTP API over the device engine: the reference's OpenAI-style server (server.cpp:193-209, 315-358) for a
// build without tokenizer, so prompts and completions are token ids. One thread owns the engine and runs its loop
// (submissions in, one step, new tokens out to each request's channel); connection threads wait on their channel.
//
// Routes: GET /health; GET /v1/models; POST /v1/completions with "prompt" an array of token ids (or one such array
// inside an array), the reference's sampling fields (temperature, top_p, top_k, min_p, presence_penalty,
// frequency_penalty, seed; same defaults), "max_tokens" (default 16), "stop_token_ids" (end-of-generation ids) and
// "stream". A completion's choice carries "tokens" (ids) and "text" "" (no detokenizer); usage and timings as the
// reference reports them. A streaming response sends one server-sent event per engine step with the new ids, a last
// event with the finish reason, then "data: [DONE]"; a client that goes away cancels its request. The chat and
// messages routes answer 400: they need the tokenizer and chat template this build does not have.
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <deque>
#include <memory>
#include <mutex>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../../include/malkin_server.h"
#include "../host/capi_internal.h"
#include "../kernels/ctx.h"
#include "http.h"
#include "json.h"

namespace malkin_hip {

namespace {

using json::Value;

struct BadRequest : std::runtime_error {
  using std::runtime_error::runtime_error;
};

int64_t now_s() {
  return std::chrono::duration_cast<std::chrono::seconds>(std::chrono::system_clock::now().time_since_epoch()).count();
}

std::string new_id(const char* prefix) {
  static std::mutex m;
  static std::mt19937_64 rng{std::random_device{}()};
  std::lock_guard<std::mutex> lk(m);
  char buf[24];
  std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(rng()));
  return std::string(prefix) + buf;
}

Value error_body(int status, const std::string& msg) {
  return Value::object(
      {{"error", Value::object({{"message", msg},
                                {"type", status == 400 ? "invalid_request_error" : "server_error"}})}});
}

// One request's results as the engine loop hands them over.
struct Channel {
  std::mutex m;
  std::condition_variable cv;
  std::vector<int32_t> tokens;  // every generated id so far
  bool done = false;
  std::string error;            // submission refused (the reference's 400 texts)
  EngineResult final;
  std::atomic<bool> cancel{false};
};

class EngineLoop {
 public:
  explicit EngineLoop(Engine& e) : e_(e), th_([this] { run(); }) {}
  ~EngineLoop() { stop(); }

  std::shared_ptr<Channel> submit(EngineRequest req) {
    auto ch = std::make_shared<Channel>();
    {
      std::lock_guard<std::mutex> lk(m_);
      if (stopping_) throw std::runtime_error("server is stopping");
      incoming_.push_back({std::move(req), ch});
    }
    cv_.notify_one();
    return ch;
  }
  void wake() { cv_.notify_one(); }

  void stop() {
    {
      std::lock_guard<std::mutex> lk(m_);
      if (stopping_ && !th_.joinable()) return;
      stopping_ = true;
    }
    cv_.notify_one();
    if (th_.joinable()) th_.join();
  }

 private:
  struct Pending {
    EngineRequest req;
    std::shared_ptr<Channel> ch;
  };
  struct Active {
    int id;
    std::shared_ptr<Channel> ch;
    size_t reported = 0;
  };

  static void close_channel(Channel& ch, const EngineResult* r, const std::string& err) {
    {
      std::lock_guard<std::mutex> lk(ch.m);
      if (r) ch.final = *r;
      ch.error = err;
      ch.done = true;
    }
    ch.cv.notify_all();
  }

  void run() {
    for (;;) {
      std::deque<Pending> in;
      bool stopping;
      {
        std::unique_lock<std::mutex> lk(m_);
        cv_.wait(lk, [this] { return stopping_ || !incoming_.empty() || !active_.empty(); });
        in.swap(incoming_);
        stopping = stopping_;
      }
      for (Pending& p : in) {
        if (stopping) {
          close_channel(*p.ch, nullptr, "server is stopping");
          continue;
        }
        try {
          active_.push_back({e_.submit(p.req), p.ch, 0});
        } catch (const std::exception& ex) {
          close_channel(*p.ch, nullptr, ex.what());
        }
      }
      for (Active& a : active_)
        if (stopping || a.ch->cancel) e_.cancel(a.id);
      try {
        if (!stopping) e_.step_once();
      } catch (const std::exception& ex) {
        for (Active& a : active_) {
          e_.cancel(a.id);
          close_channel(*a.ch, nullptr, std::string("engine: ") + ex.what());
          try {
            e_.release(a.id);
          } catch (const std::exception&) {
          }
        }
        active_.clear();
        continue;
      }
      // Hand new tokens and finished results to the connections.
      for (size_t i = 0; i < active_.size();) {
        Active& a = active_[i];
        const EngineResult& r = e_.result(a.id);
        if (r.tokens.size() > a.reported) {
          {
            std::lock_guard<std::mutex> lk(a.ch->m);
            a.ch->tokens.assign(r.tokens.begin(), r.tokens.end());
          }
          a.reported = r.tokens.size();
          a.ch->cv.notify_all();
        }
        if (r.done) {
          close_channel(*a.ch, &r, "");  // copies the result out
          e_.release(a.id);
          active_.erase(active_.begin() + static_cast<std::ptrdiff_t>(i));
        } else {
          ++i;
        }
      }
      if (stopping && active_.empty()) return;
    }
  }

  Engine& e_;
  std::mutex m_;
  std::condition_variable cv_;
  std::deque<Pending> incoming_;
  std::vector<Active> active_;  // touched by the loop thread only
  bool stopping_ = false;
  std::thread th_;
};

Value usage_json(const EngineResult& r) {  // server.cpp:143-148
  return Value::object({{"prompt_tokens", r.prompt_tokens},
                        {"completion_tokens", r.completion_tokens},
                        {"total_tokens", r.prompt_tokens + r.completion_tokens},
                        {"prompt_tokens_details", Value::object({{"cached_tokens", r.cached_tokens}})}});
}

Value timings_json(const EngineResult& r) {  // server.cpp:150-160
  const int prefilled = r.prompt_tokens - r.cached_tokens;
  return Value::object({{"prompt_n", prefilled},
                        {"prompt_ms", r.prefill_ms},
                        {"prompt_per_second", r.prefill_ms > 0 ? prefilled * 1000.0 / r.prefill_ms : 0.0},
                        {"predicted_n", r.completion_tokens},
                        {"predicted_ms", r.decode_ms},
                        {"predicted_per_second", r.decode_ms > 0 ? r.completion_tokens * 1000.0 / r.decode_ms : 0.0},
                        {"draft_n", r.drafted},
                        {"draft_n_accepted", r.accepted}});
}

std::vector<int32_t> id_list(const Value& v, const char* what, int n_vocab) {
  std::vector<int32_t> out;
  for (const Value& x : v.items()) {
    if (!x.is_integer()) throw BadRequest(std::string(what) + " must hold integer token ids");
    const int64_t id = x.as_int();
    if (id < 0 || id >= n_vocab) throw BadRequest(std::string(what) + ": token id " + std::to_string(id) +
                                                  " outside the vocabulary");
    out.push_back(static_cast<int32_t>(id));
  }
  return out;
}

// An integer field that must fit an int: out-of-range values are refused (400) rather than narrowed.
int int_field(const Value& v, const char* name) {
  const int64_t x = v.as_int();
  if (x < INT32_MIN || x > INT32_MAX) throw BadRequest(std::string(name) + " is out of range");
  return static_cast<int>(x);
}

// sampling_from (server.cpp:59-69): the reference's defaults, each field optional.
SamplingParams sampling_from(const Value& b) {
  SamplingParams p;
  auto num = [&](const char* k, float& dst) {
    if (b.has(k) && !b[k].is_null()) dst = static_cast<float>(b[k].as_double());
  };
  num("temperature", p.temperature);
  num("top_p", p.top_p);
  num("min_p", p.min_p);
  num("presence_penalty", p.presence_penalty);
  num("frequency_penalty", p.frequency_penalty);
  if (b.has("top_k") && !b["top_k"].is_null()) p.top_k = int_field(b["top_k"], "top_k");
  // Any JSON integer, converted as the reference's get<uint64_t>() converts it: a negative value wraps modulo 2^64.
  if (b.has("seed") && b["seed"].is_integer()) {
    const Value& s = b["seed"];
    p.seed = s.kind() == Value::Kind::Uint ? s.as_uint() : static_cast<uint64_t>(s.as_int());
  }
  return p;
}

class Api {
 public:
  Api(Engine* e, std::string model_id) : model_id_(std::move(model_id)) {
    if (e) {
      engine_ = e;
      loop_ = std::make_unique<EngineLoop>(*e);
    }
  }
  void stop() {
    if (loop_) loop_->stop();
  }

  void handle(const http::Request& rq, http::Writer& w) {
    try {
      if (rq.path == "/health") {
        if (rq.method != "GET") return error(w, 405, "use GET");
        return reply(w, 200, Value::object({{"status", "ok"}}));
      }
      if (rq.path == "/v1/models") {
        if (rq.method != "GET") return error(w, 405, "use GET");
        Value m = Value::object({{"id", model_id_},
                                 {"object", "model"},
                                 {"created", now_s()},
                                 {"owned_by", "malkin"},
                                 {"context_length", engine_ ? engine_->n_ctx() : 0}});
        return reply(w, 200, Value::object({{"object", "list"}, {"data", Value::array({m})}}));
      }
      if (rq.path == "/v1/completions") {
        if (rq.method != "POST") return error(w, 405, "use POST");
        return completion(Value::parse(rq.body), w);
      }
      if (rq.path == "/v1/chat/completions" || rq.path == "/v1/messages")
        return error(w, 400, "this build has no tokenizer or chat template, use /v1/completions with token ids");
      return error(w, 404, "no route " + rq.path);
    } catch (const json::ParseError& ex) {
      return error(w, 400, std::string("bad json: ") + ex.what());
    } catch (const BadRequest& ex) {
      return error(w, 400, ex.what());
    } catch (const std::invalid_argument& ex) {
      return error(w, 400, ex.what());
    } catch (const std::exception& ex) {
      return error(w, 500, ex.what());
    }
  }

 private:
  static void reply(http::Writer& w, int status, const Value& v) { w.send(status, "application/json", v.dump()); }
  static void error(http::Writer& w, int status, const std::string& msg) { reply(w, status, error_body(status, msg)); }
  static std::string sse(const Value& v) { return "data: " + v.dump() + "\n\n"; }

  void completion(const Value& b, http::Writer& w) {
    if (!b.is_object()) throw BadRequest("the body must be a JSON object");
    if (!engine_) return error(w, 503, "no engine loaded");
    const Value& pr = b["prompt"];
    if (pr.is_string()) throw BadRequest("prompt must be an array of token ids: this build has no tokenizer");
    if (!pr.is_array()) throw BadRequest("prompt must be an array of token ids");
    const Value& ids = pr.items().size() == 1 && pr.items()[0].is_array() ? pr.items()[0] : pr;
    EngineRequest req;
    req.prompt = id_list(ids, "prompt", engine_->n_vocab());
    req.sampling = sampling_from(b);
    req.max_tokens = b.has("max_tokens") && !b["max_tokens"].is_null() ? int_field(b["max_tokens"], "max_tokens") : 16;
    if (req.max_tokens < 0) throw BadRequest("max_tokens must not be negative");
    // Generation stops at the model's end-of-generation ids, as the reference's engine does for every request
    // (engine.cpp:60), and at any further ids the client lists.
    req.eog = engine_->model_eog();
    if (b.has("stop_token_ids") && !b["stop_token_ids"].is_null()) {
      const std::vector<int32_t> extra = id_list(b["stop_token_ids"], "stop_token_ids", engine_->n_vocab());
      req.eog.insert(req.eog.end(), extra.begin(), extra.end());
    }
    if (b.has("stop") && !b["stop"].is_null() && !(b["stop"].is_array() && b["stop"].items().empty()))
      throw BadRequest("stop strings need a tokenizer: use stop_token_ids");
    const bool stream = b.has("stream") && b["stream"].as_bool();
    const std::string id = new_id("cmpl-");
    const int64_t created = now_s();
    auto body = [&](const std::vector<int32_t>& toks, size_t from, const Value& finish) {
      Value t = Value::array();
      for (size_t i = from; i < toks.size(); ++i) t.push(Value(static_cast<int64_t>(toks[i])));
      Value choice = Value::object({{"index", 0}, {"text", ""}, {"tokens", t}, {"finish_reason", finish}});
      return Value::object({{"id", id},
                            {"object", "text_completion"},
                            {"created", created},
                            {"model", model_id_},
                            {"choices", Value::array({choice})}});
    };
    std::shared_ptr<Channel> ch = loop_->submit(std::move(req));
    if (!stream) {
      std::unique_lock<std::mutex> lk(ch->m);
      ch->cv.wait(lk, [&] { return ch->done; });
      if (!ch->error.empty()) return error(w, 400, ch->error);
      Value out = body(ch->final.tokens, 0, Value(ch->final.finish_reason));
      out.set("usage", usage_json(ch->final));
      out.set("timings", timings_json(ch->final));
      return reply(w, 200, out);
    }
    bool open = false;  // the SSE stream starts with the first tokens, so refused submissions still get a 400
    size_t sent = 0;
    for (;;) {
      std::vector<int32_t> toks;
      bool done;
      std::string err;
      EngineResult fin;
      {
        std::unique_lock<std::mutex> lk(ch->m);
        ch->cv.wait(lk, [&] { return ch->done || ch->tokens.size() > sent; });
        toks = ch->tokens;
        done = ch->done;
        err = ch->error;
        if (done) fin = ch->final;
      }
      if (!open && !err.empty()) return error(w, 400, err);
      if (!open) {
        if (!w.begin_stream("text/event-stream")) break;
        open = true;
      }
      if (done && err.empty()) toks = fin.tokens;
      if (toks.size() > sent && !w.chunk(sse(body(toks, sent, Value())))) break;
      sent = toks.size();
      if (done) {
        if (!err.empty()) {
          w.chunk(sse(Value::object({{"error", Value::object({{"message", err}})}})));
        } else {
          Value last = body(toks, toks.size(), Value(fin.finish_reason));
          last.set("usage", usage_json(fin));
          last.set("timings", timings_json(fin));
          w.chunk(sse(last));
        }
        w.chunk("data: [DONE]\n\n");
        w.end_stream();
        return;
      }
    }
    // The client went away: cancel the request (the reference's on_text returning false) and let it finish.
    ch->cancel = true;
    loop_->wake();
    std::unique_lock<std::mutex> lk(ch->m);
    ch->cv.wait(lk, [&] { return ch->done; });
  }

  Engine* engine_ = nullptr;
  std::string model_id_;
  std::unique_ptr<EngineLoop> loop_;
};

}  // namespace

}  // namespace malkin_hip

struct mk_server {
  mk_engine* engine = nullptr;
  std::unique_ptr<malkin_hip::Api> api;
  std::unique_ptr<malkin_hip::http::Server> http;
};

extern "C" {

int mk_server_start(mk_engine* e, const char* model_id, const char* host, int port, mk_server** out,
                    int* bound_port) {
  try {
    if (!out || !host || port < 0 || port > 65535) throw std::invalid_argument("mk_server_start: bad argument");
    if (e && e->serving) throw std::invalid_argument("mk_server_start: the engine is already serving");
    auto s = std::make_unique<mk_server>();
    s->engine = e;
    s->api = std::make_unique<malkin_hip::Api>(e ? e->engine.get() : nullptr, model_id ? model_id : "malkin");
    malkin_hip::Api* api = s->api.get();
    s->http = std::make_unique<malkin_hip::http::Server>(
        [api](const malkin_hip::http::Request& rq, malkin_hip::http::Writer& w) { api->handle(rq, w); });
    const int p = s->http->bind(host, port);
    s->http->start();
    if (e) e->serving = true;
    if (bound_port) *bound_port = p;
    *out = s.release();
    return MK_OK;
  } catch (const std::exception& ex) {
    mk::set_error("%s", ex.what());
    return MK_ERR_INVALID;
  }
}

int mk_server_stop(mk_server* s) {
  if (!s) return MK_OK;
  // No new connections; the engine loop cancels what is in flight and ends; then the connections drain.
  s->api->stop();
  s->http->stop();
  if (s->engine) s->engine->serving = false;
  delete s;
  return MK_OK;
}

}  // extern "C"
