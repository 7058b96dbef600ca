// Continuous-batching and speculative-decoding token loop over the device Model: the greedy part of the reference's
// malkin::Engine (engine.h:51-141, engine.cpp:242-479), without text, tokenizer, sampling or threads. Requests are
// token ids in, token ids out; every forward pass and every greedy pick runs on the GPU (forward_top2 returns ids,
// never logits), and accepted tree nodes move their KV rows on the device.
//
// Semantics kept from the reference:
//   admit        a request goes to the idle slot whose cached tokens share the longest prefix with its prompt (ties:
//                least recently admitted); that prefix's KV is reused, but the last prompt token is always evaluated
//                (engine.cpp:242-265);
//   step         one target forward over every busy slot: decoding slots put their next token (plus, with a draft
//                model, the draft's greedy tree), then prompt chunks follow in slot order up to kMaxBatch tokens
//                (engine.cpp:360-424);
//   plan_drafts  draft length per decoding slot: the slot's adaptive k within its budget, its context room and a
//                share of the batch (engine.cpp:336-357);
//   propose      the draft catches its KV up to the slot's tokens (prefix reuse), then rounds in which every slot
//                takes the draft's top-1 (chain) and runner-up (alternative) and feeds the chain token back
//                (engine.cpp:267-334);
//   layout       per slot [next, chain0, alt0, chain1, alt1, ...] at KV rows P, P + 1, ...; chain i and alt i sit at
//                position P + 1 + i under chain i - 1 (engine.cpp:359-381);
//   accept       walk the tree along the target's argmax, moving each accepted node's KV row to the next cache
//                position; the first miss becomes the next token; k grows after a fully accepted chain and
//                shrinks when fewer than half the drafts hold (engine.cpp:441-479);
//   emit         a token ends the request when it is an end-of-generation id (not emitted), reaches the budget, or
//                leaves no room in the context (engine.cpp:50-88).
#pragma once

#include <chrono>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "model.h"

namespace malkin_hip {

struct EngineRequest {
  std::vector<int32_t> prompt;
  int max_tokens = 0;          // 0: until the context ends
  std::vector<int32_t> eog;    // end-of-generation ids
};

struct EngineResult {
  std::vector<int32_t> tokens;          // generated ids (an end-of-generation id is not included)
  std::string finish_reason = "length";  // "stop" (end-of-generation id) | "length" (budget or context)
  int prompt_tokens = 0, cached_tokens = 0, completion_tokens = 0;
  int drafted = 0, accepted = 0;
  double prefill_ms = 0, decode_ms = 0;
  bool done = false;
};

class Engine {
 public:
  // target: n_seq slots (one sequence each). draft (may be null): same vocabulary, at least as many sequences.
  // n_draft: maximum draft tokens per step (0: 8, the reference's default).
  Engine(Model* target, Model* draft, int n_draft);
  int submit(const EngineRequest& req);  // request id
  // Admits pending requests into idle slots, then one step; returns the number of slots still busy.
  int step_once();
  void run();  // steps until no request is pending or in flight
  const EngineResult& result(int id) const;
  int busy() const { return busy_; }

 private:
  using Clock = std::chrono::steady_clock;
  struct Request {
    EngineRequest req;
    EngineResult* res;
    int budget = 0, k = 4;
    bool decoding = false;
    int32_t next = 0;
    Clock::time_point t0, t1;
  };
  struct Slot {
    std::vector<int32_t> cache;   // tokens whose target KV is valid
    std::vector<int32_t> dcache;  // tokens whose draft KV is valid
    std::unique_ptr<Request> req;
    uint64_t used = 0;
  };
  struct Proposal {
    int seq = 0, kk = 0, root = 0;
    std::vector<int32_t> chain, alt;
  };

  void admit(std::unique_ptr<Request> r);
  void step();
  bool plan_drafts();
  void propose();
  int build_batch();
  void accept(const Proposal& p);
  bool accept_greedy(const Proposal& p, Slot& s, int P);
  bool emit(Request& q, int32_t id, size_t cached);
  void finish(Slot& s);

  Model* model_;
  Model* draft_;
  int n_draft_ = 8;
  std::vector<Slot> slots_;
  std::vector<std::unique_ptr<Request>> pending_;
  std::vector<std::unique_ptr<EngineResult>> results_;
  int busy_ = 0;
  uint64_t admitted_ = 0;
  std::vector<Proposal> props_;
  std::vector<BatchToken> batch_, dbatch_;
  std::vector<int> batch_seq_;          // prompt-finishing slot of each logits row after the decode rows
  std::vector<int32_t> top1_, dtop1_, dtop2_, dslot1_, dslot2_;
};

}  // namespace malkin_hip
