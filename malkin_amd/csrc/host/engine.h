// Continuous batching and speculative decoding over the device Model: the token loop of the reference's
// malkin::Engine (engine.h:51-141, engine.cpp:242-501), without text, tokenizer or threads. Requests are token ids
// in, token ids out; each carries the reference's SamplingParams (greedy by default here).
//
// Contract (what the reference engine does, and therefore what the streams, KV rows and counters must equal):
//   * A request waits in FIFO order for an idle lane (one model sequence). It takes the idle lane whose cached
//     tokens share the longest prefix with its prompt (ties: the lane admitted least recently), keeps that prefix's
//     KV, and always re-evaluates at least its last prompt token.
//   * One step = one target forward. Its batch holds, lane by lane, every decoding lane's pending token followed by
//     its drafts, then prompt tokens of prefilling lanes in lane order until the batch has 256 tokens.
//   * Draft depth per decoding lane: its adaptive k (4 to start, at most n_draft), limited by its remaining budget
//     and by its context room and its share of the batch (both halved for greedy lanes, whose trees hold two tokens
//     per depth).
//   * Greedy lanes (temperature <= 0): the tree after the pending token at KV row P is chain_0, alt_0, chain_1,
//     alt_1, ...: chain_i and alt_i are the draft's first and second greedy picks at depth i, at RoPE position
//     P + 1 + i, KV rows P + 1 + 2i and P + 2 + 2i, both children of chain_{i-1} (of the pending token for i = 0).
//     Acceptance walks down from the pending token: while the target's pick at the current node (the first maximum
//     of its penalized logits) equals that depth's chain (or alt) token, that token is accepted, its KV row moves to
//     the next cache position, and the walk goes on below it (an alt is a leaf); the first pick that matches neither
//     becomes the next pending token. k grows by one after a fully accepted chain at full depth and shrinks by one
//     when fewer than half the drafts held.
//   * Sampled lanes (temperature > 0): the draft's sampler (the request's parameters, seed + 1, no penalties) draws
//     a chain d_0 .. d_{k-1}, fed back one token per draft forward; the target sees [pending, d_0, ..] in a row. Each
//     d_i is verified against the target's distribution at its position (Sampler::verify); the first rejection's
//     replacement becomes the pending token, a fully accepted chain draws the pending token from the last row. k
//     grows after a fully accepted chain at full depth and shrinks when fewer than half held.
//   * Every emitted token counts towards the request sampler's repetition penalties; the distribution of a row
//     sees the tokens accepted before it.
//   * A generated token ends its request when it is an end-of-generation id (not emitted, finish "stop"), when the
//     budget is reached, or when the context has no room for another row (finish "length").
//
// Device residency: greedy drafting runs back to back on the stream. Each round's tokens are the previous round's
// picks, read from a device array (Model::enqueue id redirects); picks are scattered into a per-lane tree array on
// the device; accepted rows move on the device. The host waits once per step, for the target's picks. Sampled
// lanes draw their drafts on the device as well (top-k of the draft row, then a draw with the draft sampler's
// generator, uploaded once per step) and the host replays those draws after the step's wait; sampled lanes whose
// draft needs more than 1024 candidates, or whose target rows take penalties, add one wait per draft round (the
// draw happens on the host); penalized greedy trees add one after the step's wait (the penalties of a tree row depend
// on its path, which the host learns at that wait).
#pragma once

#include <chrono>
#include <cstdint>
#include <deque>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "model.h"
#include "sampler.h"

namespace malkin_hip {

struct EngineRequest {
  std::vector<int32_t> prompt;
  int max_tokens = 0;          // 0: until the context ends
  std::vector<int32_t> eog;    // end-of-generation ids
  SamplingParams sampling{0.0f};  // greedy unless set
};

struct EngineResult {
  std::vector<int32_t> tokens;          // generated ids (an end-of-generation id is not included)
  std::string finish_reason = "length";  // "stop" (end-of-generation id) | "length" (budget or context) | "cancelled"
  int prompt_tokens = 0, cached_tokens = 0, completion_tokens = 0;
  int drafted = 0, accepted = 0;
  double prefill_ms = 0, decode_ms = 0;
  bool done = false;
};

class Engine {
 public:
  // target: one lane per sequence. draft (may be null): same vocabulary, at least as many sequences and context.
  // n_draft: maximum draft depth (0: 8, the reference's default).
  Engine(Model* target, Model* draft, int n_draft);
  ~Engine();
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  int submit(const EngineRequest& req);  // request id
  // Admits waiting requests into idle lanes, then one step; returns the number of lanes still busy.
  int step_once();
  void run();  // steps until no request waits or runs
  const EngineResult& result(int id) const;
  // Frees a finished request's result (its id is then unknown); a request still waiting or running is refused.
  void release(int id);
  size_t results_held() const { return results_.size(); }
  // Ends a waiting or running request now, finish "cancelled" (the reference's cancelled generation,
  // engine.cpp:509-512); a finished request is left as it is.
  void cancel(int id);
  int busy() const { return busy_; }
  int n_ctx() const { return target_->n_ctx(); }
  int n_vocab() const { return target_->cfg().n_vocab; }
  // The target model's end-of-generation ids (the set the reference's Tokenizer::is_eog tests, engine.cpp:60).
  const std::vector<int32_t>& model_eog() const { return target_->cfg().eog; }
  uint64_t steps() const { return steps_; }
  // Drafts drawn on the device so far, and how many of them the host's replay drew differently.
  uint64_t device_draws() const { return device_draws_; }
  uint64_t draw_mismatches() const { return draw_mismatches_; }

 private:
  using Clock = std::chrono::steady_clock;
  struct Job {
    EngineRequest req;
    EngineResult* res = nullptr;
    int budget = 0, k = 4;
    bool decoding = false;
    int32_t pending = 0;  // generated and emitted, not yet in the KV cache
    Clock::time_point admitted, first_token;
    std::unique_ptr<Sampler> sampler, draft_sampler;
    bool plain = true;  // greedy without penalties: the device's picks are the tokens
  };
  struct Lane {
    std::vector<int32_t> kv;        // tokens whose target KV rows are valid
    std::vector<int32_t> draft_kv;  // tokens whose draft KV rows are valid
    std::unique_ptr<Job> job;       // null: idle
    uint64_t stamp = 0;             // admission counter (least recently admitted wins a tie)
  };
  struct Spec {  // a decoding lane's share of one step
    int lane = 0, depth = 0, root = 0;  // root: batch index of the lane's pending token
    bool sampled = false;
    bool on_device = false;             // sampled, and its drafts drawn on the device (mk_sample_draw)
    std::vector<int32_t> chain;         // sampled lanes: the drawn drafts
    std::vector<Distribution> q;        // ... and the draft distributions they were drawn from
    std::vector<int> draws;             // on_device: the step's candidate row of each depth's draw
    const Selector* cand = nullptr;     // non-plain lanes: candidates of the target rows root.. (index sel..)
    int sel = -1;
  };

  void admit(std::unique_ptr<Job> job);
  void step();
  void plan_specs();
  void draft_trees();
  void draft_forward(const std::vector<BatchToken>& batch, const std::vector<int32_t>& id_from,
                     const std::vector<int32_t>& chain_slot);
  int build_target_batch();
  void select_known_rows(int decode_rows);
  void select_tree_rows();
  int32_t target_pick(const Spec& sp, int node) const;
  Distribution& target_dist(const Spec& sp, int row);
  void settle(const Spec& sp);
  void settle_sampled(const Spec& sp);
  void replay_draws();
  bool emit(Job& job, int32_t id, size_t cached);
  void finish(Lane& lane);
  int32_t* tree_host(int lane) { return tree_h_ + static_cast<size_t>(lane) * 2 * max_depth_; }
  int tree_slot(int lane, int depth, bool alt) const { return lane * 2 * max_depth_ + 2 * depth + (alt ? 1 : 0); }

  Model* target_;
  Model* draft_;
  int max_depth_ = 8;
  std::vector<Lane> lanes_;
  std::deque<std::unique_ptr<Job>> waiting_;
  std::map<int, std::unique_ptr<EngineResult>> results_;  // by request id, until released
  int next_id_ = 0;
  int busy_ = 0;
  uint64_t admissions_ = 0, steps_ = 0;

  // Per step.
  std::vector<Spec> specs_;
  std::vector<BatchToken> batch_;
  std::vector<int32_t> id_from_;
  std::vector<int> finishing_lanes_;  // prefilling lanes whose last prompt token is in this step's batch
  std::vector<int> finishing_sel_;    // their candidate rows in sel_ (non-plain jobs), else -1

  // Candidate selection: target rows known before the step's wait, penalized greedy tree rows after it, draft rows.
  Selector sel_, tree_sel_, draft_sel_;
  Distribution dist_;
  std::vector<int32_t> pen_ids_;
  std::vector<float> pen_amts_;

  // Device state: the per-lane draft trees (chain / alt ids by depth), the latest draft picks, the target's picks,
  // and the step's scatter plan (destination slots of each draft forward's picks).
  DevBuf tree_, draft_top1_, draft_top2_, target_top_, plan_;
  size_t plan_cap_ = 0, plan_used_ = 0;
  int32_t* plan_h_ = nullptr;  // pinned host copy of the plan, copied once per step
  int32_t* tree_h_ = nullptr;  // pinned: trees and target picks read back at the end of a step
  int32_t* picks_h_ = nullptr;
  std::vector<std::pair<size_t, int>> pending_scatters_;  // (plan offset, rows) of each queued draft forward

  // Device draws of sampled lanes' drafts: one upload per step of the draft samplers' generators (one slot per lane),
  // the draw parameters and the draft logits rows they read; the top-k candidates of every draw, copied back with
  // the step's wait for the host's replay of each draw.
  DevBuf draw_in_d_, cand_v_d_, cand_i_d_;
  uint8_t* draw_in_h_ = nullptr;
  float* cand_v_h_ = nullptr;
  int32_t* cand_i_h_ = nullptr;
  int draw_k_ = 0;                 // candidates per drawn row this step (the largest top_k of the drawing lanes)
  uint64_t device_draws_ = 0, draw_mismatches_ = 0;
};

}  // namespace malkin_hip
