#include "engine.h"

#include <algorithm>
#include <stdexcept>

namespace malkin_hip {

namespace {

void ck(int rc) {
  if (rc != MK_OK) throw std::runtime_error(mk_last_error());
}

double ms_between(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
  return std::chrono::duration<double, std::milli>(b - a).count();
}

size_t common_prefix(const std::vector<int32_t>& a, const std::vector<int32_t>& b) {
  const size_t n = std::min(a.size(), b.size());
  size_t i = 0;
  while (i < n && a[i] == b[i]) ++i;
  return i;
}

// One draft forward of a step, planned on the host before anything is queued.
struct DraftPass {
  std::vector<BatchToken> batch;
  std::vector<int32_t> id_from;              // per token: tree slot its id comes from, or -1
  std::vector<int32_t> chain_dst, alt_dst;   // per logits row: tree slots of its first / second pick
};

}  // namespace

Engine::Engine(Model* target, Model* draft, int n_draft) : target_(target), draft_(draft) {
  if (!target_) throw std::invalid_argument("engine: no target model");
  if (draft_) {
    if (draft_->cfg().n_vocab != target_->cfg().n_vocab)
      throw std::runtime_error("draft model tokenizer differs from the target");  // engine.cpp:121
    if (draft_->n_seq() < target_->n_seq()) throw std::invalid_argument("engine: draft has fewer sequences");
    if (draft_->n_ctx() < target_->n_ctx()) throw std::invalid_argument("engine: draft context is shorter");
    if (draft_->ctx() != target_->ctx()) throw std::invalid_argument("engine: draft runs on another context");
  }
  if (n_draft > 0) max_depth_ = std::min(n_draft, Model::kMaxBatch - 1);  // engine.cpp:126
  lanes_.resize(static_cast<size_t>(target_->n_seq()));
  mk_ctx* c = target_->ctx();
  const size_t S = lanes_.size(), slots = S * 2 * static_cast<size_t>(max_depth_);
  tree_ = DevBuf(c, slots * sizeof(int32_t));
  ck(mk_fill(c, tree_.p, 0, tree_.bytes));
  draft_top1_ = DevBuf(c, Model::kMaxBatch * sizeof(int32_t));
  draft_top2_ = DevBuf(c, Model::kMaxBatch * sizeof(int32_t));
  target_top_ = DevBuf(c, Model::kMaxBatch * sizeof(int32_t));
  // Scatter destinations of one step: every draft forward has at most one logits row per lane; there are at most
  // (catch-up forwards) + (rounds) of them: a lane's catch-up is at most its context, in 256-token forwards.
  const size_t catchup = S + S * static_cast<size_t>(target_->n_ctx()) / Model::kMaxBatch + 1;
  plan_cap_ = 2 * S * (catchup + static_cast<size_t>(max_depth_) + 1);
  plan_ = DevBuf(c, plan_cap_ * sizeof(int32_t));
  void* h = nullptr;
  ck(mk_host_alloc(c, plan_cap_ * sizeof(int32_t), &h));
  plan_h_ = static_cast<int32_t*>(h);
  ck(mk_host_alloc(c, (slots + Model::kMaxBatch) * sizeof(int32_t), &h));
  tree_h_ = static_cast<int32_t*>(h);
  picks_h_ = tree_h_ + slots;
}

Engine::~Engine() {
  mk_ctx* c = target_->ctx();
  (void)mk_host_free(c, plan_h_);
  (void)mk_host_free(c, tree_h_);
}

int Engine::submit(const EngineRequest& req) {
  const int n_ctx = target_->n_ctx();
  if (req.prompt.empty()) throw std::invalid_argument("empty prompt");  // engine.cpp:227-232
  if (static_cast<int>(req.prompt.size()) >= n_ctx)
    throw std::invalid_argument("prompt has " + std::to_string(req.prompt.size()) + " tokens, context is " +
                                std::to_string(n_ctx));
  for (int32_t id : req.prompt)
    if (id < 0 || id >= target_->cfg().n_vocab) throw std::invalid_argument("prompt token id out of range");
  results_.push_back(std::make_unique<EngineResult>());
  auto job = std::make_unique<Job>();
  job->req = req;
  job->res = results_.back().get();
  job->budget = req.max_tokens > 0 ? req.max_tokens : n_ctx;
  job->admitted = Clock::now();
  waiting_.push_back(std::move(job));
  return static_cast<int>(results_.size()) - 1;
}

const EngineResult& Engine::result(int id) const {
  if (id < 0 || id >= static_cast<int>(results_.size())) throw std::invalid_argument("engine: bad request id");
  return *results_[static_cast<size_t>(id)];
}

int Engine::step_once() {
  while (!waiting_.empty() && busy_ < static_cast<int>(lanes_.size())) {
    admit(std::move(waiting_.front()));
    waiting_.pop_front();
  }
  if (busy_ > 0) step();
  return busy_;
}

void Engine::run() {
  while (!waiting_.empty() || busy_ > 0) step_once();
}

void Engine::admit(std::unique_ptr<Job> job) {
  const auto& prompt = job->req.prompt;
  Lane* best = nullptr;
  size_t best_len = 0;
  for (Lane& lane : lanes_) {
    if (lane.job) continue;
    const size_t len = common_prefix(lane.kv, prompt);
    if (!best || len > best_len || (len == best_len && lane.stamp < best->stamp)) {
      best = &lane;
      best_len = len;
    }
  }
  const size_t keep = std::min(best_len, prompt.size() - 1);  // the last prompt token is evaluated for its logits
  best->kv.resize(keep);
  job->res->prompt_tokens = static_cast<int>(prompt.size());
  job->res->cached_tokens = static_cast<int>(keep);
  job->res->finish_reason = "length";
  job->k = std::min(4, max_depth_);
  best->stamp = ++admissions_;
  best->job = std::move(job);
  ++busy_;
}

void Engine::plan_specs() {
  specs_.clear();
  for (size_t i = 0; i < lanes_.size(); ++i)
    if (lanes_[i].job && lanes_[i].job->decoding) specs_.push_back(Spec{static_cast<int>(i), 0, 0});
  if (!draft_ || specs_.empty()) return;
  const int share = Model::kMaxBatch / static_cast<int>(specs_.size()) - 1;  // tokens per lane after its pending one
  for (Spec& sp : specs_) {
    const Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
    const Job& job = *lane.job;
    const int left = job.budget - job.res->completion_tokens;
    const int room = target_->n_ctx() - static_cast<int>(lane.kv.size()) - 2;
    // two tree tokens (chain and alt) per depth
    sp.depth = std::max(0, std::min({job.k, left, room / 2, share / 2}));
  }
}

// The draft's part of a step, all queued before the host waits: catch-up forwards that bring each drafting lane's
// draft KV to its target tokens plus the pending token (prefix rows reused), then one forward per depth that feeds
// every lane's chain token of that depth. Each forward's picks go to the next depth's tree slots.
void Engine::draft_trees() {
  std::vector<DraftPass> passes(1);
  std::vector<int> fed_from(lanes_.size(), -1);  // draft_kv index of each lane's first chain token fed
  auto room_for = [&](DraftPass& p) -> DraftPass& {
    if (static_cast<int>(p.batch.size()) < Model::kMaxBatch) return p;
    passes.emplace_back();
    return passes.back();
  };
  for (const Spec& sp : specs_) {
    if (sp.depth == 0) continue;
    Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
    const size_t n_tok = lane.kv.size() + 1;  // target tokens plus the pending one
    size_t keep = common_prefix(lane.draft_kv, lane.kv);
    if (keep == lane.kv.size() && lane.draft_kv.size() > keep && lane.draft_kv[keep] == lane.job->pending) ++keep;
    keep = std::min(keep, n_tok - 1);  // the last token is evaluated for its logits
    lane.draft_kv.resize(keep);
    for (size_t pos = keep; pos < n_tok; ++pos) {
      const int32_t id = pos < lane.kv.size() ? lane.kv[pos] : lane.job->pending;
      const bool last = pos + 1 == n_tok;
      DraftPass& p = room_for(passes.back());
      p.batch.push_back(BatchToken{id, sp.lane, static_cast<int>(pos), last});
      p.id_from.push_back(-1);
      if (last) {
        p.chain_dst.push_back(tree_slot(sp.lane, 0, false));
        p.alt_dst.push_back(tree_slot(sp.lane, 0, true));
      }
      lane.draft_kv.push_back(id);
    }
  }
  for (int d = 0;; ++d) {  // depth d's chain tokens fed, their picks are depth d + 1
    DraftPass p;
    for (const Spec& sp : specs_) {
      if (d + 1 >= sp.depth) continue;
      Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
      if (d == 0) fed_from[static_cast<size_t>(sp.lane)] = static_cast<int>(lane.draft_kv.size());
      p.batch.push_back(BatchToken{0, sp.lane, static_cast<int>(lane.draft_kv.size()), true});
      p.id_from.push_back(tree_slot(sp.lane, d, false));
      p.chain_dst.push_back(tree_slot(sp.lane, d + 1, false));
      p.alt_dst.push_back(tree_slot(sp.lane, d + 1, true));
      lane.draft_kv.push_back(-1);  // the chain id, known on the host after the step's wait
    }
    if (p.batch.empty()) break;
    passes.push_back(std::move(p));
  }
  // The scatter plan of all passes in one pinned block and one copy.
  size_t off = 0;
  std::vector<size_t> at(passes.size());
  for (size_t i = 0; i < passes.size(); ++i) {
    at[i] = off;
    const size_t m = passes[i].chain_dst.size();
    if (off + 2 * m > plan_cap_) throw std::runtime_error("engine: draft plan exceeds its buffer");
    std::copy(passes[i].chain_dst.begin(), passes[i].chain_dst.end(), plan_h_ + off);
    std::copy(passes[i].alt_dst.begin(), passes[i].alt_dst.end(), plan_h_ + off + m);
    off += 2 * m;
  }
  mk_ctx* c = target_->ctx();
  ck(mk_copy_async(c, plan_.p, plan_h_, off * sizeof(int32_t)));
  int32_t* tree = tree_.as<int32_t>();
  for (size_t i = 0; i < passes.size(); ++i) {
    const DraftPass& p = passes[i];
    if (p.batch.empty()) continue;
    const int m = static_cast<int>(p.chain_dst.size());
    draft_->enqueue(p.batch.data(), static_cast<int>(p.batch.size()), p.id_from.data(), tree, draft_top1_.as<int32_t>(),
                    draft_top2_.as<int32_t>());
    int32_t* dst = plan_.as<int32_t>() + at[i];
    ck(mk_move_ids(c, tree, dst, draft_top1_.as<int32_t>(), nullptr, m));
    ck(mk_move_ids(c, tree, dst + m, draft_top2_.as<int32_t>(), nullptr, m));
  }
  // Remember where each lane's chain tokens sit in draft_kv (filled in after the wait).
  for (Spec& sp : specs_) sp.root = fed_from[static_cast<size_t>(sp.lane)];
}

// Decoding lanes' pending tokens and trees, then prompt tokens; returns the number of decode rows.
int Engine::build_target_batch() {
  batch_.clear();
  id_from_.clear();
  finishing_lanes_.clear();
  for (Spec& sp : specs_) {
    const Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
    const int P = static_cast<int>(lane.kv.size());
    const int root = static_cast<int>(batch_.size());
    batch_.push_back(BatchToken{lane.job->pending, sp.lane, P, true});
    id_from_.push_back(-1);
    for (int d = 0; d < sp.depth; ++d) {
      const int parent = d == 0 ? root : root + 2 * d - 1;  // chain_{d-1}
      batch_.push_back(BatchToken{0, sp.lane, P + 1 + d, true, P + 1 + 2 * d, parent});
      id_from_.push_back(tree_slot(sp.lane, d, false));
      batch_.push_back(BatchToken{0, sp.lane, P + 1 + d, true, P + 2 + 2 * d, parent});
      id_from_.push_back(tree_slot(sp.lane, d, true));
    }
    sp.root = root;
  }
  const int decode_rows = static_cast<int>(batch_.size());
  for (size_t i = 0; i < lanes_.size(); ++i) {
    const Lane& lane = lanes_[i];
    if (!lane.job || lane.job->decoding) continue;
    const auto& prompt = lane.job->req.prompt;
    const int from = static_cast<int>(lane.kv.size());
    const int take = std::min(Model::kMaxBatch - static_cast<int>(batch_.size()), static_cast<int>(prompt.size()) - from);
    for (int pos = from; pos < from + take; ++pos) {
      const bool last = pos + 1 == static_cast<int>(prompt.size());
      batch_.push_back(BatchToken{prompt[static_cast<size_t>(pos)], static_cast<int>(i), pos, last});
      id_from_.push_back(-1);
      if (last) finishing_lanes_.push_back(static_cast<int>(i));
    }
  }
  return decode_rows;
}

void Engine::step() {
  plan_specs();
  std::vector<int> chain_at;
  const bool drafting = std::any_of(specs_.begin(), specs_.end(), [](const Spec& s) { return s.depth > 0; });
  if (drafting) {
    draft_trees();
    for (const Spec& sp : specs_) chain_at.push_back(sp.root);
  }
  const int decode_rows = build_target_batch();
  const int n = static_cast<int>(batch_.size());
  if (n == 0) return;
  mk_ctx* c = target_->ctx();
  target_->enqueue(batch_.data(), n, id_from_.data(), tree_.as<int32_t>(), target_top_.as<int32_t>(), nullptr);
  const int rows = target_->n_out();
  ck(mk_copy_async(c, picks_h_, target_top_.p, static_cast<size_t>(rows) * sizeof(int32_t)));
  if (drafting) ck(mk_copy_async(c, tree_h_, tree_.p, lanes_.size() * 2 * max_depth_ * sizeof(int32_t)));
  ck(mk_synchronize(c));  // the step's one host wait
  ++steps_;

  if (drafting)  // the chain ids fed to the draft, now known on the host
    for (size_t i = 0; i < specs_.size(); ++i) {
      const Spec& sp = specs_[i];
      if (chain_at[i] < 0) continue;
      Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
      for (int d = 0; d + 1 < sp.depth; ++d)
        lane.draft_kv[static_cast<size_t>(chain_at[i] + d)] = tree_host(sp.lane)[2 * d];
    }
  for (int t = decode_rows; t < n; ++t) lanes_[static_cast<size_t>(batch_[t].seq)].kv.push_back(batch_[t].id);
  for (size_t j = 0; j < finishing_lanes_.size(); ++j) {  // prompts that finished: their first token
    Lane& lane = lanes_[static_cast<size_t>(finishing_lanes_[j])];
    Job& job = *lane.job;
    job.first_token = Clock::now();
    job.res->prefill_ms = ms_between(job.admitted, job.first_token);
    job.decoding = true;
    job.pending = picks_h_[decode_rows + static_cast<int>(j)];
    if (!emit(job, job.pending, lane.kv.size())) finish(lane);
  }
  for (const Spec& sp : specs_) settle(sp, picks_h_);
}

// The acceptance walk of one decoding lane over the target's picks (rows root.. of this step).
void Engine::settle(const Spec& sp, const int32_t* picks) {
  Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
  Job& job = *lane.job;
  const int P = static_cast<int>(lane.kv.size());
  lane.kv.push_back(job.pending);
  job.res->drafted += sp.depth;
  bool alive = true, missed = false;
  int node = 0, held = 0;  // tree node the walk stands on (0 = the pending token), draft depths accepted
  const int32_t* tree = tree_host(sp.lane);
  for (int d = 0; d < sp.depth; ++d) {
    const int32_t want = picks[sp.root + node];
    int next = -1;
    if (want == tree[2 * d])
      next = 1 + 2 * d;
    else if (want == tree[2 * d + 1])
      next = 2 + 2 * d;
    if (next < 0) {  // the target disagrees with both: its pick is the next pending token
      job.pending = want;
      missed = true;
      break;
    }
    target_->move_kv(P + next, static_cast<int>(lane.kv.size()), sp.lane);
    lane.kv.push_back(want);
    ++job.res->accepted;
    node = next;
    alive = emit(job, want, lane.kv.size());
    if (!alive) break;
    held = d + 1;
    if (next == 2 + 2 * d) break;  // an alt token has no children
  }
  if (alive && !missed) job.pending = picks[sp.root + node];
  if (sp.depth > 0) {
    if (held == sp.depth && sp.depth == job.k && node == 2 * sp.depth - 1)
      job.k = std::min(job.k + 1, max_depth_);
    else if (2 * held < sp.depth)
      job.k = std::max(1, job.k - 1);
  }
  if (alive) alive = emit(job, job.pending, lane.kv.size());
  if (!alive) finish(lane);
}

bool Engine::emit(Job& job, int32_t id, size_t cached) {
  if (std::find(job.req.eog.begin(), job.req.eog.end(), id) != job.req.eog.end()) {
    job.res->finish_reason = "stop";
    return false;
  }
  job.res->tokens.push_back(id);
  ++job.res->completion_tokens;
  if (job.res->completion_tokens >= job.budget) return false;
  return static_cast<int>(cached) + 1 < target_->n_ctx();
}

void Engine::finish(Lane& lane) {
  Job& job = *lane.job;
  job.res->decode_ms = ms_between(job.first_token, Clock::now());
  job.res->done = true;
  lane.job.reset();
  --busy_;
}

}  // namespace malkin_hip
