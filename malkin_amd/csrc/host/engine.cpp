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
  std::vector<int32_t> chain_dst, alt_dst;   // per logits row: tree slots of its first / second pick (-1: none)
  int depth = -1;                            // round passes: the depth whose chain tokens are fed
  std::vector<std::pair<int, int>> fed;      // (batch index, spec) of sampled lanes' chain tokens, set at launch
  std::vector<std::pair<int, int>> drawn;    // (logits row, spec) whose row the host draws the next draft from
  std::vector<std::pair<int, int>> dev_drawn;  // (logits row, spec) whose row the device draws the next draft from
};

// Upload block of the device draws: generators [lanes][MK_MT64_WORDS], then params [rows], then logits rows [rows].
static_assert(Mt64::kWords == MK_MT64_WORDS, "the host generator's layout is mk_sample_draw's");

size_t draw_block_bytes(size_t lanes, size_t rows) {
  return lanes * MK_MT64_WORDS * sizeof(uint64_t) + rows * (sizeof(mk_draw_params) + sizeof(int32_t));
}

}  // namespace

Engine::Engine(Model* target, Model* draft, int n_draft)
    : target_(target),
      draft_(draft),
      sel_(target->ctx(), target->cfg().n_vocab),
      tree_sel_(target->ctx(), target->cfg().n_vocab),
      draft_sel_(target->ctx(), target->cfg().n_vocab) {
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
  if (draft_) {  // at most one draw per lane and depth in a step
    const size_t rows = S * static_cast<size_t>(max_depth_), cand = rows * Selector::kMaxDeviceK;
    draw_in_d_ = DevBuf(c, draw_block_bytes(S, rows));
    ck(mk_host_alloc(c, draw_block_bytes(S, rows), &h));
    draw_in_h_ = static_cast<uint8_t*>(h);
    cand_v_d_ = DevBuf(c, cand * sizeof(float));
    cand_i_d_ = DevBuf(c, cand * sizeof(int32_t));
    ck(mk_host_alloc(c, cand * sizeof(float), &h));
    cand_v_h_ = static_cast<float*>(h);
    ck(mk_host_alloc(c, cand * sizeof(int32_t), &h));
    cand_i_h_ = static_cast<int32_t*>(h);
  }
}

Engine::~Engine() {
  mk_ctx* c = target_->ctx();
  (void)mk_host_free(c, plan_h_);
  (void)mk_host_free(c, tree_h_);
  (void)mk_host_free(c, draw_in_h_);
  (void)mk_host_free(c, cand_v_h_);
  (void)mk_host_free(c, cand_i_h_);
}

int Engine::submit(const EngineRequest& req) {
  const int n_ctx = target_->n_ctx();
  if (req.prompt.empty()) throw std::invalid_argument("empty prompt");  // engine.cpp:227-232
  if (static_cast<int>(req.prompt.size()) >= n_ctx)
    throw std::invalid_argument("prompt has " + std::to_string(req.prompt.size()) + " tokens, context is " +
                                std::to_string(n_ctx));
  for (int32_t id : req.prompt)
    if (id < 0 || id >= target_->cfg().n_vocab) throw std::invalid_argument("prompt token id out of range");
  const int id = next_id_++;
  auto job = std::make_unique<Job>();
  job->req = req;
  job->res = (results_[id] = std::make_unique<EngineResult>()).get();
  job->budget = req.max_tokens > 0 ? req.max_tokens : n_ctx;
  job->admitted = Clock::now();
  // The request's sampler counts its tokens for the penalties; the draft's draws with seed + 1 and no penalties
  // (engine.cpp:40-44).
  job->sampler = std::make_unique<Sampler>(req.sampling, true);
  SamplingParams dp = req.sampling;
  dp.seed = dp.seed ? dp.seed + 1 : 0;
  job->draft_sampler = std::make_unique<Sampler>(dp, false);
  job->plain = job->sampler->greedy() && !job->sampler->penalizes();
  waiting_.push_back(std::move(job));
  return id;
}

const EngineResult& Engine::result(int id) const {
  const auto it = results_.find(id);
  if (it == results_.end()) throw std::invalid_argument("engine: bad request id");
  return *it->second;
}

void Engine::release(int id) {
  const auto it = results_.find(id);
  if (it == results_.end()) throw std::invalid_argument("engine: bad request id");
  if (!it->second->done) throw std::invalid_argument("engine: request still in flight");
  results_.erase(it);
}

void Engine::cancel(int id) {
  const auto it = results_.find(id);
  if (it == results_.end()) throw std::invalid_argument("engine: bad request id");
  EngineResult* r = it->second.get();
  if (r->done) return;
  r->finish_reason = "cancelled";
  for (auto it = waiting_.begin(); it != waiting_.end(); ++it)
    if ((*it)->res == r) {
      r->done = true;
      waiting_.erase(it);
      return;
    }
  for (Lane& lane : lanes_)
    if (lane.job && lane.job->res == r) {
      finish(lane);
      return;
    }
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
    if (lanes_[i].job && lanes_[i].job->decoding) {
      specs_.emplace_back();
      specs_.back().lane = static_cast<int>(i);
      specs_.back().sampled = !lanes_[i].job->sampler->greedy();
    }
  if (!draft_ || specs_.empty()) return;
  const int share = Model::kMaxBatch / static_cast<int>(specs_.size()) - 1;  // tokens per lane after its pending one
  for (Spec& sp : specs_) {
    const Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
    const Job& job = *lane.job;
    const int left = job.budget - job.res->completion_tokens;
    const int room = target_->n_ctx() - static_cast<int>(lane.kv.size()) - 2;
    const int per_depth = sp.sampled ? 1 : 2;  // a greedy tree holds chain and alt tokens
    sp.depth = std::max(0, std::min({job.k, left, room / per_depth, share / per_depth}));
    // The device draws a sampled lane's drafts when its draft sampler's candidates fit mk_topk and the target rows'
    // penalties do not depend on the drafts (the target's candidates are then selected before the step's wait).
    sp.on_device = sp.sampled && sp.depth > 0 && !job.sampler->penalizes() &&
                   job.draft_sampler->candidates(target_->cfg().n_vocab) <= Selector::kMaxDeviceK;
  }
}

// The draft's part of a step: catch-up forwards that bring each drafting lane's draft KV to its target tokens plus
// the pending token (prefix rows reused), then one forward per depth that feeds every lane's chain token of that
// depth. Greedy lanes: each forward's picks go to the next depth's tree slots on the device, nothing waits.
// Sampled lanes whose draft candidates fit mk_topk (and whose target rows take no penalties): the device cuts each
// row they draw from to its top-k and draws from it with the draft sampler's generator (uploaded once per step) into
// the next depth's chain slot; nothing waits, and the host replays the draws after the step's wait. Other sampled
// lanes: after a forward that produced a row they draw from, the host waits, draws, and feeds the draw to the next
// forward.
void Engine::draft_trees() {
  std::vector<DraftPass> passes(1);
  std::vector<int> fed_from(lanes_.size(), -1);  // draft_kv index of each lane's first chain token fed
  auto room_for = [&](DraftPass& p) -> DraftPass& {
    if (static_cast<int>(p.batch.size()) < Model::kMaxBatch) return p;
    passes.emplace_back();
    return passes.back();
  };
  for (size_t si = 0; si < specs_.size(); ++si) {
    const Spec& sp = specs_[si];
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
        if (sp.on_device)
          p.dev_drawn.emplace_back(static_cast<int>(p.chain_dst.size()), static_cast<int>(si));
        else if (sp.sampled)
          p.drawn.emplace_back(static_cast<int>(p.chain_dst.size()), static_cast<int>(si));
        p.chain_dst.push_back(sp.sampled ? -1 : tree_slot(sp.lane, 0, false));
        p.alt_dst.push_back(sp.sampled ? -1 : tree_slot(sp.lane, 0, true));
      }
      lane.draft_kv.push_back(id);
    }
  }
  for (int d = 0;; ++d) {  // depth d's chain tokens fed, their picks (draws) are depth d + 1
    DraftPass p;
    p.depth = d;
    for (size_t si = 0; si < specs_.size(); ++si) {
      const Spec& sp = specs_[si];
      if (d + 1 >= sp.depth) continue;
      Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
      if (d == 0) fed_from[static_cast<size_t>(sp.lane)] = static_cast<int>(lane.draft_kv.size());
      const int row = static_cast<int>(p.batch.size());
      p.batch.push_back(BatchToken{0, sp.lane, static_cast<int>(lane.draft_kv.size()), true});
      if (sp.on_device) {  // the chain token from its tree slot, the next one drawn into the next slot
        p.id_from.push_back(tree_slot(sp.lane, d, false));
        p.dev_drawn.emplace_back(row, static_cast<int>(si));
        p.chain_dst.push_back(-1);
        p.alt_dst.push_back(-1);
      } else if (sp.sampled) {
        p.id_from.push_back(-1);
        p.fed.emplace_back(row, static_cast<int>(si));
        p.drawn.emplace_back(row, static_cast<int>(si));
        p.chain_dst.push_back(-1);
        p.alt_dst.push_back(-1);
      } else {
        p.id_from.push_back(tree_slot(sp.lane, d, false));
        p.chain_dst.push_back(tree_slot(sp.lane, d + 1, false));
        p.alt_dst.push_back(tree_slot(sp.lane, d + 1, true));
      }
      lane.draft_kv.push_back(-1);  // the chain id, filled in once the host knows it
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
  const int n_vocab = target_->cfg().n_vocab;
  // Device draws: each drawing lane's generator, then per drawn row (in pass order) its parameters and logits row.
  const size_t S = lanes_.size(), max_rows = S * static_cast<size_t>(max_depth_);
  auto* states_h = reinterpret_cast<uint64_t*>(draw_in_h_);
  auto* params_h = reinterpret_cast<mk_draw_params*>(states_h + S * MK_MT64_WORDS);
  auto* rows_h = reinterpret_cast<int32_t*>(params_h + max_rows);
  size_t n_draws = 0;
  draw_k_ = 0;
  for (Spec& sp : specs_) {
    sp.draws.clear();
    if (!sp.on_device) continue;
    const Sampler& ds = *lanes_[static_cast<size_t>(sp.lane)].job->draft_sampler;
    std::copy(ds.generator().w, ds.generator().w + MK_MT64_WORDS, states_h + static_cast<size_t>(sp.lane) * MK_MT64_WORDS);
    draw_k_ = std::max(draw_k_, ds.candidates(n_vocab));
  }
  std::vector<size_t> first_draw(passes.size());
  for (size_t i = 0; i < passes.size(); ++i) {
    first_draw[i] = n_draws;
    for (const auto& [row, si] : passes[i].dev_drawn) {
      Spec& sp = specs_[static_cast<size_t>(si)];
      const SamplingParams& sq = lanes_[static_cast<size_t>(sp.lane)].job->draft_sampler->params();
      if (n_draws >= max_rows) throw std::runtime_error("engine: device draws exceed their buffer");
      params_h[n_draws] = mk_draw_params{lanes_[static_cast<size_t>(sp.lane)].job->draft_sampler->candidates(n_vocab),
                                         sq.temperature, sq.min_p, sq.top_p, sp.lane,
                                         tree_slot(sp.lane, static_cast<int>(sp.draws.size()), false)};
      rows_h[n_draws] = row;
      sp.draws.push_back(static_cast<int>(n_draws));
      ++n_draws;
    }
  }
  const auto* states_d = draw_in_d_.as<uint64_t>();
  const auto* params_d = reinterpret_cast<const mk_draw_params*>(states_d + S * MK_MT64_WORDS);
  const auto* rows_d = reinterpret_cast<const int32_t*>(params_d + max_rows);
  if (n_draws > 0) ck(mk_copy_async(c, draw_in_d_.p, draw_in_h_, draw_block_bytes(S, max_rows)));
  for (size_t i = 0; i < passes.size(); ++i) {
    DraftPass& p = passes[i];
    if (p.batch.empty()) continue;
    for (const auto& [b, si] : p.fed) p.batch[static_cast<size_t>(b)].id = specs_[static_cast<size_t>(si)].chain[static_cast<size_t>(p.depth)];
    const int m = static_cast<int>(p.chain_dst.size());
    draft_->enqueue(p.batch.data(), static_cast<int>(p.batch.size()), p.id_from.data(), tree, draft_top1_.as<int32_t>(),
                    draft_top2_.as<int32_t>());
    int32_t* dst = plan_.as<int32_t>() + at[i];
    ck(mk_move_ids(c, tree, dst, draft_top1_.as<int32_t>(), nullptr, m));
    ck(mk_move_ids(c, tree, dst + m, draft_top2_.as<int32_t>(), nullptr, m));
    if (!p.dev_drawn.empty()) {  // top-k of the drawing rows, then each row's draw into its lane's next tree slot
      const size_t j = first_draw[i];
      const int nr = static_cast<int>(p.dev_drawn.size());
      float* cv = cand_v_d_.as<float>() + j * static_cast<size_t>(draw_k_);
      int32_t* ci = cand_i_d_.as<int32_t>() + j * static_cast<size_t>(draw_k_);
      ck(mk_topk(c, draft_->dev_logits(), n_vocab, rows_d + j, nr, n_vocab, draw_k_, cv, ci));
      ck(mk_sample_draw(c, cv, ci, draw_k_, nr, params_d + j, const_cast<uint64_t*>(states_d), static_cast<int>(S),
                        tree, static_cast<int>(tree_.bytes / sizeof(int32_t))));
    }
    if (p.drawn.empty()) continue;
    // Sampled lanes: the draft sampler's distribution of each row, one wait, then the draws (engine.cpp:319-323).
    draft_sel_.clear();
    for (const auto& [row, si] : p.drawn) {
      const Job& job = *lanes_[static_cast<size_t>(specs_[static_cast<size_t>(si)].lane)].job;
      draft_sel_.add(row, *job.draft_sampler, pen_ids_, pen_amts_);
    }
    draft_sel_.enqueue(draft_->dev_logits());
    ck(mk_synchronize(c));
    draft_->check_device();
    draft_sel_.collect();
    for (size_t j = 0; j < p.drawn.size(); ++j) {
      Spec& sp = specs_[static_cast<size_t>(p.drawn[j].second)];
      Sampler& ds = *lanes_[static_cast<size_t>(sp.lane)].job->draft_sampler;
      const int r = static_cast<int>(j);
      sp.q.emplace_back();
      ds.finish(draft_sel_, r, sp.q.back());
      sp.chain.push_back(ds.draw(sp.q.back()));
    }
  }
  if (n_draws > 0) {  // the candidates of every device draw, for the host's replay after the step's wait
    const size_t n = n_draws * static_cast<size_t>(draw_k_);
    ck(mk_copy_async(c, cand_v_h_, cand_v_d_.p, n * sizeof(float)));
    ck(mk_copy_async(c, cand_i_h_, cand_i_d_.p, n * sizeof(int32_t)));
  }
  // Remember where each lane's chain tokens sit in draft_kv (greedy ones and device draws filled in after the step's
  // wait).
  for (Spec& sp : specs_) {
    sp.root = fed_from[static_cast<size_t>(sp.lane)];
    if (!sp.sampled || sp.on_device || sp.root < 0) continue;
    Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
    for (int d = 0; d + 1 < sp.depth; ++d) lane.draft_kv[static_cast<size_t>(sp.root + d)] = sp.chain[static_cast<size_t>(d)];
  }
}

// Decoding lanes' pending tokens and drafts, then prompt tokens; returns the number of decode rows.
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
      if (sp.on_device) {  // a chain in a row, its ids in the tree slots the device drew them into
        batch_.push_back(BatchToken{0, sp.lane, P + 1 + d, true});
        id_from_.push_back(tree_slot(sp.lane, d, false));
        continue;
      }
      if (sp.sampled) {  // a chain in a row: ordinary causal tokens
        batch_.push_back(BatchToken{sp.chain[static_cast<size_t>(d)], sp.lane, P + 1 + d, true});
        id_from_.push_back(-1);
        continue;
      }
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

// Candidates of the target rows whose penalties the host knows before the step's wait: sampled lanes' rows (the
// path to row i is the chain before it), penalized greedy lanes without a tree, and finished prompts of non-plain
// requests.
void Engine::select_known_rows(int decode_rows) {
  const int n_vocab = target_->cfg().n_vocab;
  sel_.clear();
  for (Spec& sp : specs_) {
    const Job& job = *lanes_[static_cast<size_t>(sp.lane)].job;
    if (job.plain || (!sp.sampled && sp.depth > 0)) continue;
    sp.cand = &sel_;
    const int rows = sp.sampled ? sp.depth + 1 : 1;
    for (int i = 0; i < rows; ++i) {
      pen_ids_.clear();
      pen_amts_.clear();
      job.sampler->penalties(sp.chain.data(), i, pen_ids_, pen_amts_);
      const int at = sel_.add(sp.root + i, *job.sampler, pen_ids_, pen_amts_);
      if (i == 0) sp.sel = at;
    }
  }
  finishing_sel_.assign(finishing_lanes_.size(), -1);
  for (size_t j = 0; j < finishing_lanes_.size(); ++j) {
    const Job& job = *lanes_[static_cast<size_t>(finishing_lanes_[j])].job;
    if (job.plain) continue;
    pen_ids_.clear();
    pen_amts_.clear();
    job.sampler->penalties(nullptr, 0, pen_ids_, pen_amts_);
    finishing_sel_[j] = sel_.add(decode_rows + static_cast<int>(j), *job.sampler, pen_ids_, pen_amts_);
  }
  pen_ids_.clear();
  pen_amts_.clear();
}

// Penalized greedy trees: every node's row with the penalties of its path (chain tokens above it, then itself),
// known once the tree is on the host. One more wait.
void Engine::select_tree_rows() {
  tree_sel_.clear();
  for (Spec& sp : specs_) {
    const Job& job = *lanes_[static_cast<size_t>(sp.lane)].job;
    if (job.plain || sp.sampled || sp.depth == 0) continue;
    sp.cand = &tree_sel_;
    const int32_t* tree = tree_host(sp.lane);
    std::vector<int32_t> path;
    for (int node = 0; node < 1 + 2 * sp.depth; ++node) {
      path.clear();
      if (node > 0) {
        const int d = (node - 1) / 2;  // depth of the node; chain nodes are odd
        for (int e = 0; e < d; ++e) path.push_back(tree[2 * e]);
        path.push_back(tree[2 * d + (node % 2 == 1 ? 0 : 1)]);
      }
      pen_ids_.clear();
      pen_amts_.clear();
      job.sampler->penalties(path.data(), static_cast<int>(path.size()), pen_ids_, pen_amts_);
      const int at = tree_sel_.add(sp.root + node, 1, pen_ids_, pen_amts_);
      if (node == 0) sp.sel = at;
    }
  }
  pen_ids_.clear();
  pen_amts_.clear();
  if (tree_sel_.empty()) return;
  tree_sel_.enqueue(target_->dev_logits());
  ck(mk_synchronize(target_->ctx()));
  target_->check_device();
  tree_sel_.collect();
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
  select_known_rows(decode_rows);
  sel_.enqueue(target_->dev_logits());
  const int rows = target_->n_out();
  ck(mk_copy_async(c, picks_h_, target_top_.p, static_cast<size_t>(rows) * sizeof(int32_t)));
  if (drafting) ck(mk_copy_async(c, tree_h_, tree_.p, lanes_.size() * 2 * max_depth_ * sizeof(int32_t)));
  ck(mk_synchronize(c));  // the step's one host wait
  target_->check_device();
  if (draft_) draft_->check_device();
  ++steps_;
  sel_.collect();

  if (drafting) replay_draws();
  if (drafting)  // the greedy chain ids and device-drawn drafts fed to the draft, now known on the host
    for (size_t i = 0; i < specs_.size(); ++i) {
      const Spec& sp = specs_[i];
      if (chain_at[i] < 0 || (sp.sampled && !sp.on_device)) continue;
      Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
      for (int d = 0; d + 1 < sp.depth; ++d)
        lane.draft_kv[static_cast<size_t>(chain_at[i] + d)] = tree_host(sp.lane)[2 * d];
    }
  select_tree_rows();
  for (int t = decode_rows; t < n; ++t) lanes_[static_cast<size_t>(batch_[t].seq)].kv.push_back(batch_[t].id);
  for (size_t j = 0; j < finishing_lanes_.size(); ++j) {  // prompts that finished: their first token
    Lane& lane = lanes_[static_cast<size_t>(finishing_lanes_[j])];
    Job& job = *lane.job;
    job.first_token = Clock::now();
    job.res->prefill_ms = ms_between(job.admitted, job.first_token);
    job.decoding = true;
    if (job.plain) {
      job.pending = picks_h_[decode_rows + static_cast<int>(j)];
    } else {
      const int r = finishing_sel_[j];
      job.sampler->finish(sel_, r, dist_);
      job.pending = job.sampler->draw(dist_);
    }
    if (!emit(job, job.pending, lane.kv.size())) finish(lane);
  }
  for (const Spec& sp : specs_) {
    if (sp.sampled)
      settle_sampled(sp);
    else
      settle(sp);
  }
}

// Sampled lanes whose drafts the device drew: the draft sampler's distribution of each draw's candidates and its draw
// with the host's generator, in depth order (the reference's draws, engine.cpp:319-323), leaving the host generator
// where the reference's is. The drafts are the device's picks, which the target has verified already; a replay that
// picks differently (a device weight one ulp off the C library's expf) is counted, and the next step's draws start
// again from the host generator.
void Engine::replay_draws() {
  const int n_vocab = target_->cfg().n_vocab;
  for (Spec& sp : specs_) {
    if (!sp.on_device) continue;
    Sampler& ds = *lanes_[static_cast<size_t>(sp.lane)].job->draft_sampler;
    const int k = ds.candidates(n_vocab);
    if (static_cast<int>(sp.draws.size()) != sp.depth) throw std::logic_error("engine: device draws missing");
    for (int d = 0; d < sp.depth; ++d) {
      const size_t j = static_cast<size_t>(sp.draws[static_cast<size_t>(d)]) * static_cast<size_t>(draw_k_);
      sp.q.emplace_back();
      ds.finish(cand_v_h_ + j, cand_i_h_ + j, k, sp.q.back());
      const int32_t host = ds.draw(sp.q.back());
      const int32_t dev = tree_host(sp.lane)[2 * d];
      ++device_draws_;
      if (host != dev) ++draw_mismatches_;
      sp.chain.push_back(dev);
    }
  }
}

// The target's greedy pick at tree node `node` of a lane: the device's first maximum, or for a penalized request
// the first maximum of the penalized row.
int32_t Engine::target_pick(const Spec& sp, int node) const {
  if (!sp.cand) return picks_h_[sp.root + node];
  return sp.cand->ids(sp.sel + node)[0];
}

// The request sampler's distribution of target row `row` (0 = the pending token's) of a non-plain lane.
Distribution& Engine::target_dist(const Spec& sp, int row) {
  const Sampler& s = *lanes_[static_cast<size_t>(sp.lane)].job->sampler;
  const int r = sp.sel + row;
  s.finish(*sp.cand, r, dist_);
  return dist_;
}

// The acceptance walk of one greedy lane over the target's picks (rows root.. of this step).
void Engine::settle(const Spec& sp) {
  Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
  Job& job = *lane.job;
  const int P = static_cast<int>(lane.kv.size());
  lane.kv.push_back(job.pending);
  job.res->drafted += sp.depth;
  bool alive = true, missed = false;
  int node = 0, held = 0;  // tree node the walk stands on (0 = the pending token), draft depths accepted
  const int32_t* tree = tree_host(sp.lane);
  for (int d = 0; d < sp.depth; ++d) {
    const int32_t want = target_pick(sp, node);
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
  if (alive && !missed) job.pending = target_pick(sp, node);
  if (sp.depth > 0) {
    if (held == sp.depth && sp.depth == job.k && node == 2 * sp.depth - 1)
      job.k = std::min(job.k + 1, max_depth_);
    else if (2 * held < sp.depth)
      job.k = std::max(1, job.k - 1);
  }
  if (alive) alive = emit(job, job.pending, lane.kv.size());
  if (!alive) finish(lane);
}

// A sampled lane: each draft d_i verified against the target's distribution at its row (the rows sit at KV rows
// P + 1 + i already, so nothing moves); a rejection's replacement, or a draw from the row after a fully accepted
// chain, is the next pending token.
void Engine::settle_sampled(const Spec& sp) {
  Lane& lane = lanes_[static_cast<size_t>(sp.lane)];
  Job& job = *lane.job;
  Sampler& s = *job.sampler;
  lane.kv.push_back(job.pending);
  job.res->drafted += sp.depth;
  bool alive = true;
  int held = 0;  // drafts accepted
  while (held < sp.depth) {
    bool ok = false;
    const int32_t t = s.verify(target_dist(sp, held), sp.q[static_cast<size_t>(held)], sp.chain[static_cast<size_t>(held)], ok);
    if (!ok) {
      job.pending = t;
      break;
    }
    ++job.res->accepted;
    lane.kv.push_back(t);
    alive = emit(job, t, lane.kv.size());
    if (!alive) break;
    ++held;
  }
  if (alive && held == sp.depth) job.pending = s.draw(target_dist(sp, sp.depth));
  if (sp.depth > 0) {
    if (held == sp.depth && sp.depth == job.k)
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
  job.sampler->accept(id);
  job.res->tokens.push_back(id);
  ++job.res->completion_tokens;
  if (job.res->completion_tokens >= job.budget) return false;
  return static_cast<int>(cached) + 1 < target_->n_ctx();
}

void Engine::finish(Lane& lane) {
  Job& job = *lane.job;
  job.res->decode_ms = job.decoding ? ms_between(job.first_token, Clock::now()) : 0.0;
  job.res->done = true;
  lane.job.reset();
  --busy_;
}

}  // namespace malkin_hip
