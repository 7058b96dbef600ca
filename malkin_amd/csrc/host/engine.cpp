#include "engine.h"

#include <algorithm>
#include <stdexcept>

namespace malkin_hip {

namespace {

double ms_between(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
  return std::chrono::duration<double, std::milli>(b - a).count();
}

}  // namespace

Engine::Engine(Model* target, Model* draft, int n_draft) : model_(target), draft_(draft) {
  if (!model_) throw std::invalid_argument("engine: no target model");
  if (draft_) {
    if (draft_->cfg().n_vocab != model_->cfg().n_vocab)
      throw std::runtime_error("draft model tokenizer differs from the target");  // engine.cpp:121
    if (draft_->n_seq() < model_->n_seq()) throw std::invalid_argument("engine: draft has fewer sequences");
    if (draft_->n_ctx() < model_->n_ctx()) throw std::invalid_argument("engine: draft context is shorter");
  }
  if (n_draft > 0) n_draft_ = std::min(n_draft, Model::kMaxBatch - 1);  // engine.cpp:126
  slots_.resize(static_cast<size_t>(model_->n_seq()));
  top1_.resize(Model::kMaxBatch);
  dtop1_.resize(Model::kMaxBatch);
  dtop2_.resize(Model::kMaxBatch);
  dslot1_.resize(slots_.size());
  dslot2_.resize(slots_.size());
}

int Engine::submit(const EngineRequest& req) {
  const int n_ctx = model_->n_ctx();
  if (req.prompt.empty()) throw std::invalid_argument("empty prompt");  // engine.cpp:227-232
  if (static_cast<int>(req.prompt.size()) >= n_ctx)
    throw std::invalid_argument("prompt has " + std::to_string(req.prompt.size()) + " tokens, context is " +
                                std::to_string(n_ctx));
  for (int32_t id : req.prompt)
    if (id < 0 || id >= model_->cfg().n_vocab) throw std::invalid_argument("prompt token id out of range");
  results_.push_back(std::make_unique<EngineResult>());
  auto r = std::make_unique<Request>();
  r->req = req;
  r->res = results_.back().get();
  r->budget = req.max_tokens > 0 ? req.max_tokens : n_ctx;
  r->t0 = Clock::now();
  pending_.push_back(std::move(r));
  return static_cast<int>(results_.size()) - 1;
}

const EngineResult& Engine::result(int id) const {
  if (id < 0 || id >= static_cast<int>(results_.size())) throw std::invalid_argument("engine: bad request id");
  return *results_[static_cast<size_t>(id)];
}

int Engine::step_once() {
  // engine.cpp:200-215: take as many pending requests as there are idle slots, then step the busy ones.
  const size_t take = std::min(pending_.size(), slots_.size() - static_cast<size_t>(busy_));
  for (size_t i = 0; i < take; ++i) admit(std::move(pending_[i]));
  pending_.erase(pending_.begin(), pending_.begin() + static_cast<std::ptrdiff_t>(take));
  if (busy_ > 0) step();
  return busy_;
}

void Engine::run() {
  while (!pending_.empty() || busy_ > 0) step_once();
}

void Engine::admit(std::unique_ptr<Request> r) {
  const auto& prompt = r->req.prompt;
  int best = -1;
  size_t best_common = 0;
  for (int i = 0; i < static_cast<int>(slots_.size()); ++i) {
    const Slot& s = slots_[static_cast<size_t>(i)];
    if (s.req) continue;
    size_t c = 0;
    while (c < s.cache.size() && c < prompt.size() && s.cache[c] == prompt[c]) ++c;
    if (best < 0 || c > best_common || (c == best_common && s.used < slots_[static_cast<size_t>(best)].used)) {
      best = i;
      best_common = c;
    }
  }
  Slot& s = slots_[static_cast<size_t>(best)];
  best_common = std::min(best_common, prompt.size() - 1);
  s.cache.resize(best_common);
  r->res->prompt_tokens = static_cast<int>(prompt.size());
  r->res->cached_tokens = static_cast<int>(best_common);
  r->res->finish_reason = "length";
  s.used = ++admitted_;
  r->k = std::min(4, n_draft_);
  s.req = std::move(r);
  ++busy_;
}

bool Engine::plan_drafts() {
  const int n_ctx = model_->n_ctx();
  props_.clear();
  for (size_t i = 0; i < slots_.size(); ++i) {
    if (!slots_[i].req || !slots_[i].req->decoding) continue;
    props_.emplace_back();
    props_.back().seq = static_cast<int>(i);
  }
  if (!draft_ || props_.empty()) return false;
  const int nd = static_cast<int>(props_.size());
  bool drafting = false;
  for (Proposal& p : props_) {
    const Slot& s = slots_[static_cast<size_t>(p.seq)];
    const Request& q = *s.req;
    const int left = q.budget - q.res->completion_tokens;
    const int room = n_ctx - static_cast<int>(s.cache.size()) - 2;
    const int cap = Model::kMaxBatch / nd - 1;  // tokens per slot after its next token
    p.kk = std::max(0, std::min({q.k, left, room / 2, cap / 2}));  // greedy trees: two tokens per draft position
    drafting = drafting || p.kk > 0;
  }
  return drafting;
}

void Engine::propose() {
  // One draft pass over dbatch_: the greedy picks of its logits rows are kept per slot (the last row of a slot wins).
  auto flush = [&] {
    if (dbatch_.empty()) return;
    draft_->forward_top2(dbatch_.data(), static_cast<int>(dbatch_.size()), dtop1_.data(), dtop2_.data());
    int row = 0;
    for (const BatchToken& b : dbatch_) {
      if (!b.logits) continue;
      dslot1_[static_cast<size_t>(b.seq)] = dtop1_[static_cast<size_t>(row)];
      dslot2_[static_cast<size_t>(b.seq)] = dtop2_[static_cast<size_t>(row)];
      ++row;
    }
    dbatch_.clear();
  };
  // Catch up: the draft's KV of each proposing slot to its cached tokens plus next, reusing the common prefix.
  for (const Proposal& p : props_) {
    if (p.kk == 0) continue;
    Slot& s = slots_[static_cast<size_t>(p.seq)];
    const size_t len = s.cache.size() + 1;
    size_t common = 0;
    while (common < s.dcache.size() && common < s.cache.size() && s.dcache[common] == s.cache[common]) ++common;
    if (common == s.cache.size() && common < s.dcache.size() && s.dcache[common] == s.req->next) ++common;
    common = std::min(common, len - 1);  // the last token is evaluated for its logits
    s.dcache.resize(common);
    for (size_t pos = common; pos < len; ++pos) {
      const int32_t id = pos < s.cache.size() ? s.cache[pos] : s.req->next;
      dbatch_.push_back({id, p.seq, static_cast<int>(pos), pos + 1 == len});
      s.dcache.push_back(id);
      if (static_cast<int>(dbatch_.size()) == Model::kMaxBatch) flush();
    }
  }
  flush();
  // Rounds: each slot takes its chain token (top-1) and alternative (runner-up), then all feed the chain in one pass.
  for (int i = 0;; ++i) {
    bool more = false;
    for (Proposal& p : props_) {
      if (i >= p.kk) continue;
      Slot& s = slots_[static_cast<size_t>(p.seq)];
      const int32_t a = dslot1_[static_cast<size_t>(p.seq)];
      p.chain.push_back(a);
      p.alt.push_back(dslot2_[static_cast<size_t>(p.seq)]);
      if (i + 1 < p.kk) {
        dbatch_.push_back({a, p.seq, static_cast<int>(s.dcache.size()), true});
        s.dcache.push_back(a);
        more = true;
      }
    }
    flush();
    if (!more) break;
  }
}

int Engine::build_batch() {
  batch_.clear();
  batch_seq_.clear();
  for (Proposal& p : props_) {
    const Slot& s = slots_[static_cast<size_t>(p.seq)];
    const int P = static_cast<int>(s.cache.size());
    p.root = static_cast<int>(batch_.size());
    batch_.push_back({s.req->next, p.seq, P, true});
    for (int i = 0; i < p.kk; ++i) {
      const int par = i == 0 ? p.root : p.root + 2 * i - 1;
      batch_.push_back({p.chain[static_cast<size_t>(i)], p.seq, P + 1 + i, true, P + 1 + 2 * i, par});
      batch_.push_back({p.alt[static_cast<size_t>(i)], p.seq, P + 1 + i, true, P + 2 + 2 * i, par});
    }
  }
  const int decode_rows = static_cast<int>(batch_.size());
  for (size_t i = 0; i < slots_.size(); ++i) {  // prompt chunks in slot order, up to kMaxBatch tokens
    const Slot& s = slots_[i];
    if (!s.req || s.req->decoding) continue;
    const auto& prompt = s.req->req.prompt;
    const int from = static_cast<int>(s.cache.size());
    const int take =
        std::min(Model::kMaxBatch - static_cast<int>(batch_.size()), static_cast<int>(prompt.size()) - from);
    for (int pos = from; pos < from + take; ++pos) {
      const bool last = pos + 1 == static_cast<int>(prompt.size());
      batch_.push_back({prompt[static_cast<size_t>(pos)], static_cast<int>(i), pos, last});
      if (last) batch_seq_.push_back(static_cast<int>(i));
    }
  }
  return decode_rows;
}

void Engine::step() {
  if (plan_drafts()) propose();
  const int decode_rows = build_batch(), n = static_cast<int>(batch_.size());
  if (n == 0) return;
  model_->forward_top2(batch_.data(), n, top1_.data(), nullptr);
  for (int t = decode_rows; t < n; ++t)
    slots_[static_cast<size_t>(batch_[static_cast<size_t>(t)].seq)].cache.push_back(batch_[static_cast<size_t>(t)].id);
  // Prompts that finished: their first token.
  for (size_t j = 0; j < batch_seq_.size(); ++j) {
    Slot& s = slots_[static_cast<size_t>(batch_seq_[j])];
    Request& q = *s.req;
    q.t1 = Clock::now();
    q.res->prefill_ms = ms_between(q.t0, q.t1);
    q.decoding = true;
    q.next = top1_[static_cast<size_t>(decode_rows) + j];
    if (!emit(q, q.next, s.cache.size())) finish(s);
  }
  for (const Proposal& p : props_) accept(p);
}

void Engine::accept(const Proposal& p) {
  Slot& s = slots_[static_cast<size_t>(p.seq)];
  Request& q = *s.req;
  const int P = static_cast<int>(s.cache.size());
  s.cache.push_back(q.next);
  q.res->drafted += p.kk;
  bool go = true;
  if (p.kk == 0)
    q.next = top1_[static_cast<size_t>(p.root)];
  else
    go = accept_greedy(p, s, P);
  if (go) go = emit(q, q.next, s.cache.size());
  if (!go) finish(s);
}

bool Engine::accept_greedy(const Proposal& p, Slot& s, int P) {
  Request& q = *s.req;
  auto pick = [&](int node) { return top1_[static_cast<size_t>(p.root + node)]; };
  int cur = 0, done = 0;  // tree node reached, draft positions settled
  bool go = true, bonus = false;
  for (int i = 0; i < p.kk; ++i) {
    const int32_t a = pick(cur);
    int node = -1;
    if (a == p.chain[static_cast<size_t>(i)])
      node = 1 + 2 * i;
    else if (a == p.alt[static_cast<size_t>(i)])
      node = 2 + 2 * i;
    if (node < 0) {
      q.next = a;
      bonus = true;
      break;
    }
    model_->move_kv(P + node, static_cast<int>(s.cache.size()), p.seq);
    s.cache.push_back(a);
    ++q.res->accepted;
    cur = node;
    go = emit(q, a, s.cache.size());
    if (!go) break;
    done = i + 1;
    if (node == 2 + 2 * i) break;  // an alternative is a leaf
  }
  if (go && !bonus) q.next = pick(cur);
  if (done == p.kk && p.kk == q.k && cur == 2 * p.kk - 1)
    q.k = std::min(q.k + 1, n_draft_);
  else if (2 * done < p.kk)
    q.k = std::max(1, q.k - 1);
  return go;
}

bool Engine::emit(Request& q, int32_t id, size_t cached) {
  if (std::find(q.req.eog.begin(), q.req.eog.end(), id) != q.req.eog.end()) {
    q.res->finish_reason = "stop";
    return false;
  }
  q.res->tokens.push_back(id);
  ++q.res->completion_tokens;
  if (q.res->completion_tokens >= q.budget) return false;
  return static_cast<int>(cached) + 1 < model_->n_ctx();
}

void Engine::finish(Slot& s) {
  Request& q = *s.req;
  q.res->decode_ms = ms_between(q.t1, Clock::now());
  q.res->done = true;
  s.req.reset();
  --busy_;
}

}  // namespace malkin_hip
