#include "sampler.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace malkin_hip {

namespace {

void ck(int rc) {
  if (rc != MK_OK) throw std::runtime_error(mk_last_error());
}

// The device top-k's order on floats: larger key = larger value (+0 above -0).
uint32_t order_key(float f) {
  uint32_t u;
  std::memcpy(&u, &f, sizeof(u));
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

float prob_in(const Distribution& d, int32_t id) {
  for (const Candidate& c : d)
    if (c.id == id) return c.p;
  return 0.0f;
}

}  // namespace

Sampler::Sampler(const SamplingParams& params, bool penalties)
    : p_(params), penalties_(penalties), rng_(params.seed ? params.seed : std::random_device{}()) {}

int Sampler::candidates(int n_vocab) const {
  if (greedy()) return 1;
  return p_.top_k > 0 ? std::min(p_.top_k, n_vocab) : n_vocab;
}

void Sampler::penalties(const int32_t* path, int n_path, std::vector<int32_t>& ids,
                        std::vector<float>& amounts) const {
  if (!penalizes()) return;
  auto amount = [&](int seen) { return std::fmaf(p_.frequency_penalty, static_cast<float>(seen), p_.presence_penalty); };
  // Path tokens first (their counts include the path's own occurrences), then the counted tokens the path misses.
  std::vector<std::pair<int32_t, int>> extra;
  for (int i = 0; i < n_path; ++i) {
    auto it = std::find_if(extra.begin(), extra.end(), [&](const auto& e) { return e.first == path[i]; });
    if (it == extra.end())
      extra.emplace_back(path[i], 1);
    else
      ++it->second;
  }
  for (const auto& [id, more] : extra) {
    const auto c = counts_.find(id);
    ids.push_back(id);
    amounts.push_back(amount((c == counts_.end() ? 0 : c->second) + more));
  }
  for (const auto& [id, seen] : counts_) {
    if (std::any_of(extra.begin(), extra.end(), [&](const auto& e) { return e.first == id; })) continue;
    ids.push_back(id);
    amounts.push_back(amount(seen));
  }
}

void Sampler::finish(const float* values, const int32_t* ids, int n, Distribution& out) const {
  out.clear();
  if (n <= 0) throw std::invalid_argument("sampler: no candidates");
  if (greedy()) {
    out.push_back(Candidate{1.0f, ids[0]});
    return;
  }
  const float top = values[0];
  weights_.resize(static_cast<size_t>(n));
  double all = 0.0;
  for (int i = 0; i < n; ++i) {
    const float w = std::exp((values[i] - top) / p_.temperature);
    weights_[static_cast<size_t>(i)] = w;
    all += w;
  }
  // Keep the head: min-p floor relative to the first weight, then the nucleus (the candidate that reaches top_p of
  // the total is kept).
  const double floor_w = static_cast<double>(p_.min_p) * weights_[0];
  const double nucleus = static_cast<double>(p_.top_p) * all;
  double run = 0.0;
  int keep = 0;
  while (keep < n) {
    const double w = weights_[static_cast<size_t>(keep)];
    if (keep > 0 && w < floor_w) break;
    run += w;
    ++keep;
    if (run >= nucleus) break;
  }
  keep = std::max(keep, 1);
  double kept = 0.0;
  for (int i = 0; i < keep; ++i) kept += weights_[static_cast<size_t>(i)];
  out.reserve(static_cast<size_t>(keep));
  for (int i = 0; i < keep; ++i)
    out.push_back(Candidate{static_cast<float>(weights_[static_cast<size_t>(i)] / kept), ids[i]});
}

double Sampler::uniform() { return std::uniform_real_distribution<double>(0.0, 1.0)(rng_); }

int32_t Sampler::draw(const Distribution& d) {
  if (d.empty()) throw std::invalid_argument("sampler: empty distribution");
  if (d.size() == 1) return d[0].id;
  double u = uniform();
  for (const Candidate& c : d) {
    u -= c.p;
    if (u <= 0.0) return c.id;
  }
  return d.back().id;
}

int32_t Sampler::verify(const Distribution& p, const Distribution& q, int32_t draft, bool& accepted) {
  const float pd = prob_in(p, draft), qd = prob_in(q, draft);
  const double u = uniform();
  accepted = qd > 0.0f && u * qd < pd;
  if (accepted) return draft;
  Distribution excess;
  double total = 0.0;
  for (const Candidate& c : p) {
    const float r = c.p - prob_in(q, c.id);
    if (r > 0.0f) {
      excess.push_back(Candidate{r, c.id});
      total += r;
    }
  }
  if (excess.empty()) return draw(p);
  for (Candidate& c : excess) c.p = static_cast<float>(c.p / total);
  return draw(excess);
}

// ---- Selector ----

Selector::Selector(mk_ctx* ctx, int n_vocab) : ctx_(ctx), n_vocab_(n_vocab) {}

Selector::~Selector() {
  (void)mk_host_free(ctx_, in_h_);
  (void)mk_host_free(ctx_, out_v_h_);
  (void)mk_host_free(ctx_, out_i_h_);
  (void)mk_host_free(ctx_, full_h_);
}

void Selector::clear() {
  reqs_.clear();
  pen_off_.assign(1, 0);
  pen_id_.clear();
  pen_amt_.clear();
  k_max_ = 0;
  n_full_ = 0;
}

int Selector::add(int row, int k, const std::vector<int32_t>& pen_ids, const std::vector<float>& pen_amounts) {
  if (k < 1 || k > n_vocab_) throw std::invalid_argument("selector: bad candidate count");
  if (pen_ids.size() != pen_amounts.size()) throw std::invalid_argument("selector: penalty lists differ in length");
  if (pen_off_.empty()) pen_off_.assign(1, 0);
  Req r{row, k, -1};
  if (k > kMaxDeviceK)
    r.full = n_full_++;
  else
    k_max_ = std::max(k_max_, k);
  reqs_.push_back(r);
  pen_id_.insert(pen_id_.end(), pen_ids.begin(), pen_ids.end());
  pen_amt_.insert(pen_amt_.end(), pen_amounts.begin(), pen_amounts.end());
  pen_off_.push_back(static_cast<int32_t>(pen_id_.size()));
  return static_cast<int>(reqs_.size()) - 1;
}

void Selector::reserve_host(size_t words) {
  if (words <= in_words_) return;
  const size_t want = std::max(words, 2 * in_words_);
  (void)mk_host_free(ctx_, in_h_);
  in_h_ = nullptr;
  void* h = nullptr;
  ck(mk_host_alloc(ctx_, want * sizeof(int32_t), &h));
  in_h_ = static_cast<int32_t*>(h);
  in_d_ = DevBuf(ctx_, want * sizeof(int32_t));
  in_words_ = want;
}

void Selector::reserve_out(size_t rows, int k) {
  const size_t need = rows * static_cast<size_t>(k);
  if (need <= out_cap_) return;
  const size_t want = std::max(need, 2 * out_cap_);
  (void)mk_host_free(ctx_, out_v_h_);
  (void)mk_host_free(ctx_, out_i_h_);
  out_v_h_ = nullptr;
  out_i_h_ = nullptr;
  void* h = nullptr;
  ck(mk_host_alloc(ctx_, want * sizeof(float), &h));
  out_v_h_ = static_cast<float*>(h);
  ck(mk_host_alloc(ctx_, want * sizeof(int32_t), &h));
  out_i_h_ = static_cast<int32_t*>(h);
  out_v_d_ = DevBuf(ctx_, want * sizeof(float));
  out_i_d_ = DevBuf(ctx_, want * sizeof(int32_t));
  out_cap_ = want;
}

void Selector::reserve_full(size_t rows) {
  if (rows <= full_rows_) return;
  (void)mk_host_free(ctx_, full_h_);
  full_h_ = nullptr;
  void* h = nullptr;
  ck(mk_host_alloc(ctx_, rows * static_cast<size_t>(n_vocab_) * sizeof(float), &h));
  full_h_ = static_cast<float*>(h);
  full_rows_ = rows;
}

void Selector::enqueue(float* dev_logits) {
  const size_t n = reqs_.size();
  if (n == 0) return;
  // One upload: rows [n], pen_off [n + 1], pen_id [m], pen_amt [m].
  const size_t m = pen_id_.size(), words = n + (n + 1) + 2 * m;
  reserve_host(words);
  int32_t* h = in_h_;
  for (size_t i = 0; i < n; ++i) h[i] = reqs_[i].row;
  std::copy(pen_off_.begin(), pen_off_.end(), h + n);
  std::copy(pen_id_.begin(), pen_id_.end(), h + 2 * n + 1);
  std::memcpy(h + 2 * n + 1 + m, pen_amt_.data(), m * sizeof(float));
  ck(mk_copy_async(ctx_, in_d_.p, h, words * sizeof(int32_t)));
  const int32_t* d = in_d_.as<int32_t>();
  const int64_t stride = n_vocab_;
  if (m > 0)
    ck(mk_penalize(ctx_, dev_logits, stride, d, static_cast<int>(n), n_vocab_, d + n, d + 2 * n + 1,
                   reinterpret_cast<const float*>(d + 2 * n + 1 + m)));
  out_k_ = k_max_;
  if (k_max_ > 0) {
    reserve_out(n, k_max_);
    ck(mk_topk(ctx_, dev_logits, stride, d, static_cast<int>(n), n_vocab_, k_max_, out_v_d_.as<float>(),
               out_i_d_.as<int32_t>()));
    ck(mk_copy_async(ctx_, out_v_h_, out_v_d_.p, n * static_cast<size_t>(k_max_) * sizeof(float)));
    ck(mk_copy_async(ctx_, out_i_h_, out_i_d_.p, n * static_cast<size_t>(k_max_) * sizeof(int32_t)));
  }
  if (n_full_ > 0) {
    reserve_full(static_cast<size_t>(n_full_));
    for (const Req& r : reqs_)
      if (r.full >= 0)
        ck(mk_copy_async(ctx_, full_h_ + static_cast<size_t>(r.full) * n_vocab_,
                         dev_logits + static_cast<int64_t>(r.row) * stride, n_vocab_ * sizeof(float)));
  }
}

void Selector::collect() {
  full_ids_.resize(static_cast<size_t>(n_full_));
  full_vals_.resize(static_cast<size_t>(n_full_));
  for (const Req& r : reqs_) {
    if (r.full < 0) continue;
    const float* l = full_h_ + static_cast<size_t>(r.full) * n_vocab_;
    std::vector<int32_t>& ids = full_ids_[static_cast<size_t>(r.full)];
    ids.resize(static_cast<size_t>(n_vocab_));
    for (int i = 0; i < n_vocab_; ++i) ids[static_cast<size_t>(i)] = i;
    // Highest first, equal values by lower id (the device top-k's order).
    auto before = [&](int32_t a, int32_t b) {
      const uint32_t ka = order_key(l[a]), kb = order_key(l[b]);
      return ka > kb || (ka == kb && a < b);
    };
    std::partial_sort(ids.begin(), ids.begin() + r.k, ids.end(), before);
    ids.resize(static_cast<size_t>(r.k));
    std::vector<float>& v = full_vals_[static_cast<size_t>(r.full)];
    v.resize(static_cast<size_t>(r.k));
    for (int i = 0; i < r.k; ++i) v[static_cast<size_t>(i)] = l[ids[static_cast<size_t>(i)]];
  }
}

const float* Selector::values(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  if (r.full >= 0) return full_vals_[static_cast<size_t>(r.full)].data();
  return out_v_h_ + static_cast<size_t>(i) * out_k_;
}

const int32_t* Selector::ids(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  if (r.full >= 0) return full_ids_[static_cast<size_t>(r.full)].data();
  return out_i_h_ + static_cast<size_t>(i) * out_k_;
}

}  // namespace malkin_hip
