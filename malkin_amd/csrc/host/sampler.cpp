#include "sampler.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <stdexcept>

namespace malkin_hip {

namespace {

void ck(int rc) {
  if (rc != MK_OK) throw std::runtime_error(mk_last_error());
}

float prob_in(const Distribution& d, int32_t id) {
  for (const Candidate& c : d)
    if (c.id == id) return c.p;
  return 0.0f;
}

}  // namespace

Mt64::Mt64(uint64_t seed) {
  w[0] = seed;
  for (int i = 1; i < kN; ++i) w[i] = 6364136223846793005ull * (w[i - 1] ^ (w[i - 1] >> 62)) + static_cast<uint64_t>(i);
  w[kN] = kN;
}

uint64_t Mt64::next() {
  constexpr int kM = 156;
  if (w[kN] >= static_cast<uint64_t>(kN)) {
    // The recurrence x[i] = x[i + m] ^ twist(x[i], x[i + 1]) over the words in order: the first n - m read only
    // words not yet replaced, the rest read replaced words i - m (and the last, replaced word 0).
    auto mix = [](uint64_t hi, uint64_t lo, uint64_t far) {
      const uint64_t y = (hi & 0xFFFFFFFF80000000ull) | (lo & 0x7FFFFFFFull);
      return far ^ (y >> 1) ^ ((y & 1) ? 0xB5026F5AA96619E9ull : 0);
    };
    for (int i = 0; i < kN - kM; ++i) w[i] = mix(w[i], w[i + 1], w[i + kM]);
    for (int i = kN - kM; i < kN - 1; ++i) w[i] = mix(w[i], w[i + 1], w[i - (kN - kM)]);
    w[kN - 1] = mix(w[kN - 1], w[0], w[kM - 1]);
    w[kN] = 0;
  }
  uint64_t z = w[w[kN]++];
  z ^= (z >> 29) & 0x5555555555555555ull;
  z ^= (z << 17) & 0x71D67FFFEDA60000ull;
  z ^= (z << 37) & 0xFFF7EEE000000000ull;
  return z ^ (z >> 43);
}

double Mt64::uniform() {
  const double u = static_cast<double>(next()) * 0x1p-64;
  return u < 1.0 ? u : std::nextafter(1.0, 0.0);
}

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

void Sampler::finish(const Selector& sel, int i, Distribution& out) const {
  const float* values = sel.values(i);
  const int32_t* ids = sel.ids(i);
  const int n = sel.count(i);
  if (!sel.cut(i)) return finish(values, ids, n, out);
  // The device kept the first keep(i) of the row's candidates against its total of all their weights. The same walk
  // over the host's weights of the candidates here (the head and one past it) and that total; where the walk stops
  // inside them, its count is used (the device's otherwise), then the kept weights are normalised as above.
  out.clear();
  if (n <= 0) throw std::invalid_argument("sampler: no candidates");
  if (greedy()) {
    out.push_back(Candidate{1.0f, ids[0]});
    return;
  }
  const float top = values[0];
  weights_.resize(static_cast<size_t>(n));
  for (int j = 0; j < n; ++j) weights_[static_cast<size_t>(j)] = std::exp((values[j] - top) / p_.temperature);
  const double floor_w = static_cast<double>(p_.min_p) * weights_[0];
  const double nucleus = static_cast<double>(p_.top_p) * sel.total(i);
  double run = 0.0;
  int keep = -1;
  for (int j = 0; j < n; ++j) {
    const double w = weights_[static_cast<size_t>(j)];
    if (j > 0 && w < floor_w) {
      keep = j;
      break;
    }
    run += w;
    if (run >= nucleus) {
      keep = j + 1;
      break;
    }
  }
  if (keep < 0) keep = sel.keep(i);
  keep = std::max(1, std::min(keep, n));
  double kept = 0.0;
  for (int j = 0; j < keep; ++j) kept += weights_[static_cast<size_t>(j)];
  out.reserve(static_cast<size_t>(keep));
  for (int j = 0; j < keep; ++j)
    out.push_back(Candidate{static_cast<float>(weights_[static_cast<size_t>(j)] / kept), ids[j]});
}

double Sampler::uniform() { return rng_.uniform(); }

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
  (void)mk_host_free(ctx_, cut_par_h_);
  (void)mk_host_free(ctx_, cut_v_h_);
  (void)mk_host_free(ctx_, cut_i_h_);
  (void)mk_host_free(ctx_, cut_keep_h_);
  (void)mk_host_free(ctx_, cut_sum_h_);
}

void Selector::clear() {
  reqs_.clear();
  pen_off_.assign(1, 0);
  pen_id_.clear();
  pen_amt_.clear();
  k_max_ = 0;
  n_cut_ = 0;
}

int Selector::add(int row, int k, const std::vector<int32_t>& pen_ids, const std::vector<float>& pen_amounts) {
  if (k < 1 || k > n_vocab_) throw std::invalid_argument("selector: bad candidate count");
  if (pen_ids.size() != pen_amounts.size()) throw std::invalid_argument("selector: penalty lists differ in length");
  if (pen_off_.empty()) pen_off_.assign(1, 0);
  Req r{row, k};
  if (k > kMaxDeviceK)
    throw std::invalid_argument("selector: more than 1024 candidates need the request's sampler");
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

int Selector::add(int row, const Sampler& s, const std::vector<int32_t>& pen_ids,
                  const std::vector<float>& pen_amounts) {
  const int k = s.candidates(n_vocab_);
  if (k <= kMaxDeviceK) return add(row, k, pen_ids, pen_amounts);
  if (pen_ids.size() != pen_amounts.size()) throw std::invalid_argument("selector: penalty lists differ in length");
  if (pen_off_.empty()) pen_off_.assign(1, 0);
  Req r{row, k, n_cut_++, s.params().temperature, s.params().min_p, s.params().top_p};
  reqs_.push_back(r);
  pen_id_.insert(pen_id_.end(), pen_ids.begin(), pen_ids.end());
  pen_amt_.insert(pen_amt_.end(), pen_amounts.begin(), pen_amounts.end());
  pen_off_.push_back(static_cast<int32_t>(pen_id_.size()));
  return static_cast<int>(reqs_.size()) - 1;
}

void Selector::reserve_cut(size_t rows) {
  if (rows <= cut_rows_) return;
  const size_t want = std::max(rows, 2 * cut_rows_);
  for (void* p : {static_cast<void*>(cut_par_h_), static_cast<void*>(cut_v_h_), static_cast<void*>(cut_i_h_),
                  static_cast<void*>(cut_keep_h_), static_cast<void*>(cut_sum_h_)})
    (void)mk_host_free(ctx_, p);
  cut_par_h_ = nullptr, cut_v_h_ = nullptr, cut_i_h_ = nullptr, cut_keep_h_ = nullptr, cut_sum_h_ = nullptr;
  auto host = [&](size_t bytes) {
    void* h = nullptr;
    ck(mk_host_alloc(ctx_, bytes, &h));
    return h;
  };
  cut_par_h_ = static_cast<mk_cut_params*>(host(want * (sizeof(mk_cut_params) + sizeof(int32_t))));  // + the rows
  cut_v_h_ = static_cast<float*>(host(want * kCutCap * sizeof(float)));
  cut_i_h_ = static_cast<int32_t*>(host(want * kCutCap * sizeof(int32_t)));
  cut_keep_h_ = static_cast<int32_t*>(host(want * sizeof(int32_t)));
  cut_sum_h_ = static_cast<double*>(host(want * sizeof(double)));
  cut_par_d_ = DevBuf(ctx_, want * (sizeof(mk_cut_params) + sizeof(int32_t)));  // params, then the rows
  cut_v_d_ = DevBuf(ctx_, want * kCutCap * sizeof(float));
  cut_i_d_ = DevBuf(ctx_, want * kCutCap * sizeof(int32_t));
  cut_keep_d_ = DevBuf(ctx_, want * sizeof(int32_t));
  cut_sum_d_ = DevBuf(ctx_, want * sizeof(double));
  cut_ws_bytes_ = mk_sample_cut_workspace(static_cast<int>(want), n_vocab_);
  if (cut_ws_bytes_ == 0) throw std::runtime_error(mk_last_error());
  cut_ws_ = DevBuf(ctx_, cut_ws_bytes_);
  cut_rows_ = want;
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
  if (n_cut_ > 0) {
    const size_t nc = static_cast<size_t>(n_cut_);
    reserve_cut(nc);
    cut_rows_h_.assign(nc, 0);
    for (const Req& r : reqs_) {
      if (r.cut < 0) continue;
      cut_par_h_[r.cut] = mk_cut_params{r.k, r.temperature, r.min_p, r.top_p};
      cut_rows_h_[static_cast<size_t>(r.cut)] = r.row;
    }
    std::memcpy(reinterpret_cast<uint8_t*>(cut_par_h_) + nc * sizeof(mk_cut_params), cut_rows_h_.data(),
                nc * sizeof(int32_t));
    ck(mk_copy_async(ctx_, cut_par_d_.p, cut_par_h_, nc * (sizeof(mk_cut_params) + sizeof(int32_t))));
    const auto* par = cut_par_d_.as<mk_cut_params>();
    const auto* rows = reinterpret_cast<const int32_t*>(cut_par_d_.as<uint8_t>() + nc * sizeof(mk_cut_params));
    ck(mk_sample_cut(ctx_, dev_logits, stride, rows, n_cut_, n_vocab_, par, kCutCap, cut_v_d_.as<float>(),
                     cut_i_d_.as<int32_t>(), cut_keep_d_.as<int32_t>(), cut_sum_d_.as<double>(), cut_ws_.p,
                     cut_ws_bytes_));
    ck(mk_copy_async(ctx_, cut_keep_h_, cut_keep_d_.p, nc * sizeof(int32_t)));
    ck(mk_copy_async(ctx_, cut_sum_h_, cut_sum_d_.p, nc * sizeof(double)));
    ck(mk_copy_async(ctx_, cut_v_h_, cut_v_d_.p, nc * kCutCap * sizeof(float)));
    ck(mk_copy_async(ctx_, cut_i_h_, cut_i_d_.p, nc * kCutCap * sizeof(int32_t)));
  }
}

// Device-cut rows: the kept head and one candidate past it (fewer when the head is the whole row); a head longer than
// kCutCap is fetched from the sorted row left in the workspace, with one more wait.
void Selector::collect() {
  cut_vals_.resize(static_cast<size_t>(n_cut_));
  cut_ids_.resize(static_cast<size_t>(n_cut_));
  for (const Req& r : reqs_) {
    if (r.cut < 0) continue;
    const size_t c = static_cast<size_t>(r.cut);
    const int keep = cut_keep_h_[c];
    if (keep < 1 || keep > r.k) throw std::runtime_error("selector: device cut returned a bad keep count");
    const int m = std::min(keep + 1, r.k);
    std::vector<float>& v = cut_vals_[c];
    std::vector<int32_t>& id = cut_ids_[c];
    v.assign(cut_v_h_ + c * kCutCap, cut_v_h_ + c * kCutCap + std::min(m, kCutCap));
    id.assign(cut_i_h_ + c * kCutCap, cut_i_h_ + c * kCutCap + std::min(m, kCutCap));
    if (m > kCutCap) {  // values, then ids, in one device block (room for a whole row) and one download
      const size_t more = static_cast<size_t>(m - kCutCap);
      if (!cut_tail_d_.p) cut_tail_d_ = DevBuf(ctx_, static_cast<size_t>(n_vocab_) * 8);
      float* tv = cut_tail_d_.as<float>();
      int32_t* ti = reinterpret_cast<int32_t*>(tv + more);
      ck(mk_sample_cut_tail(ctx_, cut_ws_.p, n_cut_, n_vocab_, r.cut, kCutCap, static_cast<int>(more), tv, ti));
      tail_h_.resize(2 * more);
      ck(mk_download(ctx_, tail_h_.data(), tv, 2 * more * sizeof(float)));
      v.insert(v.end(), tail_h_.begin(), tail_h_.begin() + static_cast<std::ptrdiff_t>(more));
      const auto* tid = reinterpret_cast<const int32_t*>(tail_h_.data() + more);
      id.insert(id.end(), tid, tid + more);
    }
  }
}

int Selector::count(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  return r.cut >= 0 ? static_cast<int>(cut_ids_[static_cast<size_t>(r.cut)].size()) : r.k;
}

int Selector::keep(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  return r.cut >= 0 ? cut_keep_h_[r.cut] : r.k;
}

double Selector::total(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  return r.cut >= 0 ? cut_sum_h_[r.cut] : 0.0;
}

const float* Selector::values(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  if (r.cut >= 0) return cut_vals_[static_cast<size_t>(r.cut)].data();
  return out_v_h_ + static_cast<size_t>(i) * out_k_;
}

const int32_t* Selector::ids(int i) const {
  const Req& r = reqs_[static_cast<size_t>(i)];
  if (r.cut >= 0) return cut_ids_[static_cast<size_t>(r.cut)].data();
  return out_i_h_ + static_cast<size_t>(i) * out_k_;
}

}  // namespace malkin_hip
