// Stochastic sampling over device logits: the reference's malkin::Sampler (sampler.h:10-43, sampler.cpp:22-97) split
// at its one expensive step. The device applies the repetition penalties and cuts each logits row to its top-k
// candidates (mk_penalize, mk_topk); the host turns those k values into the final distribution (temperature,
// min-p, nucleus, normalisation), draws from it and runs the speculative accept/reject test. Only k (value, id)
// pairs per row cross PCIe instead of the whole logits row.
//
// What must equal the reference for the same seed (and therefore is computed the same way):
//   * the penalty of a token seen c times: presence + frequency * c, one fused multiply-add in float, subtracted
//     from its logit;
//   * greedy (temperature <= 0): the first maximum of the penalized logits;
//   * candidates: the top_k largest penalized logits (top_k <= 0: the whole vocabulary), highest first; weights
//     exp((l - l_max) / T) in float, summed in double in that order; kept: the first candidate, then candidates
//     while their weight is at least min_p * w_0, up to and including the one whose running sum reaches
//     top_p * (sum of all candidate weights); probabilities: weight / (sum of kept weights), rounded to float;
//   * draws: u ~ U[0, 1) from std::mt19937_64 (seeded with the request's seed, or std::random_device for seed 0)
//     through std::uniform_real_distribution<double> (Mt64 below: the same generator and the same conversion); the first candidate where the running u - p_i <= 0, the last
//     if rounding leaves u above zero; a one-entry distribution draws nothing;
//   * verify (Leviathan et al. 2023, speculative sampling): accept draft d when u * q(d) < p(d) (and q(d) > 0),
//     else draw from the normalised positive part of p - q over p's candidates (from p itself when that is empty).
// Equal logits at the top-k boundary are ordered by lower id here; the reference's partial_sort leaves their order
// unspecified.
#pragma once

#include <cstdint>
#include <unordered_map>
#include <vector>

#include "model.h"

namespace malkin_hip {

struct SamplingParams {  // sampler.h:10-18 (same fields and defaults)
  float temperature = 0.8f;  // <= 0: greedy
  float top_p = 0.95f;
  int top_k = 40;  // <= 0: whole vocabulary
  float min_p = 0.05f;
  float presence_penalty = 0.0f;
  float frequency_penalty = 0.0f;
  uint64_t seed = 0;  // 0: random
};

// std::mt19937_64 ([rand.predef]: the 64-bit Mersenne Twister of Matsumoto and Nishimura, n 312, m 156, r 31,
// a 0xB5026F5AA96619E9, tempering (29, 0x5555555555555555), (17, 0x71D67FFFEDA60000), (37, 0xFFF7EEE000000000), 43,
// seeding multiplier 6364136223846793005) with its state in one plain array, so that the engine can hand a draft
// sampler's generator to the device's draws (mk_sample_draw, which advances the same layout).
struct Mt64 {
  static constexpr int kN = 312;
  static constexpr int kWords = kN + 1;  // mk_sample_draw's layout: the state words, then the index of the next one
  uint64_t w[kWords];
  explicit Mt64(uint64_t seed);
  uint64_t next();
  // libstdc++'s std::uniform_real_distribution<double>(0, 1) on a 64-bit generator: generate_canonical with one
  // output x, (double)x / 2^64, and a result that rounds to 1 replaced by the largest double below 1.
  double uniform();
};

struct Candidate {
  float p;
  int32_t id;
};
using Distribution = std::vector<Candidate>;  // highest probability first

class Sampler {
 public:
  Sampler(const SamplingParams& params, bool penalties);
  const SamplingParams& params() const { return p_; }
  bool greedy() const { return p_.temperature <= 0.0f; }
  // Penalties change logits (both zero: they cannot).
  bool penalizes() const { return penalties_ && (p_.presence_penalty != 0.0f || p_.frequency_penalty != 0.0f); }
  // Candidates the distribution needs from a row of n_vocab logits: 1 for greedy, else min(top_k, n_vocab), or
  // n_vocab when top_k <= 0.
  int candidates(int n_vocab) const;
  // The penalties a row gets when the tokens `path` are accepted after those already counted: (id, amount) pairs
  // appended to ids / amounts.
  void penalties(const int32_t* path, int n_path, std::vector<int32_t>& ids, std::vector<float>& amounts) const;
  // The distribution from a row's candidates: values (penalized logits) and ids, highest first, n of them
  // (candidates(n_vocab), or fewer only for greedy).
  void finish(const float* values, const int32_t* ids, int n, Distribution& out) const;
  // The same from request i of a collected Selector: its candidates, or for a row cut on the device (more than
  // Selector::kMaxDeviceK candidates) its kept head and total.
  void finish(const class Selector& sel, int i, Distribution& out) const;
  int32_t draw(const Distribution& d);
  int32_t verify(const Distribution& p, const Distribution& q, int32_t draft, bool& accepted);
  void accept(int32_t id) { ++counts_[id]; }
  const Mt64& generator() const { return rng_; }

 private:
  double uniform();

  SamplingParams p_;
  bool penalties_;
  Mt64 rng_;
  std::unordered_map<int32_t, int> counts_;
  mutable std::vector<double> weights_;
};

// Candidate selection for several logits rows with one host wait: per row its penalties and candidate count; the
// device penalizes the rows in place and cuts the top-k (up to 1024 candidates); a row that needs more (top_k <= 0,
// or above 1024) is sorted and cut on the device with its request's temperature, min_p and top_p (mk_sample_cut),
// and only its kept head and total come back. enqueue() queues the work and the copies on the context's stream;
// after the caller's next mk_synchronize, collect() makes the candidates readable (a kept head longer than
// kCutCap takes one more copy and wait there).
class Selector {
 public:
  static constexpr int kMaxDeviceK = 1024;
  static constexpr int kCutCap = 4096;  // candidates of a device-cut row copied back with the step's wait
  Selector(mk_ctx* ctx, int n_vocab);
  ~Selector();
  Selector(const Selector&) = delete;
  Selector& operator=(const Selector&) = delete;

  void clear();
  // Logits row `row` of the buffer the next enqueue() reads; penalties (may be empty) are applied in place.
  // Returns the request's index.
  int add(int row, int k, const std::vector<int32_t>& pen_ids, const std::vector<float>& pen_amounts);
  // The same for a request's sampler: its candidate count, and its parameters for a device cut.
  int add(int row, const Sampler& s, const std::vector<int32_t>& pen_ids, const std::vector<float>& pen_amounts);
  bool empty() const { return reqs_.empty(); }
  void enqueue(float* dev_logits);
  void collect();
  // After collect(): candidates of request i, highest first (count(i) of them).
  const float* values(int i) const;
  const int32_t* ids(int i) const;
  int count(int i) const;
  // A row cut on the device: count(i) candidates of which the first keep(i) are kept, the total of all weights.
  bool cut(int i) const { return reqs_[static_cast<size_t>(i)].cut >= 0; }
  int keep(int i) const;
  double total(int i) const;

 private:
  struct Req {
    int row, k;
    int cut = -1;  // index among the device-cut rows, or -1
    float temperature = 1.0f, min_p = 0.0f, top_p = 1.0f;
  };
  void reserve_host(size_t words);
  void reserve_out(size_t rows, int k);
  void reserve_cut(size_t rows);

  mk_ctx* ctx_;
  int n_vocab_;
  std::vector<Req> reqs_;
  std::vector<int32_t> pen_off_, pen_id_;
  std::vector<float> pen_amt_;
  int k_max_ = 0, n_cut_ = 0;
  // Upload block (rows, pen_off, pen_id, pen_amt) in pinned memory and on the device; results likewise.
  int32_t* in_h_ = nullptr;
  size_t in_words_ = 0;
  DevBuf in_d_;
  float* out_v_h_ = nullptr;
  int32_t* out_i_h_ = nullptr;
  size_t out_cap_ = 0;  // rows * k entries
  DevBuf out_v_d_, out_i_d_;
  // Device-cut rows: parameters, outputs and workspace on the device; outputs in pinned memory; after collect()
  // each row's candidates (the kept head and one past it) on the host.
  size_t cut_rows_ = 0;
  DevBuf cut_ws_, cut_par_d_, cut_v_d_, cut_i_d_, cut_keep_d_, cut_sum_d_;
  size_t cut_ws_bytes_ = 0;
  mk_cut_params* cut_par_h_ = nullptr;
  float* cut_v_h_ = nullptr;
  int32_t* cut_i_h_ = nullptr;
  int32_t* cut_keep_h_ = nullptr;
  double* cut_sum_h_ = nullptr;
  std::vector<int32_t> cut_rows_h_;
  DevBuf cut_tail_d_;          // a kept head past kCutCap: its candidates from the sorted row
  std::vector<float> tail_h_;
  std::vector<std::vector<float>> cut_vals_;
  std::vector<std::vector<int32_t>> cut_ids_;
  int out_k_ = 0;
};

}  // namespace malkin_hip
