// Sampler::distribution's cut for rows with more candidates than the top-k selection holds (top_k <= 0: the whole
// vocabulary, or top_k above 1024), sampler.cpp:27-56, on the device: per row the k largest logits sorted highest
// first (equal logits by lower id), their weights exp((l - l_max) / T) as floats, summed in double in that order,
// and the kept head (the first candidate, then candidates while the weight reaches min_p times the first and the
// running sum has not reached top_p of the total). The host downloads the kept candidates and the total instead of
// the 608 KB row, and normalises the kept weights itself.
//
// k_draw finishes a top-k row the same way and draws from it with a std::mt19937_64 held in device memory (the
// draft's proposals: one row per sequence and draft depth, no host round trip between draft forwards).
//
// The sort is rocPRIM's stable device-wide radix sort of (order key, id) pairs, one row at a time (a row is 152k pairs:
// hundreds of workgroups). The cut is one 1024-thread workgroup per row: the weights in parallel into the workspace,
// then the sum and the keep scan in the reference's sequential order by one wave, 64 weights per load, each added
// in turn (a double sum's rounding depends on its order, so it is not split).
//
// The weights are exp of a float argument rounded to float. The reference calls the C library's expf; here exp is
// evaluated in double (error below 1 ulp of a double) and rounded to float, which gives the correctly rounded
// float. The C library's expf returns the correctly rounded result except where the exact value lies within about
// 2^-60 of a rounding boundary, and the double evaluation can misround only within about 2^-52 of one: a weight can
// differ in its last bit with a probability of the order of 2^-28. Only the keep count depends on the device's
// weights and total (the host recomputes the kept weights with the C library), and it changes only if such a
// difference moves the running sum across top_p of the total.
#include <rocprim/device/device_radix_sort.hpp>

#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kCutThreads = 1024;

__device__ __forceinline__ uint32_t cut_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float cut_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct CutWs {
  uint32_t *key_in, *key_out;
  int32_t *id_in, *id_out;
  float* w;
};

// Workspace layout for n_rows rows of n_vocab: keys in / out, ids in / out, weights, then the sort's storage.
__host__ __device__ inline size_t cut_row_words(int n_vocab) { return ((size_t)n_vocab + 63) & ~(size_t)63; }
__host__ __device__ inline CutWs cut_ws(void* base, int n_rows, int n_vocab) {
  const size_t n = cut_row_words(n_vocab) * (size_t)n_rows;
  uint32_t* p = static_cast<uint32_t*>(base);
  return CutWs{p, p + n, reinterpret_cast<int32_t*>(p + 2 * n), reinterpret_cast<int32_t*>(p + 3 * n),
               reinterpret_cast<float*>(p + 4 * n)};
}

__global__ void k_cut_keys(const float* __restrict__ logits, int64_t stride, const int32_t* __restrict__ rows,
                           int n_vocab, CutWs ws) {
  const int r = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_vocab) return;
  const float* l = logits + (int64_t)(rows ? rows[r] : r) * stride;
  const size_t o = cut_row_words(n_vocab) * (size_t)r + (size_t)i;
  ws.key_in[o] = cut_key(l[i]);
  ws.id_in[o] = i;
}

// One wave walks the weights w[0..k) in order, 64 per load; f(weight, index) returns false to stop. Every lane runs
// the same sequence (the weight comes from a lane read), so the state it updates is the same in every lane.
template <typename F>
__device__ __forceinline__ void walk_weights(const float* w, int k, F&& f) {
  const int lane = threadIdx.x & 63;
  for (int c = 0; c < k; c += 64) {
    const float mine = c + lane < k ? w[c + lane] : 0.0f;
    const int m = min(64, k - c);
    for (int j = 0; j < m; ++j) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), j));
      if (!f(wj, c + j)) return;
    }
  }
}

__global__ __launch_bounds__(kCutThreads) void k_cut(const mk_cut_params* __restrict__ params, int n_vocab, CutWs ws,
                                                     int cap, float* __restrict__ out_v, int32_t* __restrict__ out_i,
                                                     int32_t* __restrict__ keep_out, double* __restrict__ sum_out) {
  const int r = blockIdx.x, tid = threadIdx.x;
  const mk_cut_params p = params[r];
  const int k = p.k > 0 ? min(p.k, n_vocab) : n_vocab;
  const size_t o = cut_row_words(n_vocab) * (size_t)r;
  const uint32_t* key = ws.key_out + o;
  const int32_t* id = ws.id_out + o;
  float* w = ws.w + o;
  const float top = cut_value(key[0]);
  for (int i = tid; i < k; i += kCutThreads)
    w[i] = (float)exp((double)((cut_value(key[i]) - top) / p.temperature));
  __syncthreads();
  __shared__ int keep_s;
  if (tid < 64) {
    // sampler.cpp:41-45: the total, in sorted order.
    double sum = 0.0;
    walk_weights(w, k, [&](float wi, int) {
      sum += (double)wi;
      return true;
    });
    // sampler.cpp:47-55: the head above min_p of the first weight, up to the candidate whose running sum reaches
    // top_p of the total.
    const double floor = (double)p.min_p * (double)w[0];
    double kept = 0.0;
    int n = k;
    walk_weights(w, k, [&](float wi, int i) {
      if (i > 0 && (double)wi < floor) {
        n = i;
        return false;
      }
      kept += (double)wi;
      if (kept >= (double)p.top_p * sum) {
        n = i + 1;
        return false;
      }
      return true;
    });
    n = max(n, 1);
    if (tid == 0) {
      keep_s = n;
      keep_out[r] = n;
      sum_out[r] = sum;
    }
  }
  __syncthreads();
  // The kept head and one candidate past it (the host checks the stop there), up to cap.
  const int m = min(min(keep_s + 1, k), cap);
  for (int i = tid; i < m; i += kCutThreads) {
    out_v[(int64_t)r * cap + i] = cut_value(key[i]);
    out_i[(int64_t)r * cap + i] = id[i];
  }
}

__global__ void k_cut_tail(const uint32_t* __restrict__ key, const int32_t* __restrict__ id, int n,
                           float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out_v[i] = cut_value(key[i]);
  out_i[i] = id[i];
}

// ---- one draw per top-k row from a std::mt19937_64 kept on the device ----

constexpr int kMtN = 312, kMtM = 156;
constexpr int kDrawMax = 1024;  // candidates per row (mk_topk's limit)

__device__ __forceinline__ uint64_t mt_mix(uint64_t hi, uint64_t lo, uint64_t far) {
  const uint64_t y = (hi & 0xFFFFFFFF80000000ull) | (lo & 0x7FFFFFFFull);
  return far ^ (y >> 1) ^ ((y & 1) ? 0xB5026F5AA96619E9ull : 0ull);
}

// The state regenerated by one wave, in LDS: x[i] = x[i + m] ^ twist(x[i], x[i + 1]) in index order means that words
// 0..155 read only old words (all read before any is replaced), and words 156..311 read old words i + 1, the new
// word 0 (for 311) and new words i - 156.
__device__ void mt_regenerate(uint64_t* x) {
  const int lane = threadIdx.x;
  uint64_t v[3];
  for (int j = 0; j < 3; ++j) {
    const int i = lane + 64 * j;
    if (i < kMtM) v[j] = mt_mix(x[i], x[i + 1], x[i + kMtM]);
  }
  __syncthreads();
  for (int j = 0; j < 3; ++j) {
    const int i = lane + 64 * j;
    if (i < kMtM) x[i] = v[j];
  }
  __syncthreads();
  for (int j = 0; j < 3; ++j) {
    const int i = kMtM + lane + 64 * j;
    if (i < kMtN) v[j] = mt_mix(x[i], x[i + 1 < kMtN ? i + 1 : 0], x[i - kMtM]);
  }
  __syncthreads();
  for (int j = 0; j < 3; ++j) {
    const int i = kMtM + lane + 64 * j;
    if (i < kMtN) x[i] = v[j];
  }
  __syncthreads();
}

__device__ __forceinline__ uint64_t mt_temper(uint64_t z) {
  z ^= (z >> 29) & 0x5555555555555555ull;
  z ^= (z << 17) & 0x71D67FFFEDA60000ull;
  z ^= (z << 37) & 0xFFF7EEE000000000ull;
  return z ^ (z >> 43);
}

// One wave per row. The weights go to LDS; every sum and walk below runs in the reference's sequential order in all
// lanes alike (walk_weights), so each lane holds the same result.
__global__ __launch_bounds__(64) void k_draw(const float* __restrict__ values, const int32_t* __restrict__ ids,
                                             int stride, const mk_draw_params* __restrict__ params,
                                             uint64_t* __restrict__ states, int n_states, int32_t* __restrict__ out,
                                             int n_out) {
  __shared__ float w[kDrawMax];
  __shared__ uint64_t x[kMtN];
  const int r = blockIdx.x, lane = threadIdx.x;
  const mk_draw_params p = params[r];
  if (p.state < 0 || p.state >= n_states || p.dst < 0 || p.dst >= n_out) return;
  const int k = min(max(p.k, 1), stride);
  const float* v = values + (int64_t)r * stride;
  const int32_t* id = ids + (int64_t)r * stride;
  // sampler.cpp:37-45: weights exp((l - l_max) / T) as floats, their total in double in order.
  const float top = v[0];
  for (int i = lane; i < k; i += 64) w[i] = (float)exp((double)((v[i] - top) / p.temperature));
  __syncthreads();
  double all = 0.0;
  walk_weights(w, k, [&](float wi, int) {
    all += (double)wi;
    return true;
  });
  // sampler.cpp:47-56: the head above min_p of the first weight, up to the candidate whose running sum reaches top_p
  // of the total; the kept total is that running sum.
  const double floor_w = (double)p.min_p * (double)w[0], nucleus = (double)p.top_p * all;
  double run = 0.0;
  int keep = k;
  walk_weights(w, k, [&](float wi, int i) {
    if (i > 0 && (double)wi < floor_w) {
      keep = i;
      return false;
    }
    run += (double)wi;
    if (run >= nucleus) {
      keep = i + 1;
      return false;
    }
    return true;
  });
  int32_t pick = id[0];
  if (keep > 1) {
    // sampler.cpp:108-116: u from the generator, then the first candidate where the running u - p_i is <= 0.
    uint64_t* g = states + (int64_t)MK_MT64_WORDS * p.state;
    for (int i = lane; i < kMtN; i += 64) x[i] = g[i];
    uint64_t at = g[kMtN];
    __syncthreads();
    const bool regen = at >= (uint64_t)kMtN;
    if (regen) {
      mt_regenerate(x);
      at = 0;
    }
    double u = (double)mt_temper(x[at]) * 0x1p-64;
    if (u >= 1.0) u = 0x1.fffffffffffffp-1;
    pick = id[keep - 1];
    walk_weights(w, keep, [&](float wi, int i) {
      u -= (double)(float)((double)wi / run);
      if (u <= 0.0) {
        pick = id[i];
        return false;
      }
      return true;
    });
    if (regen)
      for (int i = lane; i < kMtN; i += 64) g[i] = x[i];
    if (lane == 0) g[kMtN] = at + 1;
  }
  if (lane == 0) out[p.dst] = pick;
}

size_t sort_storage(int n_vocab) {
  size_t bytes = 0;
  check(rocprim::radix_sort_pairs_desc(nullptr, bytes, static_cast<const uint32_t*>(nullptr),
                                       static_cast<uint32_t*>(nullptr), static_cast<const int32_t*>(nullptr),
                                       static_cast<int32_t*>(nullptr), (size_t)n_vocab),
        "radix_sort_pairs_desc (size)");
  return (bytes + 255) & ~(size_t)255;
}

}  // namespace

size_t sample_cut_workspace(int n_rows, int n_vocab) {
  if (n_rows <= 0 || n_vocab <= 0) return 0;
  return cut_row_words(n_vocab) * (size_t)n_rows * 5 * 4 + sort_storage(n_vocab);
}

void sample_cut(hipStream_t s, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
                const mk_cut_params* params, int cap, float* out_v, int32_t* out_i, int32_t* keep, double* sums,
                void* workspace, size_t workspace_bytes) {
  if (n_rows <= 0) return;
  require(n_vocab >= 1 && cap >= 1, "sample_cut: empty vocabulary or no output room");
  require(workspace != nullptr && workspace_bytes >= sample_cut_workspace(n_rows, n_vocab),
          "sample_cut: workspace smaller than mk_sample_cut_workspace");
  const CutWs ws = cut_ws(workspace, n_rows, n_vocab);
  hipLaunchKernelGGL(k_cut_keys, dim3((n_vocab + 255) / 256, n_rows), dim3(256), 0, s, logits, stride, rows, n_vocab,
                     ws);
  check_launch("sample_cut keys");
  void* sort_tmp = static_cast<uint8_t*>(workspace) + cut_row_words(n_vocab) * (size_t)n_rows * 5 * 4;
  size_t sort_bytes = sort_storage(n_vocab);
  for (int r = 0; r < n_rows; ++r) {
    const size_t o = cut_row_words(n_vocab) * (size_t)r;
    check(rocprim::radix_sort_pairs_desc(sort_tmp, sort_bytes, ws.key_in + o, ws.key_out + o, ws.id_in + o,
                                         ws.id_out + o, (size_t)n_vocab, 0, 32, s),
          "radix_sort_pairs_desc");
  }
  hipLaunchKernelGGL(k_cut, dim3(n_rows), dim3(kCutThreads), 0, s, params, n_vocab, ws, cap, out_v, out_i, keep, sums);
  check_launch("sample_cut");
}

void sample_cut_tail(hipStream_t s, void* workspace, int n_rows, int n_vocab, int row, int from, int count,
                     float* out_v, int32_t* out_i) {
  require(row >= 0 && row < n_rows && from >= 0 && count >= 0 && from + count <= n_vocab,
          "sample_cut_tail: range outside the row");
  if (count == 0) return;
  const CutWs ws = cut_ws(workspace, n_rows, n_vocab);
  const size_t o = cut_row_words(n_vocab) * (size_t)row + (size_t)from;
  hipLaunchKernelGGL(k_cut_tail, dim3((count + 255) / 256), dim3(256), 0, s, ws.key_out + o, ws.id_out + o, count,
                     out_v, out_i);
  check_launch("sample_cut_tail");
}

void sample_draw(hipStream_t s, const float* values, const int32_t* ids, int stride, int n_rows,
                 const mk_draw_params* params, uint64_t* states, int n_states, int32_t* out, int n_out) {
  if (n_rows <= 0) return;
  require(stride >= 1 && stride <= kDrawMax, "sample_draw: stride outside 1..1024");
  hipLaunchKernelGGL(k_draw, dim3(n_rows), dim3(64), 0, s, values, ids, stride, params, states, n_states, out, n_out);
  check_launch("sample_draw");
}

}  // namespace mk
