// Sampler::distribution's cut for rows with more candidates than the top-k selection holds (top_k <= 0: the whole
// vocabulary, or top_k above 1024), sampler.cpp:27-56, on the device: per row the k largest logits sorted highest
// first (equal logits by lower id), their weights exp((l - l_max) / T) as floats, summed in double in that order,
// and the kept head (the first candidate, then candidates while the weight reaches min_p times the first and the
// running sum has not reached top_p of the total). The host downloads the kept candidates and the total instead of
// the 608 KB row, and normalises the kept weights itself.
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

}  // namespace mk
