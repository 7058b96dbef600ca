// Candidate selection for stochastic sampling on the device (the first half of the reference's
// Sampler::distribution, sampler.cpp:22-40): repetition penalties applied to the logits in place, then per row the
// top k logits, highest first, ties by lower token id (where std::partial_sort leaves ties in an unspecified order).
// The host finishes the distribution over those k candidates (temperature, min-p, top-p, normalisation, draw), so a
// sampled request downloads k (value, id) pairs per row instead of the 608 KB logits row.
//
// Top-k per row, one 1024-thread workgroup: the logits become order-preserving 32-bit keys; an MSB-first radix
// select (four 8-bit digits, a 256-bin LDS histogram each) finds the k-th largest key T and how many keys exceed it;
// the keys above T are collected, then the lowest-indexed keys equal to T in index order; a bitonic sort in LDS
// orders the k candidates by (key desc, id asc).
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kMaxTopK = 1024;  // candidates per row held in LDS

// Larger float -> larger key (finite values and infinities; NaN logits are not expected).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One row per block: l[pen_id[i]] -= pen_amt[i] for this row's entries pen_off[r] .. pen_off[r + 1].
__global__ void k_penalize(float* __restrict__ logits, int64_t stride, const int32_t* __restrict__ rows,
                           const int32_t* __restrict__ pen_off, const int32_t* __restrict__ pen_id,
                           const float* __restrict__ pen_amt, int n_vocab) {
  const int r = blockIdx.x;
  float* l = logits + (int64_t)(rows ? rows[r] : r) * stride;
  for (int i = pen_off[r] + (int)threadIdx.x; i < pen_off[r + 1]; i += (int)blockDim.x) {
    const int id = pen_id[i];
    if (id >= 0 && id < n_vocab) l[id] = l[id] - pen_amt[i];
  }
}

__global__ __launch_bounds__(kSelThreads) void k_topk(const float* __restrict__ logits, int64_t stride,
                                                       const int32_t* __restrict__ rows, int n_vocab, int k,
                                                       float* __restrict__ out_v, int32_t* __restrict__ out_i) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t prefix_s, remain_s, count_s;
  __shared__ uint32_t ckey[kMaxTopK];
  __shared__ int32_t cidx[kMaxTopK];
  __shared__ uint32_t scan[kSelThreads / 64];
  const int tid = threadIdx.x;
  const int r = blockIdx.x;
  const float* l = logits + (int64_t)(rows ? rows[r] : r) * stride;

  // Radix select: after digit d, `prefix` holds the top 8 (d + 1) bits of T and `remain` the rank of T among the
  // keys that share them (1 = the largest).
  if (tid == 0) {
    prefix_s = 0;
    remain_s = (uint32_t)k;
  }
  for (int d = 0; d < 4; ++d) {
    const int shift = 24 - 8 * d;
    const uint32_t hmask = d == 0 ? 0u : 0xFFFFFFFFu << (32 - 8 * d);
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const uint32_t prefix = prefix_s;
    for (int i = tid; i < n_vocab; i += kSelThreads) {
      const uint32_t key = order_key(l[i]);
      if ((key & hmask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFF], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t rem = remain_s, b = 255;
      for (;; --b) {  // from the largest digit down: the bin that holds the rem-th largest key
        if (hist[b] >= rem || b == 0) break;
        rem -= hist[b];
      }
      prefix_s = prefix | (b << shift);
      remain_s = rem;
    }
    __syncthreads();
  }
  const uint32_t T = prefix_s;
  const uint32_t need_eq = remain_s;  // keys equal to T to take, lowest indices first
  // Keys above T: exactly k - need_eq of them, in any order (sorted below).
  if (tid == 0) count_s = 0;
  __syncthreads();
  for (int i = tid; i < n_vocab; i += kSelThreads) {
    const uint32_t key = order_key(l[i]);
    if (key > T) {
      const uint32_t slot = atomicAdd(&count_s, 1u);
      ckey[slot] = key;
      cidx[slot] = i;
    }
  }
  __syncthreads();
  // Keys equal to T in index order: chunks of kSelThreads consecutive indices, ranked by a block prefix count.
  uint32_t taken = 0;
  const uint32_t base = (uint32_t)k - need_eq;
  for (int c0 = 0; c0 < n_vocab && taken < need_eq; c0 += kSelThreads) {
    const int i = c0 + tid;
    const bool eq = i < n_vocab && order_key(l[i]) == T;
    const unsigned long long bal = __ballot(eq);
    const uint32_t lane = tid & 63, wave = tid >> 6;
    if (lane == 0) scan[wave] = (uint32_t)__popcll(bal);
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int w = 0; w < kSelThreads / 64; ++w) {
      before += w < (int)wave ? scan[w] : 0u;
      total += scan[w];
    }
    const uint32_t rank = taken + before + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
    if (eq && rank < need_eq) {
      ckey[base + rank] = T;
      cidx[base + rank] = i;
    }
    taken += total;
    __syncthreads();
  }
  // Bitonic sort of the k candidates (padded to a power of two) by key descending, index ascending.
  int n2 = 1;
  while (n2 < k) n2 <<= 1;
  for (int i = k + tid; i < n2; i += kSelThreads) {
    ckey[i] = 0u;
    cidx[i] = 0x7FFFFFFF;
  }
  __syncthreads();
  auto before_in_order = [](uint32_t ka, int ia, uint32_t kb, int ib) { return ka > kb || (ka == kb && ia < ib); };
  for (int size = 2; size <= n2; size <<= 1)
    for (int stride2 = size >> 1; stride2 > 0; stride2 >>= 1) {
      for (int i = tid; i < n2; i += kSelThreads) {
        const int j = i ^ stride2;
        if (j > i) {
          const bool up = (i & size) == 0;  // this run sorted in order (up) or reversed
          const bool swap = up ? before_in_order(ckey[j], cidx[j], ckey[i], cidx[i])
                               : before_in_order(ckey[i], cidx[i], ckey[j], cidx[j]);
          if (swap) {
            const uint32_t tk = ckey[i];
            const int ti = cidx[i];
            ckey[i] = ckey[j];
            cidx[i] = cidx[j];
            ckey[j] = tk;
            cidx[j] = ti;
          }
        }
      }
      __syncthreads();
    }
  for (int i = tid; i < k; i += kSelThreads) {
    out_i[(int64_t)r * k + i] = cidx[i];
    out_v[(int64_t)r * k + i] = l[cidx[i]];
  }
}

}  // namespace

void penalize(hipStream_t s, float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
              const int32_t* pen_off, const int32_t* pen_id, const float* pen_amt) {
  if (n_rows <= 0) return;
  require(pen_off != nullptr && pen_id != nullptr && pen_amt != nullptr, "penalize: missing penalty lists");
  hipLaunchKernelGGL(k_penalize, dim3(n_rows), dim3(256), 0, s, logits, stride, rows, pen_off, pen_id, pen_amt,
                     n_vocab);
  check_launch("penalize");
}

void topk(hipStream_t s, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab, int k,
          float* out_v, int32_t* out_i) {
  if (n_rows <= 0) return;
  require(k >= 1 && k <= kMaxTopK && k <= n_vocab, "topk: k must be 1..1024 and at most the vocabulary");
  hipLaunchKernelGGL(k_topk, dim3(n_rows), dim3(kSelThreads), 0, s, logits, stride, rows, n_vocab, k, out_v, out_i);
  check_launch("topk");
}

}  // namespace mk
