// Decode GEMV on the CDNA layout: y[t][r] = W[r] . x[t] for up to 8 tokens per workgroup, bit-identical to the
// reference's panel kernels (gemm_avx512.cpp:67-102 Q8_0, 104-155 Q4_K, 157-205 Q6_K, 268-316 Q6_K wide).
//
// The reference accumulates each output as one sequential fp32 chain over the row's blocks:
//   acc = fma(float(int dot of block b), scale_w(b) * scale_x(b), acc),  b = 0, 1, 2, ...
// The int dots are exact, so they can be computed in any order and in parallel; only the chain is sequential.
// A workgroup owns R rows x all columns:
//   phase 1 (all 256 threads): stream the rows' quants (128-byte-coalesced planes), compute every (row, unit, token)
//            int dot with v_dot4_i32_i8 and its per-unit float terms, park them in LDS;
//   phase 2 (R * NT lanes):   run each output's chain over the parked terms in block order.
// Columns are processed in LDS-sized chunks; the chain state stays in the phase-2 lanes' registers across chunks.
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // rows x units in flight per thread in phase 1
constexpr size_t kLdsBudget = 48 * 1024;

// Q8 blocks per unit and parked floats per (unit, token, row).
template <int T>
struct Unit;
template <>
struct Unit<kQ8_0> {
  static constexpr int q8 = 1, e = 2;
};
template <>
struct Unit<kQ4_K> {
  static constexpr int q8 = 2, e = 4;
};
template <>
struct Unit<kQ6_K> {
  static constexpr int q8 = 1, e = 4;
};

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& sc, int& m) {  // kernels.h:18-26
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// Loaded weight bytes of one (row, unit).
struct Raw {
  uint4 a;      // Q8_0 lo / Q4_K lo / Q6_K nibbles
  uint4 b;      // Q8_0 hi / Q4_K hi / Q6_K: x,y = hbits
  uint4 h;      // Q4_K header / Q6_K: x = sc pair, y = d
  uint32_t s;   // Q8_0 scale
};

template <int TYPE>
__device__ __forceinline__ Raw load_unit(const uint8_t* __restrict__ W, int64_t rows, int64_t cols, int64_t g, int rr,
                                         int64_t u) {
  Raw w{};
  if constexpr (TYPE == kQ8_0) {
    const PackedQ8_0 L{rows, cols / 32};
    const uint8_t* q = W + L.quants(g, u) + rr * 16;
    w.a = *reinterpret_cast<const uint4*>(q);
    w.b = *reinterpret_cast<const uint4*>(q + 128);
    w.s = *reinterpret_cast<const uint16_t*>(W + L.scales(g, u) + rr * 2);
  } else if constexpr (TYPE == kQ4_K) {
    const PackedQ4_K L{rows, cols / 256};
    const int64_t sb = u >> 2;
    const uint8_t* q = W + L.quants(g, sb, (int)(u & 3)) + rr * 16;
    w.a = *reinterpret_cast<const uint4*>(q);
    w.b = *reinterpret_cast<const uint4*>(q + 128);
    w.h = *reinterpret_cast<const uint4*>(W + L.headers(g, sb) + rr * 16);
  } else {
    const PackedQ6_K L{rows, cols / 256};
    const int64_t sb = u >> 3;
    const int b8 = (int)(u & 7);
    const uint8_t* q = W + L.quants(g, sb, b8) + rr * 16;
    w.a = *reinterpret_cast<const uint4*>(q);
    const uint2 hb = *reinterpret_cast<const uint2*>(W + L.quants(g, sb, b8) + 128 + rr * 8);
    w.b.x = hb.x;
    w.b.y = hb.y;
    w.h.x = *reinterpret_cast<const uint16_t*>(W + L.scales(g, sb) + rr * 16 + 2 * b8);
    w.h.y = *reinterpret_cast<const uint16_t*>(W + L.dscale(g, sb) + rr * 2);
  }
  return w;
}

// x block in LDS: 10 dwords = BlockQ8 {d, s0|s1, qs[32]}.
__device__ __forceinline__ int dot8(const uint4& lo, const uint4& hi, const int* xq) {
  int ai = dot4((int)lo.x, xq[2], 0);
  ai = dot4((int)lo.y, xq[3], ai);
  ai = dot4((int)lo.z, xq[4], ai);
  ai = dot4((int)lo.w, xq[5], ai);
  ai = dot4((int)hi.x, xq[6], ai);
  ai = dot4((int)hi.y, xq[7], ai);
  ai = dot4((int)hi.z, xq[8], ai);
  ai = dot4((int)hi.w, xq[9], ai);
  return ai;
}

__device__ __forceinline__ float xd(const int* xq) { return __int_as_float(xq[0]); }
__device__ __forceinline__ int xs0(const int* xq) { return (int)(int16_t)(xq[1] & 0xFFFF); }
__device__ __forceinline__ int xs1(const int* xq) { return (int)(int16_t)((uint32_t)xq[1] >> 16); }

template <int TYPE, bool WIDE, int R, int NT>
__global__ __launch_bounds__(kThreads) void k_gemv(const uint8_t* __restrict__ W, int64_t rows, int64_t cols,
                                                   const BlockQ8* __restrict__ x, int n, float* __restrict__ y,
                                                   int64_t ys, int accumulate, int chunk) {
  constexpr int UQ8 = Unit<TYPE>::q8;
  constexpr int E = (TYPE == kQ6_K && WIDE) ? 1 : Unit<TYPE>::e;
  extern __shared__ int smem[];
  const int64_t nq8 = cols / 32, nu = nq8 / UQ8;
  const int64_t g0 = (int64_t)blockIdx.x * (R / 8);
  const int t0 = blockIdx.y * NT;
  const int nt = min(NT, n - t0);
  const int tid = threadIdx.x;

  int* xs = smem;                                                  // [NT][chunk * UQ8][10]
  float* res = reinterpret_cast<float*>(xs + NT * chunk * UQ8 * 10);  // [chunk][NT][R][E]
  float* mnv = res + (size_t)chunk * NT * R * E;                   // Q4_K: [chunk][R][2]

  const int cr = tid % R, ct = tid / R;
  const bool chain = tid < R * NT && ct < nt;
  float acc = 0.0f;

  for (int64_t c0 = 0; c0 < nu; c0 += chunk) {
    const int cn = (int)min<int64_t>(chunk, nu - c0);
    // The first group of this chunk's weight loads goes out before the activations are staged, so HBM latency
    // overlaps the staging and the barrier.
    Raw raw[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int f = tid + k * kThreads;
      if (f < R * cn) raw[k] = load_unit<TYPE>(W, rows, cols, g0 + (f % R) / 8, (f % R) % 8, c0 + f / R);
    }
    // Stage this chunk's activation blocks: 8-byte loads (BlockQ8 is 8-byte aligned), all issued before any store.
    const int pairs = cn * UQ8 * 5;  // 8-byte words per token
    constexpr int kStage = 8;
    for (int i0 = tid; i0 < nt * pairs; i0 += kThreads * kStage) {
      uint2 v[kStage];
#pragma unroll
      for (int k = 0; k < kStage; ++k) {
        const int i = i0 + k * kThreads;
        if (i < nt * pairs) {
          const int t = i / pairs, rem = i % pairs;
          v[k] = reinterpret_cast<const uint2*>(x + (int64_t)(t0 + t) * nq8 + c0 * UQ8)[rem];
        }
      }
#pragma unroll
      for (int k = 0; k < kStage; ++k) {
        const int i = i0 + k * kThreads;
        if (i < nt * pairs) {
          const int t = i / pairs, rem = i % pairs;
          reinterpret_cast<uint2*>(xs + t * chunk * UQ8 * 10)[rem] = v[k];
        }
      }
    }
    __syncthreads();

    // Phase 1: int dots and per-unit float terms.
    for (int f0 = tid; f0 < R * cn; f0 += kThreads * kUnroll) {
      if (f0 != tid) {
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) {
          const int f = f0 + k * kThreads;
          if (f < R * cn) raw[k] = load_unit<TYPE>(W, rows, cols, g0 + (f % R) / 8, (f % R) % 8, c0 + f / R);
        }
      }
#pragma unroll
      for (int k = 0; k < kUnroll; ++k) {
        const int f = f0 + k * kThreads;
        if (f >= R * cn) break;
        const int u = f / R, r = f % R;
        const Raw& w = raw[k];
        if constexpr (TYPE == kQ8_0) {
          const float dw = half_to_float((uint16_t)w.s);
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t < nt) {
              const int* xq = xs + (t * chunk + u) * 10;
              float* e = res + (((size_t)u * NT + t) * R + r) * E;
              e[0] = (float)dot8(w.a, w.b, xq);
              e[1] = dw * xd(xq);
            }
          }
        } else if constexpr (TYPE == kQ4_K) {
          const int j0 = (int)((c0 + u) & 3) * 2;  // sub-blocks j0 (low nibbles) and j0 + 1 (high nibbles)
          const uint8_t* hb = reinterpret_cast<const uint8_t*>(&w.h);
          const float d = half_to_float((uint16_t)(w.h.x & 0xFFFF)), dmin = half_to_float((uint16_t)(w.h.x >> 16));
          int sc0, m0, sc1, m1;
          scale_min_k4(j0, hb + 4, sc0, m0);
          scale_min_k4(j0 + 1, hb + 4, sc1, m1);
          const float fsc0 = d * (float)sc0, fsc1 = d * (float)sc1;
          float* mn = mnv + ((size_t)u * R + r) * 2;
          mn[0] = dmin * (float)m0;
          mn[1] = dmin * (float)m1;
          const uint32_t wd[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t < nt) {
              const int* x0 = xs + (t * chunk + u) * UQ8 * 10;
              const int* x1 = x0 + 10;
              int a0 = 0, a1 = 0;
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                a0 = dot4((int)(wd[j] & 0x0F0F0F0Fu), x0[2 + j], a0);
                a1 = dot4((int)((wd[j] >> 4) & 0x0F0F0F0Fu), x1[2 + j], a1);
              }
              float* e = res + (((size_t)u * NT + t) * R + r) * E;
              e[0] = (float)a0;
              e[1] = fsc0 * xd(x0);
              e[2] = (float)a1;
              e[3] = fsc1 * xd(x1);
            }
          }
        } else {  // Q6_K
          const uint32_t nw[4] = {w.a.x, w.a.y, w.a.z, w.a.w};
          const uint32_t hw[2] = {w.b.x, w.b.y};
          const float d = half_to_float((uint16_t)w.h.y);
          const float dsc0 = d * (float)(int8_t)(w.h.x & 0xFF), dsc1 = d * (float)(int8_t)((w.h.x >> 8) & 0xFF);
          int qv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t lo = j < 4 ? (nw[j] & 0x0F0F0F0Fu) : ((nw[j - 4] >> 4) & 0x0F0F0F0Fu);
            const uint32_t hi = ((hw[j >> 2] >> (2 * (j & 3))) & 0x03030303u) << 4;
            qv[j] = (int)(lo | hi);
          }
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t < nt) {
              const int* xq = xs + (t * chunk + u) * 10;
              int a0 = 0, a1 = 0;
#pragma unroll
              for (int j = 0; j < 4; ++j) a0 = dot4(qv[j], xq[2 + j], a0);
#pragma unroll
              for (int j = 4; j < 8; ++j) a1 = dot4(qv[j], xq[2 + j], a1);
              a0 -= 32 * xs0(xq);
              a1 -= 32 * xs1(xq);
              float* e = res + (((size_t)u * NT + t) * R + r) * E;
              if constexpr (WIDE) {
                e[0] = fma_((float)a1, dsc1, (float)a0 * dsc0);
              } else {
                e[0] = (float)a0;
                e[1] = dsc0 * xd(xq);
                e[2] = (float)a1;
                e[3] = dsc1 * xd(xq);
              }
            }
          }
        }
      }
    }
    __syncthreads();

    // Phase 2: the sequential chains, in block order.
    if (chain) {
#pragma unroll 8
      for (int u = 0; u < cn; ++u) {
        const float* e = res + (((size_t)u * NT + ct) * R + cr) * E;
        if constexpr (TYPE == kQ8_0) {
          acc = fma_(e[0], e[1], acc);
        } else if constexpr (TYPE == kQ4_K) {
          const float* mn = mnv + ((size_t)u * R + cr) * 2;
          const int* x0 = xs + (ct * chunk + u) * UQ8 * 10;
          const int* x1 = x0 + 10;
          const float dsx0 = xd(x0) * (float)(xs0(x0) + xs1(x0));
          const float dsx1 = xd(x1) * (float)(xs0(x1) + xs1(x1));
          acc = fma_(e[0], e[1], acc);
          acc = fma_(-mn[0], dsx0, acc);
          acc = fma_(e[2], e[3], acc);
          acc = fma_(-mn[1], dsx1, acc);
        } else if constexpr (WIDE) {
          acc = fma_(e[0], xd(xs + (ct * chunk + u) * 10), acc);
        } else {
          acc = fma_(e[0], e[1], acc);
          acc = fma_(e[2], e[3], acc);
        }
      }
    }
    __syncthreads();
  }
  if (chain) {
    float* o = y + (int64_t)(t0 + ct) * ys + (int64_t)blockIdx.x * R + cr;
    *o = accumulate ? *o + acc : acc;
  }
}

template <int TYPE, bool WIDE, int R, int NT>
void launch(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
            bool accumulate) {
  constexpr int UQ8 = Unit<TYPE>::q8;
  constexpr int E = (TYPE == kQ6_K && WIDE) ? 1 : Unit<TYPE>::e;
  const size_t per_unit = (size_t)NT * UQ8 * 40 + (size_t)NT * R * E * 4 + (TYPE == kQ4_K ? (size_t)R * 8 : 0);
  const int64_t nu = cols / 32 / UQ8;
  const int chunk = (int)std::min<int64_t>(nu, (int64_t)(kLdsBudget / per_unit));
  const size_t lds = per_unit * chunk;
  const dim3 grid((unsigned)(rows / R), (unsigned)((n + NT - 1) / NT));
  hipLaunchKernelGGL((k_gemv<TYPE, WIDE, R, NT>), grid, dim3(kThreads), lds, s, static_cast<const uint8_t*>(w), rows,
                     cols, x, n, y, ys, accumulate ? 1 : 0, chunk);
}

template <int TYPE, bool WIDE, int R>
void launch_nt(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
               bool acc) {
  if (n <= 1)
    launch<TYPE, WIDE, R, 1>(s, w, rows, cols, x, n, y, ys, acc);
  else if (n <= 2)
    launch<TYPE, WIDE, R, 2>(s, w, rows, cols, x, n, y, ys, acc);
  else if (n <= 4)
    launch<TYPE, WIDE, R, 4>(s, w, rows, cols, x, n, y, ys, acc);
  else
    launch<TYPE, WIDE, R, 8>(s, w, rows, cols, x, n, y, ys, acc);
}

template <int TYPE, bool WIDE>
void launch_r(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
              bool acc) {
  // Wide workgroups amortise the activation staging; narrow ones keep >= 2048 workgroups in flight.
  if (rows % 32 == 0 && rows / 32 >= 2048)
    launch_nt<TYPE, WIDE, 32>(s, w, rows, cols, x, n, y, ys, acc);
  else
    launch_nt<TYPE, WIDE, 8>(s, w, rows, cols, x, n, y, ys, acc);
}

}  // namespace

void matmul(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* xq, int n,
            float* y, int64_t ys, bool accumulate) {
  require(n > 0, "matmul: no tokens");
  require(packed_bytes(type, rows, cols) != 0, "matmul: no kernel for this weight type/shape");
  switch (type) {
    case kQ8_0:
      if (gemm_q8_0_supported(rows, cols, n))
        gemm_q8_0(s, w, rows, cols, xq, n, y, ys, accumulate);  // prefill / batches: int8 MFMA
      else
        launch_r<kQ8_0, false>(s, w, rows, cols, xq, n, y, ys, accumulate);
      break;
    case kQ4_K:
      launch_r<kQ4_K, false>(s, w, rows, cols, xq, n, y, ys, accumulate);
      break;
    case kQ6_K:
      // The reference switches Q6_K to its wide panels above kWideMinTokens = 16 tokens (quant.cpp:256).
      if (wide && n > 16)
        launch_r<kQ6_K, true>(s, w, rows, cols, xq, n, y, ys, accumulate);
      else
        launch_r<kQ6_K, false>(s, w, rows, cols, xq, n, y, ys, accumulate);
      break;
    default:
      throw Error(MK_ERR_UNSUPPORTED, "matmul: unsupported weight type");
  }
  check_launch("matmul");
}

}  // namespace mk
