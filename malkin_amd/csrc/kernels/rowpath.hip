// matmul's row path (quant.cpp:171-191 vec_dot, 330-351 matmul): the reference evaluates every output as one weight
// row (GGUF bytes, not repacked) dotted with one activation row. It runs for F32 / F16 / BF16 weights (they have no
// panels) and, with MALKIN_NO_PACK, for the quantized types too. Its arithmetic differs from the panel kernels, so it
// has its own kernel here, bit-identical to the AVX-512 row kernels (kernels_avx512.cpp:31-171):
//   a 16-lane group of a wave plays one 512-bit accumulator: lane l holds lane l of the reference's register and
//   runs its fma chain; the halving tree of _mm512_reduce_add_ps then combines the 16 lanes (shuffles 8, 4, 2, 1
//   apart); lane 0 finishes the scalar parts (the F types' k % 16 tail, Q8_0's odd last block, the K-quants' mins /
//   bias chains).
// A wave holds four groups, a workgroup sixteen: one weight row per group, NT tokens of it at once so that a row is read
// once per token tile. These weights are off the configurations' hot path (every matmul weight there is quantized and
// packed); the kernel favours the reference's exact order over bandwidth.
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kRowsThreads = 256;
constexpr int kRowsNT = 8;  // tokens per group pass

__device__ __forceinline__ float bf16_to_float(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Four bytes at any alignment, as the little-endian int of four int8 values.
__device__ __forceinline__ int ld_i8x4(const uint8_t* p) {
  return (int)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
}

// Sum over the 16 lanes of a group in the order of _mm512_reduce_add_ps (pairs 8, 4, 2, 1 apart); lane 0 holds it.
__device__ __forceinline__ float tree16(float v) {
  v = v + __shfl_down(v, 8, 16);
  v = v + __shfl_down(v, 4, 16);
  v = v + __shfl_down(v, 2, 16);
  v = v + __shfl_down(v, 1, 16);
  return v;
}

// kernels.h:18-26: the 6-bit scale and min of sub-block j from the 12 packed bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& sc, int& m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

__device__ __forceinline__ int xq_word(const BlockQ8& b, int g) { return reinterpret_cast<const int*>(b.qs)[g]; }

template <int TYPE>
__global__ __launch_bounds__(kRowsThreads) void k_rows(const uint8_t* __restrict__ W, size_t row_bytes, int64_t rows,
                                                       int64_t cols, const float* __restrict__ x, int64_t xs,
                                                       const BlockQ8* __restrict__ xq, int n, float* __restrict__ y,
                                                       int64_t ys, int accumulate) {
  const int lane = threadIdx.x & 15;
  const int64_t r = (int64_t)blockIdx.x * (kRowsThreads / 16) + threadIdx.x / 16;
  const int t0 = blockIdx.y * kRowsNT;
  if (r >= rows) return;  // a whole group leaves together: the shuffles below stay within live groups
  const int nt = min(kRowsNT, n - t0);
  const uint8_t* w = W + (size_t)r * row_bytes;
  const int64_t nb = cols / 32;
  float acc[kRowsNT], tail[kRowsNT];
#pragma unroll
  for (int t = 0; t < kRowsNT; ++t) acc[t] = 0.0f, tail[t] = 0.0f;

  if constexpr (TYPE == kF32 || TYPE == kF16 || TYPE == kBF16) {
    // kernels_avx512.cpp:82-107: lane l accumulates elements 16 i + l, then the tree, then the scalar tail.
    const int64_t full = cols / 16 * 16;
    for (int64_t i = lane; i < full; i += 16) {
      float wv;
      if constexpr (TYPE == kF32)
        wv = reinterpret_cast<const float*>(w)[i];
      else if constexpr (TYPE == kF16)
        wv = half_to_float(reinterpret_cast<const uint16_t*>(w)[i]);
      else
        wv = bf16_to_float(reinterpret_cast<const uint16_t*>(w)[i]);
#pragma unroll
      for (int t = 0; t < kRowsNT; ++t)
        if (t < nt) acc[t] = fma_(wv, x[(int64_t)(t0 + t) * xs + i], acc[t]);
    }
#pragma unroll
    for (int t = 0; t < kRowsNT; ++t) acc[t] = tree16(acc[t]);
    if (lane == 0)
      for (int64_t i = full; i < cols; ++i) {
        float wv;
        if constexpr (TYPE == kF32)
          wv = reinterpret_cast<const float*>(w)[i];
        else if constexpr (TYPE == kF16)
          wv = half_to_float(reinterpret_cast<const uint16_t*>(w)[i]);
        else
          wv = bf16_to_float(reinterpret_cast<const uint16_t*>(w)[i]);
#pragma unroll
        for (int t = 0; t < kRowsNT; ++t)
          if (t < nt) acc[t] = fma_(wv, x[(int64_t)(t0 + t) * xs + i], acc[t]);
      }
  } else if constexpr (TYPE == kQ8_0) {
    // kernels_avx512.cpp:110-137: block pairs, lane l = 4-byte group l % 8 of block 2p + l / 8.
    const int g = lane & 7;
    for (int64_t b0 = 0; b0 + 2 <= nb; b0 += 2) {
      const int64_t b = b0 + lane / 8;
      const uint8_t* blk = w + b * 34;
      const int wq = ld_i8x4(blk + 2 + 4 * g);
      const float dw = half_to_float(ld_u16(blk));
#pragma unroll
      for (int t = 0; t < kRowsNT; ++t)
        if (t < nt) {
          const BlockQ8& xb = xq[(int64_t)(t0 + t) * nb + b];
          acc[t] = fma_((float)dot4(wq, xq_word(xb, g), 0), dw * xb.d, acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < kRowsNT; ++t) acc[t] = tree16(acc[t]);
    if ((nb & 1) && lane == 0) {
      const int64_t b = nb - 1;
      const uint8_t* blk = w + b * 34;
      const float dw = half_to_float(ld_u16(blk));
#pragma unroll
      for (int t = 0; t < kRowsNT; ++t)
        if (t < nt) {
          const BlockQ8& xb = xq[(int64_t)(t0 + t) * nb + b];
          int dp = 0;
          for (int e = 0; e < 8; ++e) dp = dot4(ld_i8x4(blk + 2 + 4 * e), xq_word(xb, e), dp);
          acc[t] = fma_((float)dp * dw, xb.d, acc[t]);
        }
    }
  } else if constexpr (TYPE == kQ4_K || TYPE == kQ5_K) {
    // kernels_avx512.cpp:31-64: per sub-block pair j, lanes 0-7 the 4-value groups of sub-block 2j (low nibbles),
    // lanes 8-15 those of 2j + 1 (high nibbles); Q5_K adds each value's high bit.
    constexpr bool kHigh = TYPE == kQ5_K;
    constexpr int kBytes = kHigh ? 176 : 144;
    const int hi = lane >> 3, g = lane & 7;
    for (int64_t sb = 0; sb < cols / 256; ++sb) {
      const uint8_t* s = w + sb * kBytes;
      const float d = half_to_float(ld_u16(s)), dmin = half_to_float(ld_u16(s + 2));
      const uint8_t* qh = s + 16;
      const uint8_t* q = s + (kHigh ? 48 : 16);
      for (int j = 0; j < 4; ++j, q += 32) {
        int s0, m0, s1, m1;
        scale_min_k4(2 * j, s + 4, s0, m0);
        scale_min_k4(2 * j + 1, s + 4, s1, m1);
        const uint32_t qw = (uint32_t)ld_i8x4(q + 4 * g);
        uint32_t v = hi ? (qw >> 4) & 0x0F0F0F0Fu : qw & 0x0F0F0F0Fu;
        if constexpr (kHigh) v |= (((uint32_t)ld_i8x4(qh + 4 * g) >> (2 * j + hi)) & 0x01010101u) << 4;
#pragma unroll
        for (int t = 0; t < kRowsNT; ++t)
          if (t < nt) {
            const BlockQ8* xb = xq + (int64_t)(t0 + t) * nb + sb * 8 + 2 * j;
            const BlockQ8& xh = xb[hi];
            const float sc = d * (float)(hi ? s1 : s0) * xh.d;
            acc[t] = fma_((float)dot4((int)v, xq_word(xh, g), 0), sc, acc[t]);
            // mins = fma(dmin, fma(m0 * dx0, S0, (m1 * dx1) * S1), mins): lane 0's copy is the one used
            const float in = fma_((float)m0 * xb[0].d, (float)(xb[0].s[0] + xb[0].s[1]),
                                  ((float)m1 * xb[1].d) * (float)(xb[1].s[0] + xb[1].s[1]));
            tail[t] = fma_(dmin, in, tail[t]);
          }
      }
    }
#pragma unroll
    for (int t = 0; t < kRowsNT; ++t) acc[t] = tree16(acc[t]) - tail[t];
  } else {  // kQ6_K
    // kernels_avx512.cpp:142-171: per 128-value half, two passes; in pass p lane l takes the 4-value group l % 8 of
    // the half's 32-value group 2 p + l / 8 (unsigned q) times sub-block scale 4 p + l / 4; bias restores q - 32.
    const int g = lane & 7;
    for (int64_t sb = 0; sb < cols / 256; ++sb) {
      const uint8_t* s = w + sb * 210;
      const float d = half_to_float(ld_u16(s + 208));
      for (int hf = 0; hf < 2; ++hf) {
        const uint8_t* ql = s + 64 * hf;
        const uint8_t* qh = s + 128 + 32 * hf;
        const int8_t* sc = reinterpret_cast<const int8_t*>(s + 192 + 8 * hf);
        const uint32_t l0 = (uint32_t)ld_i8x4(ql + 4 * g), l1 = (uint32_t)ld_i8x4(ql + 32 + 4 * g);
        const uint32_t hb = (uint32_t)ld_i8x4(qh + 4 * g);
        // 32-value groups 0..3 of the half: low nibbles of bytes 0-31 / 32-63, then their high nibbles
        const uint32_t q0 = (l0 & 0x0F0F0F0Fu) | ((hb & 0x03030303u) << 4);
        const uint32_t q1 = (l1 & 0x0F0F0F0Fu) | (((hb >> 2) & 0x03030303u) << 4);
        const uint32_t q2 = ((l0 >> 4) & 0x0F0F0F0Fu) | (((hb >> 4) & 0x03030303u) << 4);
        const uint32_t q3 = ((l1 >> 4) & 0x0F0F0F0Fu) | (((hb >> 6) & 0x03030303u) << 4);
        const int up = lane >> 3;  // 0: first 32-value group of the pass, 1: second
#pragma unroll
        for (int t = 0; t < kRowsNT; ++t)
          if (t < nt) {
            const BlockQ8* xb = xq + (int64_t)(t0 + t) * nb + sb * 8 + 4 * hf;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const int grp = 2 * p + up;
              const uint32_t qv = p == 0 ? (up ? q1 : q0) : (up ? q3 : q2);
              const int dp = dot4((int)qv, xq_word(xb[grp], g), 0) * (int)sc[4 * p + lane / 4];
              acc[t] = fma_((float)dp, d * xb[grp].d, acc[t]);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
              tail[t] = fma_(d * xb[k].d * 32.0f,
                             (float)((int)sc[2 * k] * xb[k].s[0] + (int)sc[2 * k + 1] * xb[k].s[1]), tail[t]);
          }
      }
    }
#pragma unroll
    for (int t = 0; t < kRowsNT; ++t) acc[t] = tree16(acc[t]) - tail[t];
  }
  if (lane == 0)
#pragma unroll
    for (int t = 0; t < kRowsNT; ++t)
      if (t < nt) {
        float* o = y + (int64_t)(t0 + t) * ys + r;
        *o = accumulate ? *o + acc[t] : acc[t];
      }
}

// The panel kernels' arithmetic for Q4_K / Q5_K (gemm_avx512.cpp:104-155 compact, 217-266 wide: the same sequence)
// read straight from GGUF rows: per output, per 32-value sub-block j in order, acc = fma(float(int dot), (d * sc) * dx,
// acc), then acc = fma(-(dmin * m), dx * (s0 + s1), acc). An 8-lane group owns one row: lane g takes the 4-value
// group g of each sub-block, the exact int dot is summed over the group (butterfly), and every lane keeps the same
// chain. This is the device path for Q5_K weights, which have no CDNA layout.
template <bool kHigh>
__global__ __launch_bounds__(kRowsThreads) void k_gguf45(const uint8_t* __restrict__ W, size_t row_bytes, int64_t rows,
                                                         int64_t cols, const BlockQ8* __restrict__ xq, int n,
                                                         float* __restrict__ y, int64_t ys, int accumulate) {
  constexpr int kBytes = kHigh ? 176 : 144;
  const int g = threadIdx.x & 7;
  const int64_t r = (int64_t)blockIdx.x * (kRowsThreads / 8) + threadIdx.x / 8;
  const int t0 = blockIdx.y * kRowsNT;
  if (r >= rows) return;  // whole 8-lane groups leave together
  const int nt = min(kRowsNT, n - t0);
  const uint8_t* w = W + (size_t)r * row_bytes;
  const int64_t nb = cols / 32;
  float acc[kRowsNT];
#pragma unroll
  for (int t = 0; t < kRowsNT; ++t) acc[t] = 0.0f;
  for (int64_t sb = 0; sb < cols / 256; ++sb) {
    const uint8_t* s = w + sb * kBytes;
    const float d = half_to_float(ld_u16(s)), dmin = half_to_float(ld_u16(s + 2));
    const uint32_t qh = kHigh ? (uint32_t)ld_i8x4(s + 16 + 4 * g) : 0u;
    for (int j = 0; j < 8; ++j) {
      int sc, m;
      scale_min_k4(j, s + 4, sc, m);
      const float fsc = d * (float)sc, fmn = dmin * (float)m;
      const uint32_t qw = (uint32_t)ld_i8x4(s + (kHigh ? 48 : 16) + 32 * (j / 2) + 4 * g);
      uint32_t v = (j & 1) ? (qw >> 4) & 0x0F0F0F0Fu : qw & 0x0F0F0F0Fu;
      if constexpr (kHigh) v |= ((qh >> j) & 0x01010101u) << 4;
#pragma unroll
      for (int t = 0; t < kRowsNT; ++t)
        if (t < nt) {
          const BlockQ8& xb = xq[(int64_t)(t0 + t) * nb + sb * 8 + j];
          int ai = dot4((int)v, xq_word(xb, g), 0);
          ai += __shfl_xor(ai, 1, 8);
          ai += __shfl_xor(ai, 2, 8);
          ai += __shfl_xor(ai, 4, 8);
          const float dsx = xb.d * (float)(xb.s[0] + xb.s[1]);
          acc[t] = fma_((float)ai, fsc * xb.d, acc[t]);
          acc[t] = fma_(-fmn, dsx, acc[t]);
        }
    }
  }
  if (g == 0)
#pragma unroll
    for (int t = 0; t < kRowsNT; ++t)
      if (t < nt) {
        float* o = y + (int64_t)(t0 + t) * ys + r;
        *o = accumulate ? *o + acc[t] : acc[t];
      }
}

}  // namespace

bool rows_supported(int type, int64_t cols) {
  switch (type) {
    case kF32:
    case kF16:
    case kBF16:
      return cols > 0;
    case kQ8_0:
      return cols > 0 && cols % 32 == 0;
    case kQ4_K:
    case kQ5_K:
    case kQ6_K:
      return cols > 0 && cols % 256 == 0;
    default:
      return false;
  }
}

void matmul_rows(hipStream_t s, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols, const float* x,
                 int64_t xs, const BlockQ8* xq, int n, float* y, int64_t ys, bool accumulate) {
  require(rows_supported(type, cols), "matmul_rows: type / width without a row kernel");
  if (rows <= 0 || n <= 0) return;
  const bool f = type == kF32 || type == kF16 || type == kBF16;
  require(f ? x != nullptr : xq != nullptr, "matmul_rows: missing activations (fp32 for F32/F16/BF16, BlockQ8 else)");
  const dim3 grid((unsigned)((rows + kRowsThreads / 16 - 1) / (kRowsThreads / 16)), (unsigned)((n + kRowsNT - 1) / kRowsNT));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kRowsThreads), 0, s, static_cast<const uint8_t*>(w), row_bytes, rows, cols, x,
                       xs, xq, n, y, ys, accumulate ? 1 : 0);
  };
  switch (type) {
    case kF32: go(k_rows<kF32>); break;
    case kF16: go(k_rows<kF16>); break;
    case kBF16: go(k_rows<kBF16>); break;
    case kQ8_0: go(k_rows<kQ8_0>); break;
    case kQ4_K: go(k_rows<kQ4_K>); break;
    case kQ5_K: go(k_rows<kQ5_K>); break;
    default: go(k_rows<kQ6_K>); break;
  }
  check_launch("matmul_rows");
}

void matmul_gguf(hipStream_t s, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols,
                 const BlockQ8* xq, int n, float* y, int64_t ys, bool accumulate) {
  require((type == kQ4_K || type == kQ5_K) && cols > 0 && cols % 256 == 0,
          "matmul_gguf: Q4_K / Q5_K rows of a multiple of 256 values");
  require(xq != nullptr, "matmul_gguf: missing activations");
  if (rows <= 0 || n <= 0) return;
  const dim3 grid((unsigned)((rows + kRowsThreads / 8 - 1) / (kRowsThreads / 8)), (unsigned)((n + kRowsNT - 1) / kRowsNT));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kRowsThreads), 0, s, static_cast<const uint8_t*>(w), row_bytes, rows, cols, xq,
                       n, y, ys, accumulate ? 1 : 0);
  };
  if (type == kQ5_K)
    go(k_gguf45<true>);
  else
    go(k_gguf45<false>);
  check_launch("matmul_gguf");
}

}  // namespace mk
