// Prefill GEMM for Q8_0 weights on int8 MFMA (v_mfma_i32_32x32x32_i8), bit-identical to the reference's panel kernel
// (gemm_avx512.cpp:67-102):
//   y[t][r] = sum over blocks b, in order, of fma(float(int dot of block b), f16(dw[r][b]) * dx[t][b], acc).
// K = 32 of the MFMA is exactly one Q8_0 block, so every MFMA yields the exact int32 dots of one block for a 32 x 32
// (rows x tokens) tile, and the epilogue folds them into the fp32 chains with the reference's rounding.
//
// One wavefront owns a 32-row x 32-token tile and streams its operands straight from memory: in the CDNA layout
// (layout.h) the 16-byte lo/hi planes of a row's block are exactly the A-operand bytes of the lanes (row, half), and
// the B operand is the matching 16 bytes of each token's BlockQ8. A workgroup holds 4 waves = one row tile x 4 token
// tiles (128 tokens), so the weight tile is fetched once per workgroup; workgroups of the same row tile are mapped to
// the same XCD so their weight fetches hit that XCD's L2.
//
// Accumulator layout of v_mfma_i32_32x32x32_i8 (checked on gfx950): lane l, element i holds
//   row 8 * (i / 4) + 4 * (l / 32) + i % 4, column l % 32.
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;         // token tiles per workgroup
constexpr int kTile = 32;         // rows and tokens per wave tile

struct Operands {
  v4i a, b;
  uint2 dw[4];  // f16 scales of the lane's 16 rows, 4 consecutive rows per element
  float dx;
};

__device__ __forceinline__ Operands load_block(const uint8_t* __restrict__ W, const PackedQ8_0& L, int64_t rt, int li,
                                               int h, const BlockQ8* __restrict__ xb, int64_t b) {
  Operands o;
  const int64_t r = rt * kTile + li;
  o.a = *reinterpret_cast<const v4i*>(W + L.quants(r / 8, b) + h * 128 + (r % 8) * 16);
  const int8_t* xq = reinterpret_cast<const int8_t*>(xb + b) + 8 + 16 * h;  // 8-byte aligned (40-byte blocks)
  const uint2 b0 = *reinterpret_cast<const uint2*>(xq), b1 = *reinterpret_cast<const uint2*>(xq + 8);
  o.b = v4i{(int)b0.x, (int)b0.y, (int)b1.x, (int)b1.y};
  o.dx = xb[b].d;
#pragma unroll
  for (int q = 0; q < 4; ++q) o.dw[q] = *reinterpret_cast<const uint2*>(W + L.scales(rt * 4 + q, b) + 8 * h);
  return o;
}

__global__ __launch_bounds__(kWaves * 64) void k_gemm_q8_0(const uint8_t* __restrict__ W, int64_t rows, int64_t cols,
                                                           const BlockQ8* __restrict__ x, int n, float* __restrict__ y,
                                                           int64_t ys, int accumulate, int n_rt, int n_tg) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 31, h = lane >> 5;
  // Workgroup -> (row tile, token group). Consecutive workgroups go to consecutive XCDs; the n_tg token groups of a
  // row tile are laid out 8 apart so they share an XCD (and its L2).
  const int64_t wg = blockIdx.x;
  int64_t rt, tg;
  if (n_rt % 8 == 0) {
    const int64_t xcd = wg % 8, j = wg / 8;
    rt = (j / n_tg) * 8 + xcd;
    tg = j % n_tg;
  } else {
    rt = wg / n_tg;
    tg = wg % n_tg;
  }
  const int t = (int)(tg * kWaves + w) * kTile + li;  // this lane's token (B column, C column)
  const int t_load = t < n ? t : n - 1;             // out-of-range columns compute on a valid token, never stored
  const int64_t nb = cols / 32;
  const PackedQ8_0 L{rows, nb};
  const BlockQ8* xb = x + (int64_t)t_load * nb;

  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  const v16i zero = {};
  Operands cur = load_block(W, L, rt, li, h, xb, 0);
  for (int64_t b = 0; b < nb; ++b) {
    Operands nxt;
    if (b + 1 < nb) nxt = load_block(W, L, rt, li, h, xb, b + 1);
    const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a, cur.b, zero, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pair = (i & 2) ? cur.dw[i >> 2].y : cur.dw[i >> 2].x;
      const float dw = half_to_float((uint16_t)(pair >> (16 * (i & 1))));
      acc[i] = fma_((float)c[i], dw * cur.dx, acc[i]);
    }
    cur = nxt;
  }
  if (t < n) {
    float* yt = y + (int64_t)t * ys + rt * kTile;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 8 * (i >> 2) + 4 * h + (i & 3);
      yt[m] = accumulate ? yt[m] + acc[i] : acc[i];
    }
  }
}

}  // namespace

bool gemm_q8_0_supported(int64_t rows, int64_t cols, int n) { return rows % kTile == 0 && cols % 32 == 0 && n > 8; }

void gemm_q8_0(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
               bool accumulate) {
  require(gemm_q8_0_supported(rows, cols, n), "gemm_q8_0: rows must be a multiple of 32, n > 8");
  const int n_rt = (int)(rows / kTile);
  const int n_tg = (n + kWaves * kTile - 1) / (kWaves * kTile);
  hipLaunchKernelGGL(k_gemm_q8_0, dim3((unsigned)((int64_t)n_rt * n_tg)), dim3(kWaves * 64), 0, s,
                     static_cast<const uint8_t*>(w), rows, cols, x, n, y, ys, accumulate ? 1 : 0, n_rt, n_tg);
  check_launch("gemm_q8_0");
}

}  // namespace mk
