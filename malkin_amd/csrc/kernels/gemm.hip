// Prefill GEMM for Q8_0 weights on int8 MFMA (v_mfma_i32_32x32x32_i8), bit-identical to the reference's panel kernel
// (gemm_avx512.cpp:67-102):
//   y[t][r] = sum over blocks b, in order, of fma(float(int dot of block b), f16(dw[r][b]) * dx[t][b], acc).
// K = 32 of the MFMA is exactly one Q8_0 block, so every MFMA yields the exact int32 dots of one block for a 32 x 32
// (rows x tokens) tile, and the epilogue folds them into the fp32 chains with the reference's rounding. The epilogue
// (convert, scale product, fma per output and block) is VALU work that outweighs the MFMA itself, so the kernel is
// built to keep the VALU busy: operands come from LDS, never from a global load in the inner loop.
//
// A workgroup (4 waves) owns a 64-row x 64-token tile, one 32 x 32 quarter per wave, and walks the K dimension in
// stages of kKB blocks. A stage holds, in LDS:
//   A  [kKB][64 rows][32 B]   the rows' quants (copied from the CDNA planes of layout.h),
//   B  [kKB][64 tok][32 B]    the tokens' BlockQ8 quants,
//   dw [kKB][64 rows] f32     weight scales, converted from f16 once per stage,
//   dx [kKB][64 tok]  f32     activation scales.
// Rows of A and B are 32 bytes with their two 16-byte halves swapped on every other group of 8 rows, so the MFMA
// operand reads (lane l: row l % 32, half l / 32) hit distinct banks. Two stages alternate: while the waves compute
// stage s, the next stage's global loads are in flight in registers and are stored after the compute.
//
// Accumulator layout of v_mfma_i32_32x32x32_i8 (checked on gfx950): lane l, element i holds
//   row 8 * (i / 4) + 4 * (l / 32) + i % 4, column l % 32.
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kRowsT = 64, kTokT = 64;  // workgroup tile
constexpr int kKB = 8;                  // blocks per stage

struct StageLds {
  static constexpr int a = 0;                           // kKB * 64 * 32 bytes
  static constexpr int b = a + kKB * kRowsT * 32;       // kKB * 64 * 32
  static constexpr int dw = b + kKB * kTokT * 32;       // kKB * 64 floats
  static constexpr int dx = dw + kKB * kRowsT * 4;      // kKB * 64 floats
  static constexpr int bytes = dx + kKB * kTokT * 4;
};

// Byte offset of half h (0/1) of row r within a [64][32 B] operand slab.
__device__ __forceinline__ int slab_off(int r, int h) { return r * 32 + ((h ^ ((r >> 3) & 1)) << 4); }


__global__ __launch_bounds__(kThreads) void k_gemm_q8_0(const uint8_t* W, int64_t rows, int64_t cols,
                                                        const BlockQ8* x, int n, float* __restrict__ y,
                                                        int64_t ys, int accumulate, int n_rt, int n_tt) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wt = w >> 1;  // wave quarter: rows 32 wr, tokens 32 wt
  // Workgroup -> (row tile, token tile). Consecutive workgroups go to consecutive XCDs; the token tiles of a row tile
  // are placed 8 apart so they share an XCD and its L2 holds the rows once.
  int rt, tt;
  {
    const int wg = blockIdx.x;
    if (n_rt % 8 == 0) {
      const int xcd = wg % 8, j = wg / 8;
      rt = (j / n_tt) * 8 + xcd;
      tt = j % n_tt;
    } else {
      rt = wg / n_tt;
      tt = wg % n_tt;
    }
  }
  const int nb = (int)(cols / 32);
  const PackedQ8_0 L{rows, nb};
  const int64_t g0 = (int64_t)rt * (kRowsT / 8);                  // first 8-row group of the tile
  const int ngroups = (int)min<int64_t>(kRowsT / 8, rows / 8 - g0);  // 8 or 4 (rows % 64 == 32)
  const int t0 = tt * kTokT;
  const int nstages = (nb + kKB - 1) / kKB;

  // Copy mapping (loads never predicated: past the matrix they re-read valid data, unused).
  //   A piece p = tid + 256 k: block p / 128, group (p / 16) % 8, plane (p / 8) % 2, row-in-group p % 8.
  //   B word  q = tid + 256 k: token q / 40, word q % 40 of its 8 consecutive BlockQ8 (5 words each).
  //   scales: thread tid < 64: block tid / 8, group tid % 8.
  // One stage's global data, in registers between the load and the store to LDS: A, 1024 16-byte pieces per stage
  // (4 per thread); B, 512 (token, block) BlockQ8 = 2560 8-byte words (10 per thread); weight scales, 64 (group,
  // block) pieces of 8 f16 (threads 0..63).
  v4i ra[4];
  v2i rb[10];
  v4i rs;
  auto load_stage = [&](int s) __attribute__((always_inline)) {
    const int b0 = min(s, nstages - 1) * kKB;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int p = tid + kThreads * k;
      const int b = min(b0 + p / 128, nb - 1), gi = min((p / 16) % 8, ngroups - 1), pl = (p / 8) % 2, r8 = p % 8;
      ra[k] = *reinterpret_cast<const v4i*>(W + L.quants(g0 + gi, b) + pl * 128 + r8 * 16);
    }
#pragma unroll
    for (int k = 0; k < 10; ++k) {
      const int q = tid + kThreads * k;
      const int tok = min(t0 + q / 40, n - 1), wd = q % 40;
      const int b = min(b0 + wd / 5, nb - 1);
      rb[k] = reinterpret_cast<const v2i*>(x + (int64_t)tok * nb + b)[wd % 5];
    }
    {
      const int b = min(b0 + (tid & 63) / 8, nb - 1), gi = min(tid % 8, ngroups - 1);
      rs = *reinterpret_cast<const v4i*>(W + L.scales(g0 + gi, b));
    }
  };
  auto store_stage = [&](int buf) __attribute__((always_inline)) {
    uint8_t* st = smem + buf * StageLds::bytes;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int p = tid + kThreads * k;
      const int bl = p / 128, gi = (p / 16) % 8, pl = (p / 8) % 2, r8 = p % 8;
      *reinterpret_cast<v4i*>(st + StageLds::a + bl * kRowsT * 32 + slab_off(gi * 8 + r8, pl)) = ra[k];
    }
#pragma unroll
    for (int k = 0; k < 10; ++k) {
      const int q = tid + kThreads * k;
      const int tok = q / 40, wd = q % 40, bl = wd / 5, part = wd % 5;
      if (part == 0) {
        reinterpret_cast<float*>(st + StageLds::dx)[bl * kTokT + tok] = __int_as_float(rb[k].x);  // d; s unused
      } else {
        // qs bytes 8 (part - 1) .. + 7: half (part - 1) / 2, 8-byte word (part - 1) % 2 of it
        const int h = (part - 1) >> 1, wi = (part - 1) & 1;
        *reinterpret_cast<v2i*>(st + StageLds::b + bl * kTokT * 32 + slab_off(tok, h) + 8 * wi) = rb[k];
      }
    }
    if (tid < 64) {
      const int bl = tid / 8, gi = tid % 8;
      const uint32_t hw[4] = {(uint32_t)rs.x, (uint32_t)rs.y, (uint32_t)rs.z, (uint32_t)rs.w};
      float f[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = half_to_float((uint16_t)(hw[i >> 1] >> (16 * (i & 1))));
      float4* d = reinterpret_cast<float4*>(st + StageLds::dw + (bl * kRowsT + gi * 8) * 4);
      d[0] = make_float4(f[0], f[1], f[2], f[3]);
      d[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
  };

  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  const v16i zero = {};
  const int li = lane & 31, h = lane >> 5;
  const int arow = 32 * wr + li, btok = 32 * wt + li;

  // Block bl of a stage: MFMA, then the epilogue in block order.
  auto block = [&](const uint8_t* st, int bl) __attribute__((always_inline)) {
    const v4i a = *reinterpret_cast<const v4i*>(st + StageLds::a + bl * kRowsT * 32 + slab_off(arow, h));
    const v4i bv = *reinterpret_cast<const v4i*>(st + StageLds::b + bl * kTokT * 32 + slab_off(btok, h));
    const float dx = reinterpret_cast<const float*>(st + StageLds::dx)[bl * kTokT + btok];
    const float4* dw = reinterpret_cast<const float4*>(st + StageLds::dw + (bl * kRowsT + 32 * wr + 4 * h) * 4);
    float dwv[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 d4 = dw[2 * q];  // rows 32 wr + 8 q + 4 h .. + 3
      dwv[4 * q] = d4.x, dwv[4 * q + 1] = d4.y, dwv[4 * q + 2] = d4.z, dwv[4 * q + 3] = d4.w;
    }
    const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bv, zero, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = fma_((float)c[i], dwv[i] * dx, acc[i]);
  };

  load_stage(0);
  store_stage(0);
  load_stage(1);
  lds_barrier();
  for (int s = 0; s < nstages; ++s) {
    const uint8_t* st = smem + (s & 1) * StageLds::bytes;
    const int kb = min(kKB, nb - s * kKB);
    if (kb == kKB) {
#pragma unroll
      for (int bl = 0; bl < kKB; ++bl) block(st, bl);
    } else {
      for (int bl = 0; bl < kb; ++bl) block(st, bl);
    }
    if (s + 1 < nstages) store_stage((s + 1) & 1);
    lds_barrier();
    load_stage(s + 2);
  }

  const int t = t0 + btok;
  if (t < n && 32 * wr < 8 * ngroups) {
    float* yt = y + (int64_t)t * ys + (int64_t)rt * kRowsT + 32 * wr;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 8 * (i >> 2) + 4 * h + (i & 3);
      yt[m] = accumulate ? yt[m] + acc[i] : acc[i];
    }
  }
}

}  // namespace

bool gemm_q8_0_supported(int64_t rows, int64_t cols, int n) { return rows % 32 == 0 && cols % 32 == 0 && n > 8; }

void gemm_q8_0(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
               bool accumulate) {
  require(gemm_q8_0_supported(rows, cols, n), "gemm_q8_0: rows must be a multiple of 32, n > 8");
  const int n_rt = (int)((rows + kRowsT - 1) / kRowsT);
  const int n_tt = (n + kTokT - 1) / kTokT;
  const size_t lds = 2 * (size_t)StageLds::bytes;
  static bool attr = false;
  if (!attr) {
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_q8_0), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds),
          "hipFuncSetAttribute");
    attr = true;
  }
  hipLaunchKernelGGL(k_gemm_q8_0, dim3((unsigned)((int64_t)n_rt * n_tt)), dim3(kThreads), lds, s,
                     static_cast<const uint8_t*>(w), rows, cols, x, n, y, ys, accumulate ? 1 : 0, n_rt, n_tt);
  check_launch("gemm_q8_0");
}

}  // namespace mk
