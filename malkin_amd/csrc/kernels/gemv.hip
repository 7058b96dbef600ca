// Decode GEMV on the CDNA layout: y[t][r] = W[r] . x[t] for up to 8 tokens per workgroup, bit-identical to the
// reference's panel kernels (gemm_avx512.cpp:67-102 Q8_0, 104-155 Q4_K, 157-205 Q6_K, 268-316 Q6_K wide).
//
// The reference accumulates each output as one sequential fp32 chain over the row's blocks:
//   acc = fma(float(int dot of block b), scale_w(b) * scale_x(b), acc),  b = 0, 1, 2, ...
// The int dots are exact, so they can be computed in any order and in parallel; only the chain is sequential.
//
// A workgroup owns R-row groups g = blockIdx.x, blockIdx.x + gridDim.x, ... (the grid is what fits on the GPU at
// once) and streams them, all columns of one group after another, as one sequence of chunks of kChunk units:
//   waves 1-3 (workers): for chunk c, the int dots of every (row, unit, token) with v_dot4_i32_i8 and their per-unit
//            float terms, parked in LDS slot c % 2; each worker holds two chunks of weights in registers (A/B), so
//            chunk c + 2 is in flight while chunk c is computed;
//   wave 0 (chains): the R * NT sequential chains over chunk c - 1 while the workers compute chunk c.
// Barriers order LDS only (lds_barrier), so the weight loads stay in flight across them. The activation rows of the
// workgroup's tokens are staged in LDS once, as BlockQ8: copied (kProQ8), or made here from fp32 rows, which fuses
// the reference's quantize_acts (kProF32) or rmsnorm + quantize_acts (kProNorm, model.cpp:46-49, 362-364, 403-405)
// into the matmul, saving a launch per use on the decode path. With kEpiSilu the rows come in gate/up pairs (each
// 8-row group = 4 gate rows, then the 4 up rows of the same outputs) and the workgroup stores silu(gate) * up
// (kernels_avx512.cpp:271-280) in place of the two dot products.
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kThreads = 256;
constexpr int kGemvLdsMax = 128 * 1024;

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

// kernels.h:18-26 over the 12 packed scale bytes held in three words (q0 = bytes 0..3, ...). Byte selection by
// shifts and selects: indexing the bytes of a register-held header with a runtime j would place it in scratch.
__device__ __forceinline__ int scale_byte(uint32_t q0, uint32_t q1, uint32_t q2, int i) {
  const uint32_t w = i < 4 ? q0 : (i < 8 ? q1 : q2);
  return (int)((w >> (8 * (i & 3))) & 0xFFu);
}
__device__ __forceinline__ void scale_min_k4(int j, uint32_t q0, uint32_t q1, uint32_t q2, int& sc, int& m) {
  if (j < 4) {
    sc = scale_byte(q0, q1, q2, j) & 63;
    m = scale_byte(q0, q1, q2, j + 4) & 63;
  } else {
    const int hi = scale_byte(q0, q1, q2, j + 4);
    sc = (hi & 0xF) | ((scale_byte(q0, q1, q2, j - 4) >> 6) << 4);
    m = (hi >> 4) | ((scale_byte(q0, q1, q2, j) >> 6) << 4);
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
__device__ __forceinline__ Raw load_unit(const uint8_t* W, int64_t rows, int64_t cols, int64_t g, int rr,
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

enum : int { kProQ8 = 0, kProF32 = 1, kProNorm = 2 };
enum : int { kEpiStore = 0, kEpiSilu = 1 };
constexpr int kProPass = 2;  // fp32 prologues: 2 x 256 threads x 16 values = up to 8192 columns

template <int TYPE, bool WIDE, int R, int NT, int PRO = kProQ8>
struct GemvCfg {
  static constexpr int UQ8 = Unit<TYPE>::q8;
  static constexpr int E = (TYPE == kQ6_K && WIDE) ? 1 : Unit<TYPE>::e;
  static constexpr int kWorkers = kThreads - 64;
  // Units per pipeline step: the (row, unit) pairs of a chunk spread evenly over the workers. Measured on MI355X
  // (Qwen3-8B decode shapes, one token): 48 units beat 24, 96 and 144 (a shorter fill and drain per row group), and
  // a third or fourth register set in flight did not help.
  static constexpr int kChunk = R == 8 ? (NT <= 4 ? 48 : 24) : 24;
  static constexpr int kP = kChunk * R / kWorkers;  // pairs per worker per chunk
  static_assert(kChunk * R % kWorkers == 0, "chunk must split evenly over the workers");
  static_assert(R * NT <= 64, "one chain per lane of wave 0");
  // Units the chain reads per group; it runs whole groups, over zero terms past the last unit.
  static constexpr int kG = (TYPE == kQ4_K || (TYPE == kQ6_K && !WIDE)) ? 4 : 8;
  static_assert(kChunk % kG == 0, "groups tile the chunk");
  // Term slot: per chain lane (token t, row r) the chunk's units in order, E floats each, plus one group of padding,
  // plus 4 floats against bank conflicts (rows stay 16-byte aligned). Q4_K mins:
  // per row, 2 floats per unit, laid out the same way.
  static constexpr int kLane = (kChunk + kG) * E + 4;
  static constexpr int kSlot = NT * R * kLane;
  static constexpr int kMnRow = TYPE == kQ4_K ? (kChunk + kG) * 2 + 4 : 0;
  static constexpr int kMnSlot = R * kMnRow;
  static constexpr bool kXsc = TYPE == kQ4_K || (TYPE == kQ6_K && WIDE);  // per-block activation scale terms
  __host__ __device__ static int64_t xsc_row(int64_t nq8) { return nq8 + 16; }  // + zero pad: groups read past the end
  // kProNorm: the rows, transposed for the sum-of-squares chains ([NT][16][sumsq_tstride]).
  static size_t norm_floats(int64_t cols) {
    return PRO == kProNorm ? (size_t)NT * 16 * sumsq_tstride((int)(cols / 16)) : 0;
  }
  static size_t lds_bytes(int64_t cols) {
    const int64_t nq8 = cols / 32;
    return (size_t)NT * nq8 * 40 + 2 * (size_t)(kSlot + kMnSlot) * 4 + (kXsc ? (size_t)NT * xsc_row(nq8) * 4 : 0) +
           norm_floats(cols) * 4;
  }
};

template <int TYPE, bool WIDE, int R, int NT, int PRO, int EPI>
__global__ __launch_bounds__(kThreads) void k_gemv(const uint8_t* W, int64_t rows, int64_t cols, GemvIn in, int n,
                                                   float* __restrict__ y, int64_t ys, int accumulate) {
  using C = GemvCfg<TYPE, WIDE, R, NT, PRO>;
  const BlockQ8* __restrict__ x = in.xq;
  constexpr int UQ8 = C::UQ8, E = C::E, kChunk = C::kChunk, kP = C::kP, kG = C::kG;
  extern __shared__ int smem[];
  const int nq8 = (int)(cols / 32), nu = nq8 / UQ8;
  const int t0 = blockIdx.y * NT;
  const int nt = min(NT, n - t0);
  const int tid = threadIdx.x;
  const int nc = (nu + kChunk - 1) / kChunk;                // chunks per row group
  const int ngroups = (int)(rows / R);
  const int mine = (ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;  // row groups of this WG
  const int nq = mine * nc;                                  // chunks of this workgroup, in order
  // Chunk q of this workgroup: row group rg(q) (in 8-row groups g0(q)), chunk q % nc of its columns.
  auto rg = [&](int q) { return (int)blockIdx.x + (q / nc) * (int)gridDim.x; };

  int* xs = smem;                                                   // [NT][nq8][10]: BlockQ8 rows
  float* res = reinterpret_cast<float*>(xs + NT * nq8 * 10);        // [2][kSlot]
  float* mnv = res + 2 * C::kSlot;                                  // Q4_K: [2][kMnSlot]
  float* xsc = mnv + 2 * C::kMnSlot;                                // [NT][xsc_row]: Q4_K dx (s0 + s1), Q6_K wide dx
  const int xrow = (int)C::xsc_row(nq8);
  float* tr = xsc + (C::kXsc ? NT * xrow : 0);                      // kProNorm: [NT][16][tstride]

  // Waves 1-3 are the workers: pair f = wi + k * kWorkers of a chunk is (unit f / R, row f % R), and two chunks are
  // in flight (register sets A/B). Every wave issues the same sequence of loads, never predicated: wave 0 repeats
  // wave 1's (cache hits, unused), and past the last chunk or unit a load re-reads the last valid one. The compiler's
  // wait counts are then exact on every path, so waiting for chunk c never waits for chunk c + 1.
  const bool worker = tid >= 64;
  const int wi = worker ? tid - 64 : tid;
  Raw ra[kP], rb[kP];
  auto load = [&](Raw(&r)[kP], int q) {
    const int qq = min(q, nq - 1);
    const int64_t g0 = (int64_t)rg(qq) * (R / 8);
    const int cc = qq % nc;
#pragma unroll
    for (int k = 0; k < kP; ++k) {
      const int f = wi + k * C::kWorkers;
      const int u = min(cc * kChunk + f / R, nu - 1);
      r[k] = load_unit<TYPE>(W, rows, cols, g0 + (f % R) / 8, (f % R) % 8, u);
    }
  };

  // Activation rows: 8-byte loads (BlockQ8 is 8-byte aligned), a pass of kStage loads per thread at a time. The
  // first pass is issued before the first two weight chunks, so storing it to LDS waits for it alone (loads
  // complete in issue order).
  constexpr int kStage = 8;
  const int words = nq8 * 5;  // 8-byte words per token
  const int total = nt * words;
  auto stage_load = [&](uint2(&v)[kStage], int i0) {
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      const int i = i0 + k * kThreads;
      if (i < total) {
        const int t = i / words;
        v[k] = reinterpret_cast<const uint2*>(x + (int64_t)(t0 + t) * nq8)[i - t * words];
      }
    }
  };
  auto stage_store = [&](const uint2(&v)[kStage], int i0) {
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      const int i = i0 + k * kThreads;
      if (i < total) {
        const int t = i / words;
        reinterpret_cast<uint2*>(xs + t * nq8 * 10)[i - t * words] = v[k];
      }
    }
  };
  if constexpr (PRO == kProQ8) {
    {
      uint2 xv[kStage];
      stage_load(xv, tid);
      load(ra, 0);
      load(rb, 1);
      stage_store(xv, tid);
    }
    for (int i0 = tid + kThreads * kStage; i0 < total; i0 += kThreads * kStage) {
      uint2 v[kStage];
      stage_load(v, i0);
      stage_store(v, i0);
    }
    lds_barrier();
  } else if constexpr (PRO == kProF32) {
    // fp32 rows, quantized pass by pass: thread tid takes the 16-value chunk c16 = tid + 256 p (half a Q8 block) of
    // every token row. The first pass is loaded before the weight loads, so it waits for nothing else.
    const int per = nq8 * 2;  // 16-value chunks per row
    auto pass = [&](float (&v)[NT][16], int p, bool fetch) {
      const int c16 = tid + p * kThreads;
      if (fetch) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (t < nt && c16 < per) {
            const float* xr = in.xf + (int64_t)(t0 + t) * in.xfs + 16 * c16;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const float4 a = *reinterpret_cast<const float4*>(xr + 4 * k);
              v[t][4 * k] = a.x, v[t][4 * k + 1] = a.y, v[t][4 * k + 2] = a.z, v[t][4 * k + 3] = a.w;
            }
          }
        }
        return;
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t >= nt) break;  // uniform
        // per is even (cols % 32 == 0): both halves of a block are in the row or neither is.
        quantize_half_block(v[t], c16 & 1, c16 < per, reinterpret_cast<BlockQ8*>(xs + t * nq8 * 10) + c16 / 2);
      }
    };
    // One token: the first kPre passes (12288 columns) are all loaded before the weights, so the row costs one
    // memory round trip instead of one per pass.
    constexpr int kPre = NT == 1 ? 3 : 1;
    {
      float v[kPre][NT][16];
#pragma unroll
      for (int p = 0; p < kPre; ++p)
        if (p == 0 || p * kThreads < per) pass(v[p], p, true);  // uniform
      load(ra, 0);
      load(rb, 1);
#pragma unroll
      for (int p = 0; p < kPre; ++p)
        if (p == 0 || p * kThreads < per) pass(v[p], p, false);
    }
    for (int p = kPre; p * kThreads < per; ++p) {  // uniform
      float v[NT][16];
      pass(v, p, true);
      pass(v, p, false);
    }
    lds_barrier();
  } else {
    // rmsnorm + quantization: thread tid owns the 16-value chunks c16 = tid + 256 p (half a Q8 block each) of every
    // token row, read with 16-byte loads, then its norm weights. The rows go to LDS (transposed, for the chains) and
    // are read back for the scaling.
    const int per = nq8 * 2;  // 16-value chunks per row
    const int tstride = sumsq_tstride(per);
    float v[NT][kProPass][16];
#pragma unroll
    for (int p = 0; p < kProPass; ++p) {
      const int c16 = tid + p * kThreads;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t < nt && c16 < per) {
          const float* xr = in.xf + (int64_t)(t0 + t) * in.xfs + 16 * c16;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float4 a = *reinterpret_cast<const float4*>(xr + 4 * k);
            v[t][p][4 * k] = a.x, v[t][p][4 * k + 1] = a.y, v[t][p][4 * k + 2] = a.z, v[t][p][4 * k + 3] = a.w;
          }
        }
      }
    }
    // The norm weights next (never predicated: past the row they re-read its last chunk, unused). Both wait for
    // nothing else: the weight chunks are issued only once the rows are stored, so that no workgroup's rows queue
    // behind the other workgroups' weight streams (the norm's dependent chain is the critical path here).
    float wv[kProPass][16];
#pragma unroll
    for (int p = 0; p < kProPass; ++p) {
      const int c16 = min(tid + p * kThreads, per - 1);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 w4 = reinterpret_cast<const float4*>(in.nw + 16 * c16)[k];
        wv[p][4 * k] = w4.x, wv[p][4 * k + 1] = w4.y, wv[p][4 * k + 2] = w4.z, wv[p][4 * k + 3] = w4.w;
      }
    }
    __shared__ float scale_s[NT];
    {
      // rmsnorm (model.cpp:46-49): 16 sequential lane chains per token over the transposed copy (zero-padded),
      // halving tree.
      const int padded = sumsq_padded(per);
#pragma unroll
      for (int p = 0; p < kProPass; ++p) {
        const int c16 = tid + p * kThreads;
        if (c16 < padded) {
#pragma unroll
          for (int t = 0; t < NT; ++t)
            if (t < nt) {
#pragma unroll
              for (int c = 0; c < 16; ++c) tr[(t * 16 + c) * tstride + c16] = c16 < per ? v[t][p][c] : 0.0f;
            }
        }
      }
      load(ra, 0);
      load(rb, 1);
      lds_barrier();
      if (tid < 16 * nt) {
        float acc = sumsq_lane_chain(tr + tid * tstride, per);  // token tid / 16, lane tid % 16
        acc = reduce16_lanes(acc);
        if ((tid & 15) == 0) scale_s[tid >> 4] = 1.0f / sqrtf(acc / (float)cols + in.eps);
      }
      lds_barrier();
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t >= nt) break;  // uniform
      BlockQ8* row = reinterpret_cast<BlockQ8*>(xs + t * nq8 * 10);
#pragma unroll
      for (int p = 0; p < kProPass; ++p) {
        if (p * kThreads >= per) break;  // uniform
        const int c16 = tid + p * kThreads;
        float yv[16];
        const float sc = scale_s[t];
        if (c16 < per) {
#pragma unroll
          for (int c = 0; c < 16; ++c) yv[c] = tr[(t * 16 + c) * tstride + c16] * sc * wv[p][c];
        }
        // per is even (cols % 32 == 0): both halves of a block are in the row or neither is.
        quantize_half_block(yv, c16 & 1, c16 < per, row + c16 / 2);
      }
    }
    lds_barrier();
  }
  if constexpr (C::kXsc) {
    for (int i = tid; i < NT * xrow; i += kThreads) {
      const int t = i / xrow, b = i - t * xrow;
      float v = 0.0f;
      if (t < nt && b < nq8) {
        const int* xq = xs + (t * nq8 + b) * 10;
        v = TYPE == kQ4_K ? xd(xq) * (float)(xs0(xq) + xs1(xq)) : xd(xq);
      }
      xsc[i] = v;
    }
    lds_barrier();
  }

  // Phase 1 of chunk c for one register set; units past the last write zero terms.
  auto dots = [&](const Raw(&raw)[kP], int q) {
    const int c = q % nc;
    float* slot = res + (q & 1) * C::kSlot;
#pragma unroll
    for (int k = 0; k < kP; ++k) {
      const int f = wi + k * C::kWorkers;
      const int ul = f / R, r = f % R;
      const int u = c * kChunk + ul;
      const bool live = u < nu;
      const Raw& w = raw[k];
      if constexpr (TYPE == kQ8_0) {
        const float dw = half_to_float((uint16_t)w.s);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (t < nt) {
            const int* xq = xs + (t * nq8 + (live ? u : 0)) * 10;
            float* e = slot + (t * R + r) * C::kLane + ul * E;
            *reinterpret_cast<float2*>(e) =
                live ? make_float2((float)dot8(w.a, w.b, xq), dw * xd(xq)) : make_float2(0.0f, 0.0f);
          }
        }
      } else if constexpr (TYPE == kQ4_K) {
        const int j0 = (u & 3) * 2;  // sub-blocks j0 (low nibbles) and j0 + 1 (high nibbles)
        const float d = half_to_float((uint16_t)(w.h.x & 0xFFFF)), dmin = half_to_float((uint16_t)(w.h.x >> 16));
        int sc0, m0, sc1, m1;
        scale_min_k4(j0, w.h.y, w.h.z, w.h.w, sc0, m0);
        scale_min_k4(j0 + 1, w.h.y, w.h.z, w.h.w, sc1, m1);
        const float fsc0 = d * (float)sc0, fsc1 = d * (float)sc1;
        float* mn = mnv + (q & 1) * C::kMnSlot + r * C::kMnRow + ul * 2;
        *reinterpret_cast<float2*>(mn) = live ? make_float2(dmin * (float)m0, dmin * (float)m1) : make_float2(0.0f, 0.0f);
        const uint32_t wd[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (t < nt) {
            const int* x0 = xs + (t * nq8 + (live ? u : 0) * 2) * 10;
            const int* x1 = x0 + 10;
            int a0 = 0, a1 = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              a0 = dot4((int)(wd[j] & 0x0F0F0F0Fu), x0[2 + j], a0);
              a1 = dot4((int)((wd[j] >> 4) & 0x0F0F0F0Fu), x1[2 + j], a1);
            }
            float* e = slot + (t * R + r) * C::kLane + ul * E;
            *reinterpret_cast<float4*>(e) = live ? make_float4((float)a0, fsc0 * xd(x0), (float)a1, fsc1 * xd(x1))
                                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
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
            const int* xq = xs + (t * nq8 + (live ? u : 0)) * 10;
            int a0 = 0, a1 = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) a0 = dot4(qv[j], xq[2 + j], a0);
#pragma unroll
            for (int j = 4; j < 8; ++j) a1 = dot4(qv[j], xq[2 + j], a1);
            a0 -= 32 * xs0(xq);
            a1 -= 32 * xs1(xq);
            float* e = slot + (t * R + r) * C::kLane + ul * E;
            if constexpr (WIDE) {
              e[0] = live ? fma_((float)a1, dsc1, (float)a0 * dsc0) : 0.0f;
            } else {
              *reinterpret_cast<float4*>(e) = live ? make_float4((float)a0, dsc0 * xd(xq), (float)a1, dsc1 * xd(xq))
                                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
          }
        }
      }
    }
  };

  // Phase 2 of chunk c: lane (ct, cr) runs the chain of row cr, token ct over the chunk's units in order, kG units
  // per group read with 16-byte LDS loads, the next group in flight while the current one runs. Groups run whole:
  // units past the last have zero terms, and fma(0, 0, acc) == acc.
  const int cr = tid % R, ct = tid / R;
  const bool chain_lane = tid < R * NT && ct < nt;
  float acc = 0.0f;
  struct Terms {
    float4 e[kG * E / 4 > 0 ? kG * E / 4 : 1];
    float4 m[TYPE == kQ4_K ? kG * 2 / 4 : 1];
    float4 s[C::kXsc ? (TYPE == kQ4_K ? kG * 2 / 4 : kG / 4) : 1];
  };
  auto fetch = [&](Terms& T, int q, int ul0) {
    const int c = q % nc;
    const float4* e = reinterpret_cast<const float4*>(res + (q & 1) * C::kSlot + (ct * R + cr) * C::kLane + ul0 * E);
#pragma unroll
    for (int i = 0; i < kG * E / 4; ++i) T.e[i] = e[i];
    if constexpr (TYPE == kQ4_K) {
      const float4* m = reinterpret_cast<const float4*>(mnv + (q & 1) * C::kMnSlot + cr * C::kMnRow + ul0 * 2);
      const float4* q = reinterpret_cast<const float4*>(xsc + ct * xrow + (c * kChunk + ul0) * 2);
#pragma unroll
      for (int i = 0; i < kG * 2 / 4; ++i) T.m[i] = m[i], T.s[i] = q[i];
    } else if constexpr (C::kXsc) {
      const float4* q = reinterpret_cast<const float4*>(xsc + ct * xrow + c * kChunk + ul0);
#pragma unroll
      for (int i = 0; i < kG / 4; ++i) T.s[i] = q[i];
    }
  };
  auto step = [&](const Terms& T) {
    const float* e = reinterpret_cast<const float*>(T.e);
    const float* m = reinterpret_cast<const float*>(T.m);
    const float* q = reinterpret_cast<const float*>(T.s);
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      if constexpr (TYPE == kQ8_0) {
        acc = fma_(e[2 * i], e[2 * i + 1], acc);
      } else if constexpr (TYPE == kQ4_K) {
        acc = fma_(e[4 * i], e[4 * i + 1], acc);
        acc = fma_(-m[2 * i], q[2 * i], acc);
        acc = fma_(e[4 * i + 2], e[4 * i + 3], acc);
        acc = fma_(-m[2 * i + 1], q[2 * i + 1], acc);
      } else if constexpr (WIDE) {
        acc = fma_(e[i], q[i], acc);
      } else {
        acc = fma_(e[4 * i], e[4 * i + 1], acc);
        acc = fma_(e[4 * i + 2], e[4 * i + 3], acc);
      }
    }
  };
  // Chain over chunk q; after a row group's last chunk its results are stored and the chains restart.
  auto chain = [&](int q) {
    if (!chain_lane) return;
    const int c = q % nc;
    const int cn = min(kChunk, nu - c * kChunk);
    // The chunk's kChunk / kG groups, each read kAhead groups ahead of its fmas (Q8_0's small groups: two, so that
    // the LDS latency hides behind the fmas of two groups; the larger K-quant groups: one). The reads stay inside
    // the chunk's terms whatever cn is (never predicated, so the wait before each group counts exactly the reads
    // issued after it); groups past cn are skipped (wave-uniform). Scheduling barriers keep the reads ahead.
    constexpr int kNG = kChunk / kG, kAhead = TYPE == kQ8_0 ? 2 : 1;
    Terms T[kNG];
#pragma unroll
    for (int g = 0; g < kAhead; ++g) fetch(T[g], q, g * kG);
#pragma unroll
    for (int g = 0; g < kNG; ++g) {
      if (g + kAhead < kNG) fetch(T[g + kAhead], q, (g + kAhead) * kG);
      __builtin_amdgcn_sched_barrier(0);
      if (g * kG < cn) step(T[g]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c == nc - 1) {
      if constexpr (EPI == kEpiSilu) {
        // Lanes cr and cr + 4 of an 8-lane group hold gate and up of output 4 * group + cr.
        const float up = __shfl_down(acc, 4, 8);
        if (cr < 4) {
          const float e = exp512(0.0f - acc);
          y[(int64_t)(t0 + ct) * ys + (int64_t)rg(q) * (R / 2) + cr] = (acc / (1.0f + e)) * up;
        }
      } else {
        float* o = y + (int64_t)(t0 + ct) * ys + (int64_t)rg(q) * R + cr;
        *o = accumulate ? *o + acc : acc;
      }
      acc = 0.0f;
    }
  };

  // The chains are latency-bound (one dependent fma after another) and share their SIMD with other workgroups'
  // workers: wave 0 takes issue priority over them.
  if (!worker) __builtin_amdgcn_s_setprio(2);
  for (int q = 0; q < nq; q += 2) {
    if (worker)
      dots(ra, q);
    else if (q > 0)
      chain(q - 1);
    load(ra, q + 2);
    lds_barrier();
    if (q + 1 < nq) {
      if (worker)
        dots(rb, q + 1);
      else
        chain(q);
      load(rb, q + 3);
      lds_barrier();
    }
  }
  chain(nq - 1);
}

// Resident workgroups per CU of a kernel at a given dynamic LDS size (cached per size).
template <typename K>
int resident_per_cu(K kernel, size_t lds) {
  // Cached per (kernel, LDS size): every k_gemv instantiation has the same function type.
  static const void* fns[64] = {};
  static size_t keys[64] = {};
  static int vals[64] = {};
  const void* fn = reinterpret_cast<const void*>(kernel);
  for (int i = 0; i < 64 && keys[i]; ++i)
    if (fns[i] == fn && keys[i] == lds + 1) return vals[i];
  int blocks = 0;
  check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, kThreads, lds),
        "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  blocks = blocks > 0 ? blocks : 1;
  for (int i = 0; i < 64; ++i)
    if (!keys[i]) {
      fns[i] = fn;
      keys[i] = lds + 1;
      vals[i] = blocks;
      break;
    }
  return blocks;
}

template <int TYPE, bool WIDE, int R, int NT, int PRO, int EPI = kEpiStore>
void launch(hipStream_t s, const void* w, int64_t rows, int64_t cols, const GemvIn& in, int n, float* y, int64_t ys,
            bool accumulate) {
  using C = GemvCfg<TYPE, WIDE, R, NT, PRO>;
  const size_t lds = C::lds_bytes(cols);
  static bool attr = false;  // per instantiation: allow more than the default 64 KB of dynamic LDS
  if (!attr) {
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv<TYPE, WIDE, R, NT, PRO, EPI>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kGemvLdsMax),
          "hipFuncSetAttribute");
    attr = true;
  }
  // Persistent over row groups: as many workgroups as are resident at once (per token group), each streaming its
  // share of the row groups, capped per CU. Every workgroup repeats the prologue (the fp32 rows' loads, the norm's
  // chain) and takes a dispatch slot, so fewer, longer-lived workgroups win where the occupancy allows many. Caps
  // measured on MI355X over the Qwen3-8B Q8_0 decode shapes (q|k|v norm 11.8 -> 10.4 us at 2, gate|up norm + silu
  // 24.3 -> 23.6 us at 4, plain BlockQ8 input 12.2 -> 11.9 us mean at 3) and the Qwen3-14B K-quant shapes (plain
  // input: 4 is as fast or faster at one token, 3 and 2 slower; 2 at four tokens, 47.0 -> 45.1 us on 17408 x 5120).
  constexpr int kCap = TYPE != kQ8_0 ? (PRO == kProQ8 ? (NT >= 4 ? 2 : 4) : 64)
                       : PRO == kProQ8 ? 3
                       : PRO == kProF32 ? 2
                       : EPI == kEpiSilu ? 4
                                         : 2;
  const int per_cu = std::min(kCap, resident_per_cu(k_gemv<TYPE, WIDE, R, NT, PRO, EPI>, lds));
  const int64_t groups = rows / R, tgroups = (n + NT - 1) / NT;
  const int64_t resident = (int64_t)per_cu * device_cus();
  const int64_t gx = std::max<int64_t>(1, std::min<int64_t>(groups, resident / tgroups));
  const dim3 grid((unsigned)gx, (unsigned)tgroups);
  hipLaunchKernelGGL((k_gemv<TYPE, WIDE, R, NT, PRO, EPI>), grid, dim3(kThreads), lds, s, static_cast<const uint8_t*>(w),
                     rows, cols, in, n, y, ys, accumulate ? 1 : 0);
}

// Tokens per workgroup: up to 8, fewer when the activation rows and term slots would not fit in LDS. At 3-4 tokens the
// split into token groups trades the chain wave's width (R x NT chains) against workgroups per CU and the activation
// staging each group repeats. Measured on MI355X at n = 3 and 4 (every form bit-identical): 2-token groups beat one
// 4-token group on matrices of up to 8192 rows (Q6_K: up to 2048) and on those of 12288 columns or more (Q4_K
// 5120 x 5120 at 4 tokens 19.8 -> 14.6 us, 8192 x 4096 22.0 -> 17.3, Q8_0 4096 x 12288 25.4 -> 18.9, Q6_K 1024 x 5120
// 10.4 -> 8.4); 1-token groups win on Q4_K of 16384 columns or more (5120 x 17408: 51.3 -> 42.3 us); the other
// matrices keep the 4-token group (Q6_K 17408 x 5120: 36.1 us against 37.4 in 2-token groups, 5120 x 5120 16.5
// against 17.2).
template <int TYPE>
int short_batch_nt(int64_t rows, int64_t cols) {
  if (TYPE == kQ4_K && rows <= 8192 && cols >= 16384) return 1;
  if ((rows <= 8192 && TYPE != kQ6_K) || rows <= 2048 || cols >= 12288) return 2;
  return 4;
}

template <int TYPE, bool WIDE, int R>
void launch_nt(hipStream_t s, const void* w, int64_t rows, int64_t cols, const GemvIn& in, int n, float* y, int64_t ys,
               bool acc) {
  auto fits = [&](size_t bytes) { return bytes <= (size_t)kGemvLdsMax; };
  const int nt = n == 3 || n == 4 ? short_batch_nt<TYPE>(rows, cols) : 8;
  if (n <= 1 || nt == 1 || !fits(GemvCfg<TYPE, WIDE, R, 2>::lds_bytes(cols)))
    launch<TYPE, WIDE, R, 1, kProQ8>(s, w, rows, cols, in, n, y, ys, acc);
  else if (n <= 2 || nt == 2 || !fits(GemvCfg<TYPE, WIDE, R, 4>::lds_bytes(cols)))
    launch<TYPE, WIDE, R, 2, kProQ8>(s, w, rows, cols, in, n, y, ys, acc);
  else if (n <= 4 || !fits(GemvCfg<TYPE, WIDE, R, 8>::lds_bytes(cols)))
    launch<TYPE, WIDE, R, 4, kProQ8>(s, w, rows, cols, in, n, y, ys, acc);
  else
    launch<TYPE, WIDE, R, 8, kProQ8>(s, w, rows, cols, in, n, y, ys, acc);
}

template <int TYPE, bool WIDE>
void launch_r(hipStream_t s, const void* w, int64_t rows, int64_t cols, const GemvIn& in, int n, float* y, int64_t ys,
              bool acc) {
  // One-token GEMVs over very many rows (the LM head) take 32 rows per workgroup: a quarter of the activation
  // staging per weight byte.
  if (n == 1 && rows % 32 == 0 && rows / 32 >= 2048 && GemvCfg<TYPE, WIDE, 32, 1>::lds_bytes(cols) <= kGemvLdsMax)
    launch<TYPE, WIDE, 32, 1, kProQ8>(s, w, rows, cols, in, n, y, ys, acc);
  else
    launch_nt<TYPE, WIDE, 8>(s, w, rows, cols, in, n, y, ys, acc);
}

// fp32 activations, one or two tokens per workgroup.
template <int TYPE, bool WIDE, int PRO, int EPI>
void launch_f32(hipStream_t s, const void* w, int64_t rows, int64_t cols, const GemvIn& in, int n, float* y,
                int64_t ys, bool acc) {
  if (n == 1)
    launch<TYPE, WIDE, 8, 1, PRO, EPI>(s, w, rows, cols, in, n, y, ys, acc);
  else
    launch<TYPE, WIDE, 8, 2, PRO, EPI>(s, w, rows, cols, in, n, y, ys, acc);
}

template <int PRO, int EPI>
void matmul_f32_type(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const GemvIn& in,
                     int n, float* y, int64_t ys, bool acc) {
  switch (type) {
    case kQ8_0:
      launch_f32<kQ8_0, false, PRO, EPI>(s, w, rows, cols, in, n, y, ys, acc);
      break;
    case kQ4_K:
      launch_f32<kQ4_K, false, PRO, EPI>(s, w, rows, cols, in, n, y, ys, acc);
      break;
    default:  // Q6_K; n <= 2, so never the wide panels (quant.cpp:256)
      launch_f32<kQ6_K, false, PRO, EPI>(s, w, rows, cols, in, n, y, ys, acc);
      break;
  }
}

// K-quant batches past mmv's range (or where mmv_first declines): the int8-MFMA GEMM walks K serially per 128-row
// tile, so it needs many rows or many tokens to beat the GEMV.
bool kq_gemm_first(int type, int64_t rows, int n) { return n > 16 && (rows >= 16384 || n > 32); }

// Short batches on the MFMA short-batch kernels (mmv). Measured on MI355X over the Qwen3-0.6B/4B/8B/14B shapes (Q8_0,
// Q4_K, Q6_K; results of every kernel compared bit for bit): the GEMV wins up to 2 tokens, and up to 4 except on
// matrices of more than 8192 rows in Q4_K (17408 x 5120 at 4 tokens: 46.1 vs 26.5 us) or of 24576 rows and more in
// Q8_0 (the LM head: 140 vs 116 us), and at 4 tokens on 2048..8192 rows (up to 17408 in K-quants), where the K-split
// pairs win (5120 x 17408: Q4_K 42.0 -> 37.7 us, Q6_K 50.5 -> 42.5; 7168 x 5120 Q6_K 19.7 -> 15.6; 17408 x 5120 Q6_K
// 36.3 -> 35.2; 1024 x 3072: 5.9 vs 8.1 with the GEMV); from 5 to 16 tokens mmv; from 17 to 32 tokens the same,
// except that the GEMMs' 32- and 64-token tiles win on the widest matrices and the one-wave form on Q4_K.
bool mmv_first(int type, int64_t rows, int64_t cols, int n) {
  if (n <= 2 || n > 32 || !mmv_supported(type, rows, cols, n)) return false;
  if (n == 4 && rows >= 2048 && rows <= (type == kQ8_0 ? 8192 : 17408)) return true;
  if (n <= 4) return type == kQ4_K ? rows > 8192 : type == kQ8_0 && rows >= 24576;
  if (n <= 16) return true;
  return rows < (type == kQ8_0 ? 16384 : 24576);
}
// K split inside the workgroup (k_mmv_ks) or one wave per 16-row tile (k_mmv), measured on MI355X: the K split on up
// to 8192 rows (Q4_K: up to 16 tokens), and up to 8 tokens on up to 17408 rows of K-quants (17408 x 5120 at 8 tokens:
// Q4_K 27.2 -> 26.4 us, Q6_K 38.8 -> 35.5) and 12288 of Q8_0 (12288 x 4096: 17.5 -> 15.6; 24576 x 4096: 22.4 vs
// 28.7), and Q6_K at 17..32 tokens up to 17408 rows (17408 x 5120 at 17 tokens: 53.5 -> 47.2; at 12 tokens the one-
// wave form wins there, 39.4 vs 50.2).
bool mmv_ksplit(int type, int64_t rows, int64_t cols, int n) {
  if (rows <= 8192) return n <= 16 || type != kQ4_K;
  return n <= 8 ? rows <= (type == kQ8_0 ? 12288 : 17408) : n > 16 && type == kQ6_K && rows <= 17408;
}

}  // namespace

void matmul(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* xq, int n,
            float* y, int64_t ys, bool accumulate) {
  require(n > 0, "matmul: no tokens");
  require(packed_bytes(type, rows, cols) != 0, "matmul: no kernel for this weight type/shape");
  const GemvIn in{xq, nullptr, 0, nullptr, 0.0f};
  if (mmv_first(type, rows, cols, n)) {
    mmv(s, type, wide, w, rows, cols, xq, n, y, ys, accumulate, mmv_ksplit(type, rows, cols, n));
    return;
  }
  switch (type) {
    case kQ8_0:
      if (gemm_q8_0_supported(rows, cols, n))
        gemm_q8_0(s, w, rows, cols, xq, n, y, ys, accumulate);  // prefill / batches: int8 MFMA
      else
        launch_r<kQ8_0, false>(s, w, rows, cols, in, n, y, ys, accumulate);
      break;
    case kQ4_K:
      if (gemm_kq_supported(type, rows, cols, n) && kq_gemm_first(type, rows, n))
        gemm_kq(s, type, wide, w, rows, cols, xq, n, y, ys, accumulate);  // batches: int8 MFMA
      else
        launch_r<kQ4_K, false>(s, w, rows, cols, in, n, y, ys, accumulate);
      break;
    case kQ6_K:
      // The reference switches Q6_K to its wide panels above kWideMinTokens = 16 tokens (quant.cpp:256).
      if (gemm_kq_supported(type, rows, cols, n) && kq_gemm_first(type, rows, n))
        gemm_kq(s, type, wide, w, rows, cols, xq, n, y, ys, accumulate);
      else if (wide && n > 16)
        launch_r<kQ6_K, true>(s, w, rows, cols, in, n, y, ys, accumulate);
      else
        launch_r<kQ6_K, false>(s, w, rows, cols, in, n, y, ys, accumulate);
      break;
    default:
      throw Error(MK_ERR_UNSUPPORTED, "matmul: unsupported weight type");
  }
  check_launch("matmul");
}

bool matmul_f32_supported(int type, bool, int64_t rows, int64_t cols, int n, bool norm) {
  return n >= 1 && n <= 2 && cols % 32 == 0 && (!norm || cols <= kThreads * 16 * kProPass) &&
         (int64_t)n * (cols / 32) * 40 <= 64 * 1024 && packed_bytes(type, rows, cols) != 0 &&
         (type == kQ8_0 || type == kQ4_K || type == kQ6_K);
}

void matmul_f32(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const float* xf,
                int64_t xfs, const float* nw, float eps, int n, float* y, int64_t ys, bool accumulate,
                bool silu_pairs) {
  require(matmul_f32_supported(type, wide, rows, cols, n, nw != nullptr),
          "matmul_f32: needs 1 or 2 tokens, a multiple of 32 columns (<= 8192 with rmsnorm) and a quantized weight");
  require(!silu_pairs || !accumulate, "matmul_f32: the silu epilogue does not accumulate");
  const GemvIn in{nullptr, xf, xfs, nw, eps};
  if (nw && silu_pairs)
    matmul_f32_type<kProNorm, kEpiSilu>(s, type, wide, w, rows, cols, in, n, y, ys, false);
  else if (nw)
    matmul_f32_type<kProNorm, kEpiStore>(s, type, wide, w, rows, cols, in, n, y, ys, accumulate);
  else if (silu_pairs)
    matmul_f32_type<kProF32, kEpiSilu>(s, type, wide, w, rows, cols, in, n, y, ys, false);
  else
    matmul_f32_type<kProF32, kEpiStore>(s, type, wide, w, rows, cols, in, n, y, ys, accumulate);
  check_launch("matmul_f32");
}

}  // namespace mk
