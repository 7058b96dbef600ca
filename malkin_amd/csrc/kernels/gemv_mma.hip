// Short-batch matmul (2..32 tokens) on int8 MFMA, bit-identical to the reference's panel kernels: the continuous-
// batching decode steps, tree verification batches and short prompt tails, where the batch is too small for the
// prefill GEMMs' 32- and 64-token tiles and too large for the decode GEMV's per-token VALU dot products.
//
// Per output (row r, token t) the reference keeps one fp32 chain over the row's 32-weight units in order
// (gemm_avx512.cpp:67-102 Q8_0, 104-155 Q4_K, 157-205 Q6_K, 268-316 Q6_K wide):
//   Q8_0            acc = fma(float(ai), f16(dw) * dx, acc)
//   Q4_K (sub-block j)  acc = fma(float(ai), (d sc_j) * dx, acc);  acc = fma(-(dmin m_j), dx * (s0 + s1), acc)
//   Q6_K compact (halves h = 0, 1)  acc = fma(float(ai_h), (d sc_h) * dx, acc)
//   Q6_K wide       acc = fma(fma(float(ai_1), d sc_1, float(ai_0) * (d sc_0)), dx, acc)
// where ai is the exact int32 dot of the unit (of its 16-value half for Q6_K) with the BlockQ8 activation quants.
//
// A workgroup is two waves; wave w owns 16 rows (two 8-row groups of the packed layout) and computes, per unit, the
// 16 x 16 (tokens x rows) int dots with one v_mfma_i32_16x16x32_i8 (two for Q6_K: one per half, the other half's
// operand bytes zeroed) per 16-token tile, then applies the reference's epilogue to the 4 accumulator elements of
// each lane (tokens 4 (l / 16) + i, row l % 16): every chain lives in one accumulator element and advances unit by
// unit in order. The operands stream through a ring of NS LDS stages of 8 units (256 weights), filled by direct
// global -> LDS loads NS - 1 stages ahead: each wave copies its own rows' packed records (whole 1 KB pieces of the
// layout.h planes) and half of the stage's activation quants and scales, shared by both waves.
//
// Operand layouts of v_mfma_i32_16x16x32_i8 (A: tokens x K, B: K x rows): lane l holds A[l % 16][8 (l / 16) ..
// 8 (l / 16) + 7] and B[8 (l / 16) .. + 7][l % 16]; result element i of lane l is (token 4 (l / 16) + i, row l % 16).
// The int dot of a unit is independent of the order of its K index, so each lane may take any 8 of the unit's 32
// weights as long as its A bytes are the matching activations; here lane quarter c = l / 16 takes weights
// 8 c .. 8 c + 7 in natural order.
#include <utility>

#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves = 2, kThreads = 64 * kWaves;
constexpr int kRowsW = 16;                // rows per wave (MFMA N)
constexpr int kRowsT = kRowsW * kWaves;   // rows per workgroup
constexpr int kUnits = 8;                 // 32-weight units per stage

__device__ __forceinline__ void ld16(const void* g, uint8_t* l) { lds_copy16(g, l); }
__device__ __forceinline__ void ld4(const void* g, uint8_t* l) { lds_copy4(g, l); }

// q - 32 per byte for bytes q < 64 (never borrows across bytes).
__device__ __forceinline__ uint32_t minus32(uint32_t q) { return ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u; }

// scale_min_k4 (kernels.h:18-26) over the 12 packed scale bytes of a Q4_K header held in q0..q2.
__device__ __forceinline__ int hbyte(uint32_t q0, uint32_t q1, uint32_t q2, int i) {
  const uint32_t w = i < 4 ? q0 : (i < 8 ? q1 : q2);
  return (int)((w >> (8 * (i & 3))) & 0xFFu);
}
// The same for a wave-uniform j known only at run time, without branches: both forms, merged under a mask.
__device__ __forceinline__ void scale_min_sel(int j, uint32_t q0, uint32_t q1, uint32_t q2, int& sc, int& m) {
  const int sh = 8 * (j & 3), low = -(int)(j < 4);  // all ones for j < 4
  const int b0 = (int)((q0 >> sh) & 0xFFu), b1 = (int)((q1 >> sh) & 0xFFu), b2 = (int)((q2 >> sh) & 0xFFu);
  sc = ((b0 & 63) & low) | (((b2 & 0xF) | ((b0 >> 6) << 4)) & ~low);
  m = ((b1 & 63) & low) | (((b2 >> 4) | ((b1 >> 6) << 4)) & ~low);
}
__device__ __forceinline__ void scale_min(int j, uint32_t q0, uint32_t q1, uint32_t q2, int& sc, int& m) {
  if (j < 4) {
    sc = hbyte(q0, q1, q2, j) & 63;
    m = hbyte(q0, q1, q2, j + 4) & 63;
  } else {
    const int hi = hbyte(q0, q1, q2, j + 4);
    sc = (hi & 0xF) | ((hbyte(q0, q1, q2, j - 4) >> 6) << 4);
    m = (hi >> 4) | ((hbyte(q0, q1, q2, j) >> 6) << 4);
  }
}

// Stage layout (bytes) for NTT 16-token tiles. Per wave: W (its 16 rows' packed quants for the stage's 8 units), S (the
// rows' scale records: Q8_0 f16 scales, Q6_K int8 sub-scales, Q4_K headers), D (Q6_K: f16 d; 256 B because the copy
// is lane-linear). Shared: X [unit][token][32 B] quants, DX [unit][token] f32 d, XS [unit][token] (s0, s1) (Q4_K).
template <int TYPE, int NTT>
struct MmvLds {
  static constexpr int w_bytes = TYPE == kQ8_0 ? 2 * 8 * 256 : TYPE == kQ6_K ? 2 * 1536 : 2 * 1024;
  static constexpr int per_wave = w_bytes + 256 + (TYPE == kQ6_K ? 256 : 0);
  static constexpr int s_off = w_bytes, d_off = w_bytes + 256;
  static constexpr int x = kWaves * per_wave;
  static constexpr int dx = x + kUnits * 16 * NTT * 32;
  static constexpr int xs = dx + kUnits * 16 * NTT * 4;
  static constexpr int bytes = xs + (TYPE == kQ4_K ? kUnits * 16 * NTT * 4 : 0);
  // global -> LDS loads per wave per stage (every wave issues the same count)
  static constexpr int loads = w_bytes / 1024 + 1 + (TYPE == kQ6_K ? 1 : 0) + 2 * NTT + NTT + (TYPE == kQ4_K ? NTT : 0);
};

template <int TYPE, bool WIDE, int NTT, int NS>
__global__ __launch_bounds__(kThreads) void k_mmv(const uint8_t* W, int64_t rows, int64_t cols, const BlockQ8* x,
                                                  int n, float* __restrict__ y, int64_t ys, int accumulate) {
  using S = MmvLds<TYPE, NTT>;
  static_assert((NS - 1) * S::loads < 64, "the ring's loads must fit the vmcnt counter");
  constexpr int TS = 16 * NTT;                      // token slots per unit in X and DX
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rt = blockIdx.x;                        // 32-row tile
  const int t0 = blockIdx.y * 16 * NTT;             // first token of the tile
  const int ntok = min(16 * NTT, n - t0);           // tokens present (>= 1)
  const int nq8 = (int)(cols / 32);
  const int nst = nq8 / kUnits;                     // stages (cols % 256 == 0)
  const int64_t g0w = (int64_t)rt * 4 + 2 * wu;     // first 8-row group of this wave

  // Per-lane constant source offsets of the copies (bytes); the moving part is a wave-uniform base per stage.
  //   W: lane-linear 16-byte pieces of the wave's W region; S/D: 4-byte pieces of its scale records;
  //   X: WG pieces 2 NTT wu + k (k < 2 NTT): 1 KB each of [unit][token][32 B]; DX/XS: 256-byte pieces NTT wu + k.
  const uint8_t* xb = reinterpret_cast<const uint8_t*>(x + (int64_t)t0 * nq8);
  uint32_t x_off[2 * NTT], dx_off[NTT];
#pragma unroll
  for (int k = 0; k < 2 * NTT; ++k) {
    const int p = 1024 * (2 * NTT * wu + k) + 16 * lane;
    const int unit = p / (512 * NTT), rem = p % (512 * NTT);
    const int tok = min(rem / 32, ntok - 1), half = (rem % 32) / 16;
    x_off[k] = (uint32_t)((tok * nq8 + unit) * 40 + 8 + 16 * half);
  }
#pragma unroll
  for (int k = 0; k < NTT; ++k) {
    const int p = 256 * (NTT * wu + k) + 4 * lane;
    const int unit = p / (64 * NTT), tok = min((p % (64 * NTT)) / 4, ntok - 1);
    dx_off[k] = (uint32_t)((tok * nq8 + unit) * 40);
  }
  const uint8_t* wq;  // quants of group g0w at stage 0
  const uint8_t* ws;  // scale records of group g0w at stage 0
  const uint8_t* wd = nullptr;
  uint32_t w_off[S::w_bytes / 1024], s_off, d_off = 0;
  int64_t wq_step, ws_step;  // bytes per stage
  if constexpr (TYPE == kQ8_0) {
    const PackedQ8_0 L{rows, nq8};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int p = 1024 * k + 16 * lane;
      w_off[k] = (uint32_t)((p / 2048) * nq8 * 256 + p % 2048);
    }
    s_off = (uint32_t)((lane / 32) * nq8 * 16 + 4 * (lane % 32));
    wq = W + L.quants(g0w, 0);
    ws = W + L.scales(g0w, 0);
    wq_step = 8 * 256;
    ws_step = 8 * 16;
  } else if constexpr (TYPE == kQ6_K) {
    const int nsb = nq8 / 8;
    const PackedQ6_K L{rows, nsb};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int p = 1024 * k + 16 * lane;
      w_off[k] = (uint32_t)((p / 1536) * nsb * 1536 + p % 1536);
    }
    s_off = (uint32_t)((lane / 32) * nsb * 128 + 4 * (lane % 32));
    {
      const int p = 4 * min(lane, 7);
      d_off = (uint32_t)((p / 16) * nsb * 16 + p % 16);
    }
    wq = W + L.quants(g0w, 0, 0);
    ws = W + L.scales(g0w, 0);
    wd = W + L.dscale(g0w, 0);
    wq_step = 1536;
    ws_step = 128;
  } else {
    const int nsb = nq8 / 8;
    const PackedQ4_K L{rows, nsb};
#pragma unroll
    for (int k = 0; k < 2; ++k) w_off[k] = (uint32_t)(k * nsb * 1024 + 16 * lane);
    s_off = (uint32_t)((lane / 32) * nsb * 128 + 4 * (lane % 32));
    wq = W + L.quants(g0w, 0, 0);
    ws = W + L.headers(g0w, 0);
    wq_step = 1024;
    ws_step = 128;
  }

  auto issue = [&]<int BUF>(int sn) __attribute__((always_inline)) {
    uint8_t* st = smem + BUF * S::bytes;
    uint8_t* wv = st + wu * S::per_wave;
    const uint8_t* q = wq + (size_t)sn * wq_step;
#pragma unroll
    for (int k = 0; k < S::w_bytes / 1024; ++k) ld16(q + w_off[k], wv + 1024 * k);
    ld4(ws + (size_t)sn * ws_step + s_off, wv + S::s_off);
    if constexpr (TYPE == kQ6_K) ld4(wd + (size_t)sn * 16 + d_off, wv + S::d_off);
    const uint8_t* xs = xb + (size_t)sn * kUnits * 40;
#pragma unroll
    for (int k = 0; k < 2 * NTT; ++k) ld16(xs + x_off[k], st + S::x + 1024 * (2 * NTT * wu + k));
#pragma unroll
    for (int k = 0; k < NTT; ++k) ld4(xs + dx_off[k], st + S::dx + 256 * (NTT * wu + k));
    if constexpr (TYPE == kQ4_K) {
#pragma unroll
      for (int k = 0; k < NTT; ++k) ld4(xs + dx_off[k] + 4, st + S::xs + 256 * (NTT * wu + k));
    }
  };

  // This lane: row r = lane % 16 of the wave's 16 (group gi = r / 8, row rr = r % 8), weight quarter c = lane / 16;
  // accumulator elements i: tokens 4 c + i (+ 16 m for tile m).
  const int r = lane & 15, c = lane >> 4, gi = r >> 3, rr = r & 7;
  __shared__ __align__(16) float xsum_tab[TYPE == kQ4_K ? kWaves * kUnits * 16 * NTT : 4];
  float* xsum_w = xsum_tab + (TYPE == kQ4_K ? wu * kUnits * 16 * NTT : 0);
  float acc[NTT][4];
#pragma unroll
  for (int m = 0; m < NTT; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[m][i] = 0.0f;
  const v4i zero4 = {0, 0, 0, 0};

  auto stage = [&]<int BUF>(int s) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the buffer refilled below are done
    wait_vm_stages<S::loads, NS - 2>(min(NS - 2, nst - 1 - s));
    ring_barrier();
    if (s + NS - 1 < nst) issue.template operator()<(BUF + NS - 1) % NS>(s + NS - 1);
    const uint8_t* st = smem + BUF * S::bytes;
    const uint8_t* wv = st + wu * S::per_wave;
    if constexpr (TYPE == kQ8_0) {
#pragma unroll
      for (int u = 0; u < kUnits; ++u) {
        const long b = *reinterpret_cast<const long*>(wv + gi * 2048 + u * 256 + (c >> 1) * 128 + rr * 16 + 8 * (c & 1));
        const float dw = half_to_float(*reinterpret_cast<const uint16_t*>(wv + S::s_off + gi * 128 + u * 16 + rr * 2));
#pragma unroll
        for (int m = 0; m < NTT; ++m) {
          const long a = *reinterpret_cast<const long*>(st + S::x + (u * TS + 16 * m + r) * 32 + 8 * c);
          const float4 dx = *reinterpret_cast<const float4*>(st + S::dx + (u * TS + 16 * m + 4 * c) * 4);
          const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero4, 0, 0, 0);
          acc[m][0] = fma_((float)d[0], dw * dx.x, acc[m][0]);
          acc[m][1] = fma_((float)d[1], dw * dx.y, acc[m][1]);
          acc[m][2] = fma_((float)d[2], dw * dx.z, acc[m][2]);
          acc[m][3] = fma_((float)d[3], dw * dx.w, acc[m][3]);
        }
      }
    } else if constexpr (TYPE == kQ6_K) {
      const float dd = half_to_float(*reinterpret_cast<const uint16_t*>(wv + S::d_off + gi * 16 + rr * 2));
      const int hw = c >> 1, h = c & 1;
#pragma unroll
      for (int u = 0; u < kUnits; ++u) {
        const uint8_t* au = wv + gi * 1536 + u * 192;
        const uint2 nib = *reinterpret_cast<const uint2*>(au + rr * 16 + 8 * h);
        const uint2 hb = *reinterpret_cast<const uint2*>(au + 128 + rr * 8);
        // weights 8 c .. 8 c + 7 = q[16 hw + 8 h + 0..7] of the unit
        const uint32_t hv = (hw ? hb.y : hb.x) >> (4 * h);
        const uint32_t q0 = ((nib.x >> (4 * hw)) & 0x0F0F0F0Fu) | ((hv & 0x03030303u) << 4);
        const uint32_t q1 = ((nib.y >> (4 * hw)) & 0x0F0F0F0Fu) | (((hv >> 2) & 0x03030303u) << 4);
        const long bq = (long)(((uint64_t)minus32(q1) << 32) | minus32(q0));
        const long b0 = hw ? 0 : bq, b1 = hw ? bq : 0;
        const uint32_t scw = *reinterpret_cast<const uint16_t*>(wv + S::s_off + gi * 128 + rr * 16 + 2 * u);
        const float dsc0 = dd * (float)(int8_t)(scw & 0xFF), dsc1 = dd * (float)(int8_t)(scw >> 8);
#pragma unroll
        for (int m = 0; m < NTT; ++m) {
          const long a = *reinterpret_cast<const long*>(st + S::x + (u * TS + 16 * m + r) * 32 + 8 * c);
          const float4 dx4 = *reinterpret_cast<const float4*>(st + S::dx + (u * TS + 16 * m + 4 * c) * 4);
          const float dx[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
          const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, zero4, 0, 0, 0);
          const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, zero4, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (WIDE) {
              const float sm = fma_((float)d1[i], dsc1, (float)d0[i] * dsc0);
              acc[m][i] = fma_(sm, dx[i], acc[m][i]);
            } else {
              acc[m][i] = fma_((float)d0[i], dsc0 * dx[i], acc[m][i]);
              acc[m][i] = fma_((float)d1[i], dsc1 * dx[i], acc[m][i]);
            }
          }
        }
      }
    } else {  // Q4_K: unit u = sub-block j = u of the stage's super-block; chunk j2 = u / 2, nibble u % 2
      // dx (s0 + s1) of the stage's (unit, token) pairs (the reference's dsx, gemm_avx512.cpp:143), computed once per
      // stage and wave into the wave's table instead of once per row lane, read back as each lane's four tokens.
#pragma unroll
      for (int k = 0; k < kUnits * 16 * NTT / 64; ++k) {
        const int idx = lane + 64 * k;
        const uint32_t sx = *reinterpret_cast<const uint32_t*>(st + S::xs + idx * 4);
        const float dxv = *reinterpret_cast<const float*>(st + S::dx + idx * 4);
        xsum_w[idx] = dxv * (float)((int)(int16_t)(sx & 0xFFFF) + (int)(int16_t)(sx >> 16));
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      const uint4 hd = *reinterpret_cast<const uint4*>(wv + S::s_off + gi * 128 + rr * 16);
      const float d = half_to_float((uint16_t)(hd.x & 0xFFFF)), dmin = half_to_float((uint16_t)(hd.x >> 16));
#pragma unroll
      for (int j2 = 0; j2 < 4; ++j2) {
        const uint2 raw =
            *reinterpret_cast<const uint2*>(wv + gi * 1024 + j2 * 256 + (c >> 1) * 128 + rr * 16 + 8 * (c & 1));
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int u = 2 * j2 + e;
          const long bq = (long)(((uint64_t)((raw.y >> (4 * e)) & 0x0F0F0F0Fu) << 32) | ((raw.x >> (4 * e)) & 0x0F0F0F0Fu));
          int sc, mn;
          scale_min(u, hd.y, hd.z, hd.w, sc, mn);
          const float fsc = d * (float)sc, nmn = -(dmin * (float)mn);
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            const long a = *reinterpret_cast<const long*>(st + S::x + (u * TS + 16 * m + r) * 32 + 8 * c);
            const float4 dx4 = *reinterpret_cast<const float4*>(st + S::dx + (u * TS + 16 * m + 4 * c) * 4);
            const float4 xs4 = *reinterpret_cast<const float4*>(xsum_w + ((u * NTT + m) * 16 + 4 * c));
            const float dx[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            const float xsum[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
            const v4i dq = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq, zero4, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[m][i] = fma_((float)dq[i], fsc * dx[i], acc[m][i]);
              acc[m][i] = fma_(nmn, xsum[i], acc[m][i]);
            }
          }
        }
      }
    }
  };

  [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
    ((B < nst ? issue.template operator()<B>(B) : void()), ...);
  }(std::make_integer_sequence<int, NS - 1>{});
  for (int s = 0; s < nst; s += NS) {
    [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
      ((s + B < nst ? stage.template operator()<B>(s + B) : void()), ...);
    }(std::make_integer_sequence<int, NS>{});
  }

  const int64_t row = (int64_t)rt * kRowsT + wu * kRowsW + r;
#pragma unroll
  for (int m = 0; m < NTT; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * m + 4 * c + i;
      if (t < ntok) {
        float* o = y + (int64_t)(t0 + t) * ys + row;
        *o = accumulate ? *o + acc[m][i] : acc[m][i];
      }
    }
}

// K-split form for matrices with few rows (down and attn_output projections): KW = 4 or 8 term waves share one
// 16-row tile. Per stage of 8 units, term wave w computes the MFMA dots of units (8 / KW) w .. and their per-unit float
// terms (the operands of the reference's fmas, rounded as the reference rounds them) into LDS; the sequential chains
// of the tile's (row, token) outputs then run over the stage's 8 units in order, either on CW chain waves of their
// own one stage behind (double-buffered terms, one barrier per stage) or on the term waves themselves (after the
// next stage's terms when the terms are double-buffered, else after a second barrier). Terms per unit and
// output, E floats: Q8_0 {float(ai), dw dx}; Q6_K compact {float(ai_0), (d sc_0) dx, float(ai_1), (d sc_1) dx};
// Q6_K wide {fma(float(ai_1), d sc_1, float(ai_0) (d sc_0)), dx}; Q4_K {float(ai), (d sc) dx}; the chain applies
// acc = fma(e0, e1, acc) (and acc = fma(e2, e3, acc)). Q4_K's second fma, acc = fma(-(dmin m), dx (s0 + s1), acc),
// takes its operands from two small per-stage tables (per row and unit, per token and unit) instead.
template <int TYPE, bool WIDE>
struct Ks {
  static constexpr int E = (TYPE == kQ8_0 || TYPE == kQ4_K || (TYPE == kQ6_K && WIDE)) ? 2 : 4;
};
// TS: token slots per unit in X, DX, XS and the terms (16 NTT, or 20 for two token tiles holding at most 20 tokens,
// the tree verification batch: rows of padding tokens are neither copied nor stored).
template <int TYPE, bool WIDE, int NTT, int KW, int TS, int CW>
struct KsLds {
  static constexpr int w_bytes = TYPE == kQ8_0 ? 2 * 8 * 256 : TYPE == kQ6_K ? 2 * 1536 : 2 * 1024;
  static constexpr int s_off = w_bytes, d_off = w_bytes + 256;
  static constexpr int x = w_bytes + 256 + (TYPE == kQ6_K ? 256 : 0);
  static constexpr int dx_bytes = (kUnits * TS * 4 + 255) / 256 * 256;  // whole 256-byte copies
  static constexpr int dx = x + kUnits * TS * 32;
  static constexpr int xs = dx + dx_bytes;
  static constexpr int bytes = xs + (TYPE == kQ4_K ? dx_bytes : 0);  // one ring stage
  static constexpr int terms1 = kUnits * TS * 16 * Ks<TYPE, WIDE>::E * 4;   // one stage's terms
  // Double-buffered (stage s's terms written while stage s - 1's chains run) where two workgroups per CU still get
  // a three-stage ring in 80 KB each.
  static constexpr bool db = CW > 0 || (80 * 1024 - 2 * terms1) / bytes >= 3;
  static constexpr int terms = (db ? 2 : 1) * terms1;
  // The stage's copies are a list of pieces, 1 KB ones (W, then X) and 256-byte ones (S, D, DX, XS); wave w copies
  // pieces w, w + KW, ... (loads of them per stage, the last piece repeated past the end of the list).
  static constexpr int n_x4 = w_bytes / 1024 + kUnits * TS * 32 / 1024;
  static constexpr int n_dw = 1 + (TYPE == kQ6_K ? 1 : 0) + dx_bytes / 256 * (TYPE == kQ4_K ? 2 : 1);
  static constexpr int loads = (n_x4 + n_dw + KW - 1) / KW;
  static_assert(kUnits * TS * 32 % 1024 == 0, "X in whole 1 KB pieces");
  static_assert(w_bytes / 1024 <= KW, "every W piece in a wave's first slot");
};

// KW term waves (4 or 8), then CW chain waves (0: the term waves run the chains): each term wave computes the dots
// and terms of 8 / KW of a stage's 8 units.
// PAIR (at most 8 tokens, one token tile): a wave takes its units two at a time in one 16 x 16 MFMA tile, unit u's
// tokens in the tile's token rows 0..7 and unit u + 1's in rows 8..15. The first MFMA has unit u's activations in rows
// 0..7 (zero elsewhere) against unit u's weights, the second accumulates unit u + 1's activations in rows 8..15
// against unit u + 1's weights, so result element i of lane quarter c is (unit u + c / 2, token 4 (c % 2) + i):
// exact int dots of both units, and no epilogue work for padding token columns.
template <int TYPE, bool WIDE, int NTT, int NS, int KW, bool PAIR, int TS, int CW>
__global__ __launch_bounds__(64 * (KW + CW)) void k_mmv_ks(const uint8_t* W, int64_t rows, int64_t cols,
                                                            const BlockQ8* x, int n, float* __restrict__ y,
                                                            int64_t ys, int accumulate) {
  using S = KsLds<TYPE, WIDE, NTT, KW, TS, CW>;
  static_assert(!PAIR || (NTT == 1 && kUnits / KW % 2 == 0), "pairs: one token tile, an even number of units per wave");
  static_assert(NTT == 2 ? TS > 16 && TS <= 32 && TS % 4 == 0 : TS == (PAIR ? 8 : 16), "token slots");
  constexpr int E = Ks<TYPE, WIDE>::E;
  constexpr int UPW = kUnits / KW;                  // units per wave and stage
  constexpr int CT = 4 * (CW ? CW : KW);            // token rows of the chain threads (16 rows x CT tokens)
  constexpr int CPT = (TS + CT - 1) / CT;           // chains per thread
  static_assert((NS - 1) * S::loads < 64, "the ring's loads must fit the vmcnt counter");
  extern __shared__ __align__(16) uint8_t smem[];
  float* terms_base = reinterpret_cast<float*>(smem + NS * S::bytes);  // [2][unit][token][row][E]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rt = blockIdx.x;                        // 16-row tile
  const int t0 = blockIdx.y * 16 * NTT;
  const int ntok = min(16 * NTT, n - t0);
  const int nq8 = (int)(cols / 32);
  const int nst = nq8 / kUnits;
  const int64_t g0 = (int64_t)rt * 2;               // first 8-row group

  // Copies: the piece list of KsLds. Source offset of the activation bytes this lane copies into X byte p (1 KB
  // pieces: 16 bytes a lane) or DX / XS byte p (256-byte pieces: 4 bytes a lane); slots of padding tokens copy the last
  // token's bytes.
  constexpr int WP = S::w_bytes / 1024;
  const uint8_t* xb = reinterpret_cast<const uint8_t*>(x + (int64_t)t0 * nq8);
  auto x_src = [&](int p) __attribute__((always_inline)) {
    const int unit = p / (TS * 32), rem = p % (TS * 32);
    const int tok = min(rem / 32, ntok - 1), half = (rem % 32) / 16;
    return (uint32_t)((tok * nq8 + unit) * 40 + 8 + 16 * half);
  };
  auto dx_src = [&](int p) __attribute__((always_inline)) {
    const int unit = min(p / (TS * 4), kUnits - 1), tok = min((p % (TS * 4)) / 4, ntok - 1);
    return (uint32_t)((tok * nq8 + unit) * 40);
  };
  const int wp = min(wu, WP - 1);
  const uint8_t *wq, *ws, *wd = nullptr;
  uint32_t w_off, s_off, d_off = 0;
  int64_t wq_step, ws_step;
  if constexpr (TYPE == kQ8_0) {
    const PackedQ8_0 L{rows, nq8};
    const int p = 1024 * wp + 16 * lane;
    w_off = (uint32_t)((p / 2048) * nq8 * 256 + p % 2048);
    s_off = (uint32_t)((lane / 32) * nq8 * 16 + 4 * (lane % 32));
    wq = W + L.quants(g0, 0);
    ws = W + L.scales(g0, 0);
    wq_step = 8 * 256;
    ws_step = 8 * 16;
  } else if constexpr (TYPE == kQ6_K) {
    const int nsb = nq8 / 8;
    const PackedQ6_K L{rows, nsb};
    const int p = 1024 * wp + 16 * lane;
    w_off = (uint32_t)((p / 1536) * nsb * 1536 + p % 1536);
    s_off = (uint32_t)((lane / 32) * nsb * 128 + 4 * (lane % 32));
    {
      const int q = 4 * min(lane, 7);
      d_off = (uint32_t)((q / 16) * nsb * 16 + q % 16);
    }
    wq = W + L.quants(g0, 0, 0);
    ws = W + L.scales(g0, 0);
    wd = W + L.dscale(g0, 0);
    wq_step = 1536;
    ws_step = 128;
  } else {
    const int nsb = nq8 / 8;
    const PackedQ4_K L{rows, nsb};
    w_off = (uint32_t)(wp * nsb * 1024 + 16 * lane);
    s_off = (uint32_t)((lane / 32) * nsb * 128 + 4 * (lane % 32));
    wq = W + L.quants(g0, 0, 0);
    ws = W + L.headers(g0, 0);
    wq_step = 1024;
    ws_step = 128;
  }

  // Slot j of this wave copies piece min(KW j + w, pieces - 1) of every stage (source sl_src + stage sl_step, LDS
  // offset sl_dst in the stage buffer, 16 or 4 bytes a lane). W pieces are the first WP <= KW, so only slot 0 of waves
  // below WP holds one, the wave's own piece wp.
  const uint8_t* sl_src[S::loads];
  int64_t sl_step[S::loads];
  uint32_t sl_dst[S::loads];
  bool sl_x4[S::loads];
  {
#pragma unroll
    for (int j = 0; j < S::loads; ++j) {
      const int p = min(KW * j + wu, S::n_x4 + S::n_dw - 1);
      sl_x4[j] = p < S::n_x4;
      if (p < WP) {
        sl_src[j] = wq + w_off, sl_step[j] = wq_step, sl_dst[j] = 1024 * p;
      } else if (p < S::n_x4) {
        const int k = p - WP;
        sl_src[j] = xb + x_src(1024 * k + 16 * lane), sl_step[j] = kUnits * 40, sl_dst[j] = S::x + 1024 * k;
      } else if (p == S::n_x4) {
        sl_src[j] = ws + s_off, sl_step[j] = ws_step, sl_dst[j] = S::s_off;
      } else if (TYPE == kQ6_K && p == S::n_x4 + 1) {
        sl_src[j] = wd + d_off, sl_step[j] = 16, sl_dst[j] = S::d_off;
      } else {
        constexpr int per = S::dx_bytes / 256;
        const int k = p - S::n_x4 - 1 - (TYPE == kQ6_K ? 1 : 0), which = k / per, kk = k % per;  // which 1: XS
        sl_src[j] = xb + dx_src(256 * kk + 4 * lane) + 4 * which, sl_step[j] = kUnits * 40;
        sl_dst[j] = (which ? S::xs : S::dx) + 256 * kk;
      }
    }
  }

  auto issue = [&]<int BUF>(int sn) __attribute__((always_inline)) {
    uint8_t* st = smem + BUF * S::bytes;
#pragma unroll
    for (int j = 0; j < S::loads; ++j) {
      if (sl_x4[j])
        ld16(sl_src[j] + sn * sl_step[j], st + sl_dst[j]);
      else
        ld4(sl_src[j] + sn * sl_step[j], st + sl_dst[j]);
    }
  };

  // MFMA lane roles: row r = lane % 16 (group gi = r / 8, row rr = r % 8), weight quarter c = lane / 16, result
  // elements i: tokens 4 c + i (+ 16 m). Chain role: row cr = tid % 16, tokens ct + CT m (those below 16 NTT).
  const int r = lane & 15, c = lane >> 4, gi = r >> 3, rr = r & 7;
  // CW > 0: waves KW .. KW + CW - 1 run only the chains (of the previous stage, while waves 0 .. KW - 1 copy and
  // form the terms of this one); CW = 0: every wave does both, one after the other.
  const bool doter = CW == 0 || wu < KW, chainer = CW == 0 || wu >= KW;
  const int ctid = CW ? tid - 64 * KW : tid;
  const int cr = ctid & 15, ct = ctid >> 4;
  // Result element i of the second token tile holds token 16 + 4 c + i: elements i >= lim1 are padding in every lane
  // (wave-uniform, skipped), and in this lane quarter elements i >= live1; padding terms are neither stored nor read
  // (17 tokens, the tree verification batch: only element 0 of lane quarter 0).
  const int lim1 = min(4, ntok - 16), live1 = ntok - 16 - 4 * c;
  float acc[CPT];
#pragma unroll
  for (int m = 0; m < CPT; ++m) acc[m] = 0.0f;
  const v4i zero4 = {0, 0, 0, 0};
  // Q4_K per stage (double-buffered like the terms): -(dmin m) per (row, unit) and dx (s0 + s1) per (token, unit)
  __shared__ __align__(16) float nmn_tab[TYPE == kQ4_K ? 2 * 16 * kUnits : 4];
  __shared__ __align__(16) float xs_tab[TYPE == kQ4_K ? 2 * 16 * NTT * kUnits : 4];
  __shared__ __align__(16) float pair_sink[TYPE == kQ4_K ? 64 : 4];  // Q4_K stores of lanes without a slot
  float* terms = terms_base;
  float* nmn_t = nmn_tab;
  float* xs_t = xs_tab;
  auto select = [&](int sn) __attribute__((always_inline)) {  // stage sn's buffers
    const int b = S::db ? (sn & 1) : 0;
    terms = terms_base + b * (S::terms1 / 4);
    if constexpr (TYPE == kQ4_K) {
      nmn_t = nmn_tab + b * 16 * kUnits;
      xs_t = xs_tab + b * 16 * NTT * kUnits;
    }
  };
  auto put = [&](int u, int tok, const float (&e)[E]) __attribute__((always_inline)) {
    float* p = terms + ((u * TS + tok) * 16 + r) * E;
    if constexpr (E == 2)
      *reinterpret_cast<float2*>(p) = make_float2(e[0], e[1]);
    else
      *reinterpret_cast<float4*>(p) = make_float4(e[0], e[1], e[2], e[3]);
  };

  // Every lane runs its chains over stage sn's units in order.
  auto chain = [&](int sn) __attribute__((always_inline)) {
    select(sn);
    float nm[kUnits];
    if constexpr (TYPE == kQ4_K) {
#pragma unroll
      for (int h = 0; h < kUnits / 4; ++h) {
        const float4 v = *reinterpret_cast<const float4*>(nmn_t + cr * kUnits + 4 * h);
        nm[4 * h] = v.x, nm[4 * h + 1] = v.y, nm[4 * h + 2] = v.z, nm[4 * h + 3] = v.w;
      }
    }
#pragma unroll
    for (int m = 0; m < CPT; ++m) {
      const int tk = ct + CT * m;
      if (CT * CPT > TS && tk >= TS) break;               // wave-uniform: threads past the token slots
      if (tk >= ntok) break;                              // padding token: its output is never stored
      float xsv[kUnits];
      if constexpr (TYPE == kQ4_K) {
#pragma unroll
        for (int h = 0; h < kUnits / 4; ++h) {
          const float4 v = *reinterpret_cast<const float4*>(xs_t + tk * kUnits + 4 * h);
          xsv[4 * h] = v.x, xsv[4 * h + 1] = v.y, xsv[4 * h + 2] = v.z, xsv[4 * h + 3] = v.w;
        }
      }
#pragma unroll
      for (int u = 0; u < kUnits; ++u) {
        const float* p = terms + ((u * TS + tk) * 16 + cr) * E;
        if constexpr (E == 2) {
          const float2 e = *reinterpret_cast<const float2*>(p);
          acc[m] = fma_(e.x, e.y, acc[m]);
          if constexpr (TYPE == kQ4_K) acc[m] = fma_(nm[u], xsv[u], acc[m]);
        } else {
          const float4 e = *reinterpret_cast<const float4*>(p);
          acc[m] = fma_(e.x, e.y, acc[m]);
          acc[m] = fma_(e.z, e.w, acc[m]);
        }
      }
    }
  };

  auto stage = [&]<int BUF>(int s) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    wait_vm_stages<S::loads, NS - 2>(min(NS - 2, nst - 1 - s));
    // stage s landed everywhere; double-buffered terms: stage s - 1's are written and the chains of stage s - 2
    // (which read the buffer stage s writes) are done; single: the chains of stage s - 1 are done
    ring_barrier();
    if (doter && s + NS - 1 < nst) issue.template operator()<(BUF + NS - 1) % NS>(s + NS - 1);
    const uint8_t* st = smem + BUF * S::bytes;
    if (doter) {
      select(s);
      if constexpr (PAIR) {
        // Lane (r, c): MFMA operand rows r (token r % 8 of unit u, or of u + 1), result unit u + ph, tokens 4 pt + i.
        const int ph = c >> 1, pt = c & 1;
        const bool lo = r < 8;
        auto xa = [&](int u) __attribute__((always_inline)) {  // operand bytes of token r % 8 of unit u
          return *reinterpret_cast<const long*>(st + S::x + (u * TS + (r & 7)) * 32 + 8 * c);
        };
        auto dxs = [&](int u0) __attribute__((always_inline)) {  // dx of this lane's result tokens
          return *reinterpret_cast<const float4*>(st + S::dx + ((u0 + ph) * TS + 4 * pt) * 4);
        };
        if constexpr (TYPE == kQ8_0) {
#pragma unroll
          for (int k = 0; k < UPW; k += 2) {
            const int u0 = UPW * wu + k;
            long bw[2];
            float dw[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              bw[e] = *reinterpret_cast<const long*>(st + gi * 2048 + (u0 + e) * 256 + (c >> 1) * 128 + rr * 16 + 8 * (c & 1));
              dw[e] = half_to_float(*reinterpret_cast<const uint16_t*>(st + S::s_off + gi * 128 + (u0 + e) * 16 + rr * 2));
            }
            const long x0 = xa(u0), x1 = xa(u0 + 1), a0 = lo ? x0 : 0, a1 = lo ? 0 : x1;  // both read, then selected
            const float4 dx4 = dxs(u0);
            const float dx[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bw[1], __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bw[0], zero4, 0, 0, 0), 0, 0, 0);
            const float dwl = ph ? dw[1] : dw[0];
#pragma unroll
            for (int i = 0; i < 4; ++i) put(u0 + ph, 4 * pt + i, {(float)d[i], dwl * dx[i]});
          }
        } else if constexpr (TYPE == kQ6_K) {
          const float dd = half_to_float(*reinterpret_cast<const uint16_t*>(st + S::d_off + gi * 16 + rr * 2));
          const int hw = c >> 1, h = c & 1;
#pragma unroll
          for (int k = 0; k < UPW; k += 2) {
            const int u0 = UPW * wu + k;
            long bl[2], bh[2];
            float s0[2], s1[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const uint8_t* au = st + gi * 1536 + (u0 + e) * 192;
              const uint2 nib = *reinterpret_cast<const uint2*>(au + rr * 16 + 8 * h);
              const uint2 hb = *reinterpret_cast<const uint2*>(au + 128 + rr * 8);
              const uint32_t hv = (hw ? hb.y : hb.x) >> (4 * h);
              const uint32_t q0 = ((nib.x >> (4 * hw)) & 0x0F0F0F0Fu) | ((hv & 0x03030303u) << 4);
              const uint32_t q1 = ((nib.y >> (4 * hw)) & 0x0F0F0F0Fu) | (((hv >> 2) & 0x03030303u) << 4);
              const long bq = (long)(((uint64_t)minus32(q1) << 32) | minus32(q0));
              bl[e] = hw ? 0 : bq;
              bh[e] = hw ? bq : 0;
              const uint32_t scw = *reinterpret_cast<const uint16_t*>(st + S::s_off + gi * 128 + rr * 16 + 2 * (u0 + e));
              s0[e] = dd * (float)(int8_t)(scw & 0xFF);
              s1[e] = dd * (float)(int8_t)(scw >> 8);
            }
            const long a0 = lo ? xa(u0) : 0, a1 = lo ? 0 : xa(u0 + 1);
            const float4 dx4 = dxs(u0);
            const float dx[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bl[1], __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bl[0], zero4, 0, 0, 0), 0, 0, 0);
            const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bh[1], __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bh[0], zero4, 0, 0, 0), 0, 0, 0);
            const float dsc0 = ph ? s0[1] : s0[0], dsc1 = ph ? s1[1] : s1[0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if constexpr (WIDE)
                put(u0 + ph, 4 * pt + i, {fma_((float)d1[i], dsc1, (float)d0[i] * dsc0), dx[i]});
              else
                put(u0 + ph, 4 * pt + i, {(float)d0[i], dsc0 * dx[i], (float)d1[i], dsc1 * dx[i]});
            }
          }
        } else {  // Q4_K: the wave's pairs are whole 64-weight chunks (even unit: low nibbles, odd: high)
          // Every LDS read of the stage first and the arithmetic without branches (only the stores predicated): a
          // branch ends the scheduler's region, and each read behind one waits out its own round trip.
          static_assert(UPW * TS <= 64, "one (unit, token) of the wave per lane");
          constexpr int NP = UPW / 2;  // the wave's pairs
          const int xi = min(lane, UPW * TS - 1), xu = UPW * wu + xi / TS, xt = xi % TS;
          const uint32_t sx = *reinterpret_cast<const uint32_t*>(st + S::xs + (xu * TS + xt) * 4);
          const float dxv = *reinterpret_cast<const float*>(st + S::dx + (xu * TS + xt) * 4);
          const uint4 hd = *reinterpret_cast<const uint4*>(st + S::s_off + gi * 128 + rr * 16);
          uint2 raw[NP];
          long xa0[NP], xa1[NP];
          float4 dx4[NP];
#pragma unroll
          for (int k = 0; k < NP; ++k) {
            const int u0 = UPW * wu + 2 * k;
            raw[k] = *reinterpret_cast<const uint2*>(st + gi * 1024 + (u0 / 2) * 256 + (c >> 1) * 128 + rr * 16 +
                                                     8 * (c & 1));
            xa0[k] = xa(u0), xa1[k] = xa(u0 + 1);
            dx4[k] = dxs(u0);
          }
          // dx (s0 + s1) of the wave's units' tokens, once per (unit, token); the other lanes store to a sink
          const float xsv = dxv * (float)((int)(int16_t)(sx & 0xFFFF) + (int)(int16_t)(sx >> 16));
          *(lane < UPW * TS ? xs_t + xt * kUnits + xu : pair_sink + lane) = xsv;
          const float d = half_to_float((uint16_t)(hd.x & 0xFFFF)), dmin = half_to_float((uint16_t)(hd.x >> 16));
#pragma unroll
          for (int k = 0; k < NP; ++k) {
            const int u0 = UPW * wu + 2 * k;
            long bq[2];
            float fsc[2], nmv[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              bq[e] = (long)(((uint64_t)((raw[k].y >> (4 * e)) & 0x0F0F0F0Fu) << 32) |
                             ((raw[k].x >> (4 * e)) & 0x0F0F0F0Fu));
              int sc, mn;
              scale_min_sel(u0 + e, hd.y, hd.z, hd.w, sc, mn);
              fsc[e] = d * (float)sc;
              nmv[e] = -(dmin * (float)mn);
            }
            *reinterpret_cast<float2*>(c == 0 ? nmn_t + r * kUnits + u0 : pair_sink + 2 * (lane & 31)) =
                make_float2(nmv[0], nmv[1]);
            const long a0 = lo ? xa0[k] : 0, a1 = lo ? 0 : xa1[k];
            const float dx[4] = {dx4[k].x, dx4[k].y, dx4[k].z, dx4[k].w};
            const v4i dq = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bq[1], __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bq[0], zero4, 0, 0, 0), 0, 0, 0);
            const float fs = ph ? fsc[1] : fsc[0];
#pragma unroll
            for (int i = 0; i < 4; ++i) put(u0 + ph, 4 * pt + i, {(float)dq[i], fs * dx[i]});
          }
        }
      } else if constexpr (TYPE == kQ8_0) {
        // Every LDS read of the stage first: the term stores could alias them as far as the compiler can tell and
        // would hold each read behind the stores before it.
        long bw[UPW], av[UPW][NTT];
        float dw[UPW];
        float4 dv[UPW][NTT];
#pragma unroll
        for (int k = 0; k < UPW; ++k) {
          const int u = UPW * wu + k;
          bw[k] = *reinterpret_cast<const long*>(st + gi * 2048 + u * 256 + (c >> 1) * 128 + rr * 16 + 8 * (c & 1));
          dw[k] = half_to_float(*reinterpret_cast<const uint16_t*>(st + S::s_off + gi * 128 + u * 16 + rr * 2));
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            av[k][m] = *reinterpret_cast<const long*>(st + S::x + (u * TS + 16 * m + r) * 32 + 8 * c);
            dv[k][m] = *reinterpret_cast<const float4*>(st + S::dx + (u * TS + 16 * m + 4 * c) * 4);
          }
        }
#pragma unroll
        for (int k = 0; k < UPW; ++k) {
          const int u = UPW * wu + k;
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            const float dx[4] = {dv[k][m].x, dv[k][m].y, dv[k][m].z, dv[k][m].w};
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[k][m], bw[k], zero4, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (m == 0 || i < lim1) {
                const float e0 = (float)d[i], e1 = dw[k] * dx[i];
                if (m == 0 || i < live1) put(u, 16 * m + 4 * c + i, {e0, e1});
              }
          }
        }
      } else if constexpr (TYPE == kQ6_K) {
        // Every LDS read of the stage first (as for Q8_0).
        const float dd = half_to_float(*reinterpret_cast<const uint16_t*>(st + S::d_off + gi * 16 + rr * 2));
        const int hw = c >> 1, h = c & 1;
        uint2 nib[UPW], hb[UPW];
        uint32_t scw[UPW];
        long av[UPW][NTT];
        float4 dv[UPW][NTT];
#pragma unroll
        for (int k = 0; k < UPW; ++k) {
          const int u = UPW * wu + k;
          const uint8_t* au = st + gi * 1536 + u * 192;
          nib[k] = *reinterpret_cast<const uint2*>(au + rr * 16 + 8 * h);
          hb[k] = *reinterpret_cast<const uint2*>(au + 128 + rr * 8);
          scw[k] = *reinterpret_cast<const uint16_t*>(st + S::s_off + gi * 128 + rr * 16 + 2 * u);
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            av[k][m] = *reinterpret_cast<const long*>(st + S::x + (u * TS + 16 * m + r) * 32 + 8 * c);
            dv[k][m] = *reinterpret_cast<const float4*>(st + S::dx + (u * TS + 16 * m + 4 * c) * 4);
          }
        }
#pragma unroll
        for (int k = 0; k < UPW; ++k) {
          const int u = UPW * wu + k;
          const uint32_t hv = (hw ? hb[k].y : hb[k].x) >> (4 * h);
          const uint32_t q0 = ((nib[k].x >> (4 * hw)) & 0x0F0F0F0Fu) | ((hv & 0x03030303u) << 4);
          const uint32_t q1 = ((nib[k].y >> (4 * hw)) & 0x0F0F0F0Fu) | (((hv >> 2) & 0x03030303u) << 4);
          const long bq = (long)(((uint64_t)minus32(q1) << 32) | minus32(q0));
          const long b0 = hw ? 0 : bq, b1 = hw ? bq : 0;
          const float dsc0 = dd * (float)(int8_t)(scw[k] & 0xFF), dsc1 = dd * (float)(int8_t)(scw[k] >> 8);
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            const float dx[4] = {dv[k][m].x, dv[k][m].y, dv[k][m].z, dv[k][m].w};
            const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[k][m], b0, zero4, 0, 0, 0);
            const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[k][m], b1, zero4, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (m > 0 && i >= lim1) continue;
              if constexpr (WIDE) {
                const float e0 = fma_((float)d1[i], dsc1, (float)d0[i] * dsc0);
                if (m == 0 || i < live1) put(u, 16 * m + 4 * c + i, {e0, dx[i]});
              } else {
                const float e0 = (float)d0[i], e1 = dsc0 * dx[i], e2 = (float)d1[i], e3 = dsc1 * dx[i];
                if (m == 0 || i < live1) put(u, 16 * m + 4 * c + i, {e0, e1, e2, e3});
              }
            }
          }
        }
      } else {  // Q4_K: the wave's units UPW w .. (64-weight chunk u / 2: even units low nibbles, odd high)
        // Every LDS read of the stage first and the arithmetic without branches, as for the pairs.
        static_assert(UPW * TS <= 64, "one (unit, token) of the wave per lane");
        const int xi = min(lane, UPW * TS - 1), xu = UPW * wu + xi / TS, xt = xi % TS;
        const uint32_t sx = *reinterpret_cast<const uint32_t*>(st + S::xs + (xu * TS + xt) * 4);
        const float dxv = *reinterpret_cast<const float*>(st + S::dx + (xu * TS + xt) * 4);
        const uint4 hd = *reinterpret_cast<const uint4*>(st + S::s_off + gi * 128 + rr * 16);
        const int j2 = UPW * wu / 2;  // the wave's 64-weight chunk
        const uint2 raw =
            *reinterpret_cast<const uint2*>(st + gi * 1024 + j2 * 256 + (c >> 1) * 128 + rr * 16 + 8 * (c & 1));
        long av[UPW][NTT];
        float4 dv[UPW][NTT];
#pragma unroll
        for (int k = 0; k < UPW; ++k) {
          const int u = UPW * wu + k;
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            av[k][m] = *reinterpret_cast<const long*>(st + S::x + (u * TS + 16 * m + r) * 32 + 8 * c);
            dv[k][m] = *reinterpret_cast<const float4*>(st + S::dx + (u * TS + 16 * m + 4 * c) * 4);
          }
        }
        // dx (s0 + s1) of the wave's units' tokens, once per (unit, token); the other lanes store to a sink
        const float xsv = dxv * (float)((int)(int16_t)(sx & 0xFFFF) + (int)(int16_t)(sx >> 16));
        *(lane < UPW * TS ? xs_t + xt * kUnits + xu : pair_sink + lane) = xsv;
        const float d = half_to_float((uint16_t)(hd.x & 0xFFFF)), dmin = half_to_float((uint16_t)(hd.x >> 16));
#pragma unroll
        for (int k = 0; k < UPW; ++k) {
          const int u = UPW * wu + k, e = u & 1;
          const long bq = (long)(((uint64_t)((raw.y >> (4 * e)) & 0x0F0F0F0Fu) << 32) | ((raw.x >> (4 * e)) & 0x0F0F0F0Fu));
          int sc, mn;
          scale_min_sel(u, hd.y, hd.z, hd.w, sc, mn);
          const float fsc = d * (float)sc;
          *(c == 0 ? nmn_t + r * kUnits + u : pair_sink + lane) = -(dmin * (float)mn);
#pragma unroll
          for (int m = 0; m < NTT; ++m) {
            const float dx[4] = {dv[k][m].x, dv[k][m].y, dv[k][m].z, dv[k][m].w};
            const v4i dq = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[k][m], bq, zero4, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (m == 0 || i < lim1) {
                const float e0 = (float)dq[i], e1 = fsc * dx[i];
                if (m == 0 || i < live1) put(u, 16 * m + 4 * c + i, {e0, e1});
              }
          }
        }
      }
    }
    if constexpr (S::db) {
      // The previous stage's terms were written before this stage's barrier: its chains run now, alongside this
      // stage's term work (the last stage's chains run after the loop).
      if (chainer && s > 0) chain(s - 1);
    } else {
      // Terms written (LDS only): then every lane runs its chains over the stage's units in order.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
      chain(s);
    }
  };

  [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
    ((B < nst ? issue.template operator()<B>(B) : void()), ...);
  }(std::make_integer_sequence<int, NS - 1>{});
  for (int s = 0; s < nst; s += NS) {
    [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
      ((s + B < nst ? stage.template operator()<B>(s + B) : void()), ...);
    }(std::make_integer_sequence<int, NS>{});
  }
  if constexpr (S::db) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();  // the last stage's terms are written
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (chainer) chain(nst - 1);
  }
  if (!chainer) return;

  const int64_t row = (int64_t)rt * 16 + cr;
#pragma unroll
  for (int m = 0; m < CPT; ++m) {
    const int t = ct + CT * m;
    if (t < ntok) {
      float* o = y + (int64_t)(t0 + t) * ys + row;
      *o = accumulate ? *o + acc[m] : acc[m];
    }
  }
}

template <int TYPE, bool WIDE, int NTT, int NS, int KW, bool PAIR, int TS, int CW>
void launch_ks_ns(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
                  int64_t ys, bool accumulate) {
  using S = KsLds<TYPE, WIDE, NTT, KW, TS, CW>;
  const size_t lds = NS * (size_t)S::bytes + S::terms;
  static bool attr = false;
  if (!attr) {
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(k_mmv_ks<TYPE, WIDE, NTT, NS, KW, PAIR, TS, CW>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
          "hipFuncSetAttribute");
    attr = true;
  }
  const int tiles = (n + 16 * NTT - 1) / (16 * NTT);
  require(n <= TS || TS == 16 * NTT, "mmv_ks: more tokens than token slots");
  hipLaunchKernelGGL((k_mmv_ks<TYPE, WIDE, NTT, NS, KW, PAIR, TS, CW>), dim3((unsigned)(rows / 16), (unsigned)tiles),
                     dim3(64 * (KW + CW)), lds, s, static_cast<const uint8_t*>(w), rows, cols, x, n, y, ys, accumulate ? 1 : 0);
}

// Term waves per 16-row tile of the K-split kernel, measured on MI355X: eight (one unit per wave and stage) for two
// token tiles (17-32 tokens: Qwen3-14B Q6_K at 17 tokens, 5120 x 17408 95.4 -> 86.3 us, 5120 x 5120 30.1 -> 27.4 us),
// for Q6_K and for Q8_0 (4096 x 12288 at 8 tokens 26.4 -> 24.5 us); four for Q4_K's single token tile (5120 x 17408
// at 8 tokens: 63.6 vs 74.4 us with eight) and for the pairs.
template <int TYPE, int NTT, bool PAIR>
constexpr int ks_waves() { return PAIR ? 4 : NTT == 2 || TYPE != kQ4_K ? 8 : 4; }

// Ring depth: the deepest ring that fits one workgroup per CU when the grid fits the GPU once, else one that lets
// two workgroups share a CU (80 KB each).
// Chain waves (one chain per thread, 16 rows x TS tokens) for the single token tile of Q8_0 and Q4_K and for the
// pairs; measured on MI355X (8 tokens, Q4_K 5120 x 17408: 46.4 -> 38.6 us, Q6_K 46.5 -> 43.4, Q8_0 4096 x 12288 19.6
// -> 18.6; 12 tokens, Q4_K 57.6 -> 53.5). Without them (the chains on the term waves after their terms) for the two
// token tiles (17 tokens, Q6_K: within 3 % either way) and for Q6_K's single tile (12 tokens: 71.9 vs 94.0 us).
template <int TYPE, int NTT, bool PAIR, int TS>
constexpr int ks_chain_waves() { return PAIR || (NTT == 1 && TYPE != kQ6_K) ? TS / 4 : 0; }

template <int TYPE, bool WIDE, int NTT, bool PAIR, int TS, int CW = ks_chain_waves<TYPE, NTT, PAIR, TS>()>
void launch_ks_ntt(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
                   int64_t ys, bool accumulate) {
  constexpr int KW = ks_waves<TYPE, NTT, PAIR>();
  using S = KsLds<TYPE, WIDE, NTT, KW, TS, CW>;
  const int64_t wgs = rows / 16 * ((n + 16 * NTT - 1) / (16 * NTT)), cus = device_cus();
  constexpr int kDeep = (150 * 1024 - S::terms) / S::bytes >= 8 ? 8 : (150 * 1024 - S::terms) / S::bytes;
  constexpr int kTwo = (80 * 1024 - S::terms) / S::bytes;
  static_assert(kDeep >= 3, "the K-split ring needs three stages");
  if constexpr (kTwo >= 3) {
    if (wgs > cus) {
      launch_ks_ns<TYPE, WIDE, NTT, (kTwo > 6 ? 6 : kTwo), KW, PAIR, TS, CW>(s, w, rows, cols, x, n, y, ys, accumulate);
      return;
    }
  }
  launch_ks_ns<TYPE, WIDE, NTT, kDeep, KW, PAIR, TS, CW>(s, w, rows, cols, x, n, y, ys, accumulate);
}

template <int TYPE, bool WIDE>
void launch_ks(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
               int64_t ys, bool accumulate) {
  if (n <= 8)
    launch_ks_ntt<TYPE, WIDE, 1, true, 8>(s, w, rows, cols, x, n, y, ys, accumulate);
  else if (n <= 16)
    launch_ks_ntt<TYPE, WIDE, 1, false, 16>(s, w, rows, cols, x, n, y, ys, accumulate);
  else if (n <= 20)
    launch_ks_ntt<TYPE, WIDE, 2, false, 20>(s, w, rows, cols, x, n, y, ys, accumulate);
  else
    launch_ks_ntt<TYPE, WIDE, 2, false, 32>(s, w, rows, cols, x, n, y, ys, accumulate);
}

template <int TYPE, bool WIDE, int NTT, int NS>
void launch_ns(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
               int64_t ys, bool accumulate) {
  const size_t lds = NS * (size_t)MmvLds<TYPE, NTT>::bytes;
  static bool attr = false;  // per instantiation: rings past 64 KB of dynamic LDS
  if (!attr) {
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(k_mmv<TYPE, WIDE, NTT, NS>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
          "hipFuncSetAttribute");
    attr = true;
  }
  const int tiles = (n + 16 * NTT - 1) / (16 * NTT);
  hipLaunchKernelGGL((k_mmv<TYPE, WIDE, NTT, NS>), dim3((unsigned)(rows / kRowsT), (unsigned)tiles), dim3(kThreads),
                     lds, s, static_cast<const uint8_t*>(w), rows, cols, x, n, y, ys, accumulate ? 1 : 0);
}

// Ring depth by grid size: with at most one workgroup per CU the deepest ring the vmcnt counter allows; with more,
// rings small enough for 2..4 resident workgroups per CU.
template <int TYPE, bool WIDE, int NTT>
void launch_ntt(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
                int64_t ys, bool accumulate) {
  const int64_t wgs = rows / kRowsT * ((n + 16 * NTT - 1) / (16 * NTT)), cus = device_cus();
  constexpr int kDeep = NTT == 1 ? 8 : 6;
  if (wgs <= cus)
    launch_ns<TYPE, WIDE, NTT, kDeep>(s, w, rows, cols, x, n, y, ys, accumulate);
  else if (wgs <= 2 * cus)
    launch_ns<TYPE, WIDE, NTT, 5>(s, w, rows, cols, x, n, y, ys, accumulate);
  else
    launch_ns<TYPE, WIDE, NTT, 3>(s, w, rows, cols, x, n, y, ys, accumulate);
}

template <int TYPE, bool WIDE>
void launch_mmv(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
                int64_t ys, bool accumulate) {
  if (n <= 16)
    launch_ntt<TYPE, WIDE, 1>(s, w, rows, cols, x, n, y, ys, accumulate);
  else
    launch_ntt<TYPE, WIDE, 2>(s, w, rows, cols, x, n, y, ys, accumulate);
}

}  // namespace

bool mmv_supported(int type, int64_t rows, int64_t cols, int n) {
  return (type == kQ8_0 || type == kQ4_K || type == kQ6_K) && n >= 1 && n <= 32 && rows % kRowsT == 0 &&
         cols % (32 * kUnits) == 0;
}

void mmv(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n,
         float* y, int64_t ys, bool accumulate, bool ksplit) {
  require(mmv_supported(type, rows, cols, n), "mmv: Q8_0/Q4_K/Q6_K, 1..32 tokens, rows % 32 == 0, cols % 256 == 0");
  if (ksplit) {
    switch (type) {
      case kQ8_0:
        launch_ks<kQ8_0, false>(s, w, rows, cols, x, n, y, ys, accumulate);
        break;
      case kQ4_K:
        launch_ks<kQ4_K, false>(s, w, rows, cols, x, n, y, ys, accumulate);
        break;
      default:
        if (wide && n > 16)
          launch_ks<kQ6_K, true>(s, w, rows, cols, x, n, y, ys, accumulate);
        else
          launch_ks<kQ6_K, false>(s, w, rows, cols, x, n, y, ys, accumulate);
        break;
    }
    check_launch("mmv");
    return;
  }
  switch (type) {
    case kQ8_0:
      launch_mmv<kQ8_0, false>(s, w, rows, cols, x, n, y, ys, accumulate);
      break;
    case kQ4_K:
      launch_mmv<kQ4_K, false>(s, w, rows, cols, x, n, y, ys, accumulate);
      break;
    default:  // Q6_K: the reference's wide panels above 16 tokens (quant.cpp:256)
      if (wide && n > 16)
        launch_mmv<kQ6_K, true>(s, w, rows, cols, x, n, y, ys, accumulate);
      else
        launch_mmv<kQ6_K, false>(s, w, rows, cols, x, n, y, ys, accumulate);
      break;
  }
  check_launch("mmv");
}

}  // namespace mk
