// Prefill / batch GEMM for K-quant weights (Q4_K, Q6_K) on int8 MFMA, bit-identical to the reference's panel kernels:
//   Q4_K (gemm_avx512.cpp:104-155, the wide panels use the same arithmetic), per 32-weight sub-block j in order:
//     acc = fma(float(sum q4 x), (d sc_j) dx, acc);  acc = fma(-(dmin m_j), dx (s0 + s1), acc)
//   Q6_K compact (gemm_avx512.cpp:157-205), per 16-value half h in order:
//     acc = fma(float(sum (q6 - 32) x), (d sc_h) dx, acc)
//   Q6_K wide (gemm_avx512.cpp:268-316; n > 16 unless MALKIN_NO_WIDE), per 32-weight block b in order:
//     s = fma(float(ai1), d sc_2b+1, float(ai0) (d sc_2b));  acc = fma(s, dx, acc)
// Every integer dot is exact (MFMA int32); every fp32 operation is the reference's, in its order.
//
// Roles are swapped against the Q8_0 kernel: the MFMA's A operand is the activations (tokens) and B the weights, so an
// accumulator element of lane l is (token 8 (i / 4) + 4 (l / 32) + i % 4, weight row l % 32) and every per-row scale
// (d sc, dmin m) is one register per lane; per-token values (dx, dx (s0 + s1)) come from LDS as 16 registers. The
// rank-1 products (d sc_h) dx and (d sc_j) dx run on the matrix cores (v_mfma_f32_32x32x1_2b_f32, one block per half
// or per sub-block), int -> float conversions as in the Q8_0 kernel (0x4B400000 accumulator start, then an fp32
// outer product adding -12582912; |dot| <= 32 * 128 * 128 < 2^22). The weights are unpacked from the CDNA planes of
// layout.h into int8 in registers: Q4_K nibbles 0..15; Q6_K q - 32 per byte as ((q | 0x80) - 0x20) ^ 0x80, which
// never borrows across bytes for q < 64.
//
// A workgroup (4 waves) owns a 128-row x 32-token tile (or a 32-row tail tile), 32 rows per wave, and walks K in
// stages of half a super-block (4 units of 32 weights) held in a ring of NS LDS buffers filled by direct global -> LDS
// loads NS - 1 stages ahead.
#include <utility>

#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

constexpr int kThreads = 256;
constexpr int kRowsT = 128, kTokT = 32;  // workgroup tile
constexpr int kKB = 4;                   // 32-weight units per stage (half a super-block)
constexpr int kMagic = 0x4B400000;       // bits of 12582912.0f
constexpr float kMagicF = 12582912.0f;

template <int TYPE>
struct KqLds;
template <>
struct KqLds<kQ6_K> {
  static constexpr int a = 0;                    // [4 units][16 groups][192 B]: nib plane 8 x 16 B, hbit plane 8 x 8 B
  static constexpr int sc = a + 4 * 16 * 192;    // [16 groups][8 rows][16 int8] (the whole super-block)
  static constexpr int d = sc + 16 * 128;        // [16 groups][8 rows] f16
  static constexpr int x = d + 16 * 16;          // [4 units][32 tok][32 B] BlockQ8 qs
  static constexpr int dx = x + 4 * 32 * 32;     // [4 units][32 tok] f32
  static constexpr int bytes = dx + 4 * 32 * 4;  // 19200
  static constexpr int loads = 6;                // global -> LDS loads per wave per stage
  static constexpr int tail_loads = 4;           // ... in a 32-row tail tile
};
template <>
struct KqLds<kQ4_K> {
  static constexpr int a = 0;                       // [2 chunks][16 groups][256 B]: lo plane 8 x 16 B, hi plane 8 x 16 B
  static constexpr int hdr = a + 2 * 16 * 256;      // [16 groups][8 rows][16 B] GGUF header (d, dmin, scales)
  static constexpr int x = hdr + 16 * 128;          // [4 units][32 tok][32 B]
  static constexpr int dx = x + 4 * 32 * 32;        // [4 units][32 tok] f32
  static constexpr int s = dx + 4 * 32 * 4;         // [4 units][32 tok] int16 pair (s0, s1)
  static constexpr int dsx = s + 4 * 32 * 4;        // [4 waves][4 units][32 tok] f32: dx (s0 + s1), one copy per wave
  static constexpr int bytes = dsx + 4 * 4 * 32 * 4;  // 17408
  static constexpr int loads = 5;
};

__device__ __forceinline__ void load_lds16(const void* g, uint8_t* l) { lds_copy16(g, l); }
__device__ __forceinline__ void load_lds4(const void* g, uint8_t* l) { lds_copy4(g, l); }
// float(int8 byte K of v)
template <int K>
__device__ __forceinline__ float sbyte_f(uint32_t v) {
  return (float)(int8_t)((v >> (8 * K)) & 0xFF);
}

__device__ __forceinline__ v16f conv(v16i c) {
  return __builtin_amdgcn_mfma_f32_16x16x1f32(-kMagicF, 1.0f, __builtin_bit_cast(v16f, c), 0, 0, 0);
}

// q - 32 per byte for bytes q < 64.
__device__ __forceinline__ uint32_t minus32(uint32_t q) { return ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u; }

// scale_min_k4 (the reference's kernels.h:18-26) of the 12 packed scale bytes held in q0..q2.
__device__ __forceinline__ int kbyte(uint32_t q0, uint32_t q1, uint32_t q2, int i) {
  const uint32_t w = i < 4 ? q0 : (i < 8 ? q1 : q2);
  return (int)((w >> (8 * (i & 3))) & 0xFFu);
}
__device__ __forceinline__ void scale_min(int j, uint32_t q0, uint32_t q1, uint32_t q2, int& sc, int& m) {
  if (j < 4) {
    sc = kbyte(q0, q1, q2, j) & 63;
    m = kbyte(q0, q1, q2, j + 4) & 63;
  } else {
    const int hi = kbyte(q0, q1, q2, j + 4);
    sc = (hi & 0xF) | ((kbyte(q0, q1, q2, j - 4) >> 6) << 4);
    m = (hi >> 4) | ((kbyte(q0, q1, q2, j) >> 6) << 4);
  }
}

// NS: stages in the LDS ring, NS - 1 of them in flight. 3 when the grid takes several workgroups per CU (prefill);
// deeper rings when few row tiles cover the matrix (short batches), where the stream is latency-bound otherwise.
// NE: accumulator elements with a live token. Element i holds tokens 8 (i / 4) + i % 4 and 8 (i / 4) + 4 + i % 4 of
// the tile, so for a batch of at most 17 tokens (config 5's tree verification) elements 9..15 hold only padding
// tokens in every lane: NE = 9 skips their epilogue (their MFMA results are computed and dropped).
template <int TYPE, bool WIDE, int NS, int NE>
__global__ __launch_bounds__(kThreads) void k_gemm_kq(const uint8_t* W, int64_t rows, int64_t cols,
                                                      const BlockQ8* x, int n, float* __restrict__ y, int64_t ys,
                                                      int accumulate, int n_rt, int n_tt, int n_big) {
  using S = KqLds<TYPE>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // Workgroup -> (row tile, token tile): tiles numbered row-major, each XCD a contiguous run of them (token tiles of a
  // row tile on one XCD, rows read once into its L2).
  // With 32-row tail tiles (n_big < n_rt, one token tile): tiles in launch order, so the n_big = CU count full tiles
  // take one CU each and the tail tiles a second slot on CUs of every XCD.
  const int tile = n_big < n_rt ? (int)blockIdx.x : xcd_run((int)blockIdx.x, n_rt * n_tt);
  const int rt = tile / n_tt, tt = tile % n_tt;
  const int nb = (int)(cols / 32), nsb = (int)(cols / 256);
  const int64_t r0 = rt < n_big ? (int64_t)rt * kRowsT : (int64_t)n_big * kRowsT + (int64_t)(rt - n_big) * 32;
  const int64_t g0 = r0 / 8;
  const int ngroups = (int)min<int64_t>(rt < n_big ? kRowsT / 8 : 4, rows / 8 - g0);  // 4 .. 16 (rows % 32 == 0)
  const bool live = 32 * wu < 8 * ngroups;  // this wave's 32 rows hold a row of the matrix (else: copies only)
  const int t0 = tt * kTokT;
  const int nstages = nb / kKB;  // cols % 256 == 0: whole stages

  // Activation copies, per lane: X (wave w: unit w; lane -> token lane / 2, 16-byte half lane % 2); per-token words
  // (unit = 2 c + lane / 32, token lane % 32).
  const uint8_t* x_base = reinterpret_cast<const uint8_t*>(x + (int64_t)t0 * nb);
  const int tx = min(t0 + (lane >> 1), n - 1) - t0, tw = min(t0 + (lane & 31), n - 1) - t0;
  const uint32_t x_off = (uint32_t)(tx * nb * 40 + 8 + 16 * (lane & 1));
  const uint32_t tw_off = (uint32_t)(tw * nb * 40 + (lane >> 5) * 40);  // + 80 c for unit 2 c + lane / 32

  // Weight copies: every piece is 16 (or 4) bytes of a packed (group, unit) record, LDS destinations lane-linear.
  uint32_t a_off[3], m_off, t_off = 0;
  const uint8_t *a_base, *m_base, *d_base = nullptr;
  uint32_t d_off = 0;
  if constexpr (TYPE == kQ6_K) {
    const PackedQ6_K L{rows, nsb};
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const int p = 64 * (3 * w + c) + lane, u = p / 192, q = p % 192;
      const int gi = min(q / 12, ngroups - 1);
      a_off[c] = (uint32_t)((gi * nsb * 8 + u) * 192 + 16 * (q % 12));
    }
    a_base = W + L.quants(g0, 0, 0);
    {
      const int p = 64 * (w & 1) + lane, gi = min(p / 8, ngroups - 1);
      m_off = (uint32_t)(gi * nsb * 128 + 16 * (p % 8));
      m_base = W + L.scales(g0, 0);
    }
    d_off = (uint32_t)(min(lane / 4, ngroups - 1) * nsb * 16 + 4 * (lane % 4));
    d_base = W + L.dscale(g0, 0);
    // Tail tile (4 groups): wave w copies unit w of the stage, lanes 0..47 its 4 x 12 pieces; lanes 48..63 re-read
    // group 3 into the unused group 4-5 slots.
    t_off = (uint32_t)((min(lane / 12, ngroups - 1) * nsb * 8 + w) * 192 + 16 * (lane % 12));
  } else {
    const PackedQ4_K L{rows, nsb};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int p = 64 * (2 * w + c) + lane, cc = p / 256, q = p % 256;
      const int gi = min(q / 16, ngroups - 1);
      a_off[c] = (uint32_t)((gi * nsb * 4 + cc) * 256 + 16 * (q % 16));
    }
    a_off[2] = 0;
    a_base = W + L.quants(g0, 0, 0);
    {
      const int p = 64 * (w & 1) + lane, gi = min(p / 8, ngroups - 1);
      m_off = (uint32_t)(gi * nsb * 128 + 16 * (p % 8));
      m_base = W + L.headers(g0, 0);
    }
  }

  // Stage sn (units 4 sn .. 4 sn + 3: super-block sn / 2, half sn % 2) into buffer BUF. Every wave issues S::loads
  // loads (a wave with fewer repeats its activation copy), so one wait count fits all; Q6_K tail tiles (TAIL) copy
  // only the 4 groups' quants and scales, S::tail_loads per wave.
  auto issue = [&]<int BUF, bool TAIL>(int sn) __attribute__((always_inline)) {
    uint8_t* st = smem + BUF * S::bytes;
    const int sb = sn >> 1, hf = sn & 1;
    const uint8_t* xb = x_base + (size_t)(4 * sn) * 40;
    if constexpr (TYPE == kQ6_K && TAIL) {
      using T = KqLds<kQ6_K>;
      const uint8_t* ab = a_base + ((size_t)sb * 8 + 4 * hf) * 192;
      load_lds16(ab + t_off, st + T::a + 3072 * wu);
      if (wu == 0)
        load_lds16(m_base + (size_t)sb * 128 + m_off, st + T::sc);
      else if (wu == 1)
        load_lds16(xb + (size_t)wu * 40 + x_off, st + T::x + 1024 * wu);
      else if (wu == 2)
        load_lds4(d_base + (size_t)sb * 16 + d_off, st + T::d);
      else
        load_lds4(xb + tw_off, st + T::dx);
      if (wu == 3)
        load_lds4(xb + 80 + tw_off, st + T::dx + 256);
      else
        load_lds16(xb + (size_t)wu * 40 + x_off, st + T::x + 1024 * wu);
      load_lds16(xb + (size_t)wu * 40 + x_off, st + T::x + 1024 * wu);
    } else if constexpr (TYPE == kQ6_K) {
      const uint8_t* ab = a_base + ((size_t)sb * 8 + 4 * hf) * 192;
#pragma unroll
      for (int c = 0; c < 3; ++c) load_lds16(ab + a_off[c], st + S::a + 1024 * (3 * wu + c));
      if (wu < 2) {
        load_lds16(m_base + (size_t)sb * 128 + m_off, st + S::sc + 1024 * wu);
      } else if (wu == 2) {
        load_lds4(d_base + (size_t)sb * 16 + d_off, st + S::d);
      } else {
        load_lds4(xb + tw_off, st + S::dx);
        load_lds4(xb + 80 + tw_off, st + S::dx + 256);
      }
      load_lds16(xb + (size_t)wu * 40 + x_off, st + S::x + 1024 * wu);
      if (wu != 3) load_lds16(xb + (size_t)wu * 40 + x_off, st + S::x + 1024 * wu);
    } else {
      const uint8_t* ab = a_base + ((size_t)sb * 4 + 2 * hf) * 256;
#pragma unroll
      for (int c = 0; c < 2; ++c) load_lds16(ab + a_off[c], st + S::a + 1024 * (2 * wu + c));
      if (wu < 2) {
        load_lds16(m_base + (size_t)sb * 128 + m_off, st + S::hdr + 1024 * wu);
        load_lds16(xb + (size_t)wu * 40 + x_off, st + S::x + 1024 * wu);
      } else if (wu == 2) {
        load_lds4(xb + tw_off, st + S::dx);
        load_lds4(xb + 80 + tw_off, st + S::dx + 256);
      } else {
        load_lds4(xb + 4 + tw_off, st + S::s);
        load_lds4(xb + 84 + tw_off, st + S::s + 256);
      }
      load_lds16(xb + (size_t)wu * 40 + x_off, st + S::x + 1024 * wu);
    }
  };

  v16f acc = {};
  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; ++i) magic[i] = kMagic;
  asm volatile("" : "+v"(magic));  // keep it in VGPRs: as a uniform value it would be copied from SGPRs per MFMA
  const v32f zero = {};
  const int li = lane & 31, h = lane >> 5;
  const int gi = 4 * w + (li >> 3), r8 = li & 7;  // this lane's weight row: group gi, row r8 of it
  const int tok_i = 4 * h;                         // tokens of element i: 8 (i / 4) + 4 h + i % 4

  // 16 per-token floats of element i from a [32 tok] f32 array: tokens 8 q + 4 h .. + 3 for q = 0..3.
  auto tok16 = [&](const uint8_t* p) __attribute__((always_inline)) {
    v16f v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 f = *reinterpret_cast<const float4*>(p + 4 * (8 * q + tok_i));
      v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
    }
    return v;
  };

  auto stage = [&]<int BUF, bool TAIL>(int s) __attribute__((always_inline)) {
    // Stage s has landed once at most the loads of the stages issued after it (s + 1 .. s + NS - 2, fewer at the
    // end) are outstanding; the buffer stage s + NS - 1 goes into was read in stage s - 1, finished by every wave
    // before this barrier.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    if constexpr (TAIL)
      wait_vm_stages<KqLds<kQ6_K>::tail_loads, NS - 2>(min(NS - 2, nstages - 1 - s));
    else
      wait_vm_stages<S::loads, NS - 2>(min(NS - 2, nstages - 1 - s));
    ring_barrier();
    if (s + NS - 1 < nstages) issue.template operator()<(BUF + NS - 1) % NS, TAIL>(s + NS - 1);
    if (!live) return;
    uint8_t* st = smem + BUF * S::bytes;
    const int hf = s & 1;
    if constexpr (TYPE == kQ6_K) {
      // weight scales of this lane's row: d, and sc_h for the 8 halves of units 4 hf .. 4 hf + 3
      const float d = half_to_float(*reinterpret_cast<const uint16_t*>(st + S::d + gi * 16 + r8 * 2));
      const uint2 scw = *reinterpret_cast<const uint2*>(st + S::sc + gi * 128 + r8 * 16 + 8 * hf);
#pragma unroll
      for (int u = 0; u < kKB; ++u) {
        const uint32_t sw = u < 2 ? scw.x : scw.y;
        const float d0 = d * sbyte_f<0>(sw >> (16 * (u & 1))), d1 = d * sbyte_f<1>(sw >> (16 * (u & 1)));
        const uint8_t* au = st + S::a + u * 3072 + gi * 192;
        const uint2 nib = *reinterpret_cast<const uint2*>(au + r8 * 16 + 8 * h);
        const uint2 hb = *reinterpret_cast<const uint2*>(au + 128 + r8 * 8);
        const uint8_t* xu = st + S::x + u * 1024 + li * 32 + 8 * h;
        const long xa0 = *reinterpret_cast<const long*>(xu), xa1 = *reinterpret_cast<const long*>(xu + 16);
        // half hw: bytes r = 0..7 are q[16 hw + 8 h + r]
        long wq[2];
#pragma unroll
        for (int hw = 0; hw < 2; ++hw) {
          const uint32_t hv = (hw ? hb.y : hb.x) >> (4 * h);
          const uint32_t q0 = ((nib.x >> (4 * hw)) & 0x0F0F0F0Fu) | ((hv & 0x03030303u) << 4);
          const uint32_t q1 = ((nib.y >> (4 * hw)) & 0x0F0F0F0Fu) | (((hv >> 2) & 0x03030303u) << 4);
          wq[hw] = (long)(((uint64_t)minus32(q1) << 32) | minus32(q0));
        }
        const v16f f0 = conv(__builtin_amdgcn_mfma_i32_32x32x16_i8(xa0, wq[0], magic, 0, 0, 0));
        const v16f f1 = conv(__builtin_amdgcn_mfma_i32_32x32x16_i8(xa1, wq[1], magic, 0, 0, 0));
        if constexpr (WIDE) {
          const v16f dx = tok16(st + S::dx + u * 128);
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            const float sm = fma_(f1[i], d1, f0[i] * d0);
            acc[i] = fma_(sm, dx[i], acc[i]);
          }
        } else {
          // (d sc_h) dx for both halves: block h of the outer product takes dx (A) and d sc_h (B)
          const float dxl = *reinterpret_cast<const float*>(st + S::dx + u * 128 + li * 4);
          const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(dxl, h ? d1 : d0, zero, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            acc[i] = fma_(f0[i], p[i], acc[i]);
            acc[i] = fma_(f1[i], p[16 + i], acc[i]);
          }
        }
      }
    } else {
      // dx (s0 + s1) of the stage's 4 units x 32 tokens, into this wave's own copy
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int p = 64 * c + lane;
        const float dxv = *reinterpret_cast<const float*>(st + S::dx + 4 * p);
        const uint32_t sv = *reinterpret_cast<const uint32_t*>(st + S::s + 4 * p);
        const int ss = (int)(int16_t)(sv & 0xFFFF) + (int)(int16_t)(sv >> 16);
        *reinterpret_cast<float*>(st + S::dsx + w * 512 + 4 * p) = dxv * (float)ss;
      }
      const uint4 hd = *reinterpret_cast<const uint4*>(st + S::hdr + gi * 128 + r8 * 16);
      const float d = half_to_float((uint16_t)(hd.x & 0xFFFF)), dmin = half_to_float((uint16_t)(hd.x >> 16));
      float fsc[kKB], fmn[kKB];
#pragma unroll
      for (int u = 0; u < kKB; ++u) {
        int sc, m;
        scale_min(4 * hf + u, hd.y, hd.z, hd.w, sc, m);
        fsc[u] = d * (float)sc;
        fmn[u] = dmin * (float)m;
      }
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const uint4 raw = *reinterpret_cast<const uint4*>(st + S::a + cc * 4096 + gi * 256 + h * 128 + r8 * 16);
        // (d sc_j) dx for units 2 cc and 2 cc + 1: block h takes unit 2 cc + h
        const float dxl = *reinterpret_cast<const float*>(st + S::dx + (2 * cc + h) * 128 + li * 4);
        const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(dxl, h ? fsc[2 * cc + 1] : fsc[2 * cc], zero, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int u = 2 * cc + e;
          const v4i wq = e ? v4i{(int)((raw.x >> 4) & 0x0F0F0F0Fu), (int)((raw.y >> 4) & 0x0F0F0F0Fu),
                                 (int)((raw.z >> 4) & 0x0F0F0F0Fu), (int)((raw.w >> 4) & 0x0F0F0F0Fu)}
                           : v4i{(int)(raw.x & 0x0F0F0F0Fu), (int)(raw.y & 0x0F0F0F0Fu), (int)(raw.z & 0x0F0F0F0Fu),
                                 (int)(raw.w & 0x0F0F0F0Fu)};
          const v4i xa = *reinterpret_cast<const v4i*>(st + S::x + u * 1024 + li * 32 + 16 * h);
          const v16f f = conv(__builtin_amdgcn_mfma_i32_32x32x32_i8(xa, wq, magic, 0, 0, 0));
          const v16f dsx = tok16(st + S::dsx + w * 512 + u * 128);
          const float nm = -fmn[u];
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            acc[i] = fma_(f[i], p[16 * e + i], acc[i]);
            acc[i] = fma_(nm, dsx[i], acc[i]);
          }
        }
      }
    }
  };

  auto run = [&]<bool TAIL>() __attribute__((always_inline)) {
    [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
      ((B < nstages ? issue.template operator()<B, TAIL>(B) : void()), ...);
    }(std::make_integer_sequence<int, NS - 1>{});
    for (int s = 0; s < nstages; s += NS) {
      [&]<int... B>(std::integer_sequence<int, B...>) __attribute__((always_inline)) {
        ((s + B < nstages ? stage.template operator()<B, TAIL>(s + B) : void()), ...);
      }(std::make_integer_sequence<int, NS>{});
    }
  };
  if constexpr (TYPE == kQ6_K) {
    if (rt >= n_big)
      run.template operator()<true>();
    else
      run.template operator()<false>();
  } else {
    run.template operator()<false>();
  }

  // Element i: token t0 + 8 (i / 4) + 4 h + i % 4, row 128 rt + 32 w + li.
  if (live) {
    float* yr = y + r0 + 32 * w + li;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = t0 + 8 * (i / 4) + tok_i + i % 4;
      if (t < n) {
        float* o = yr + (int64_t)t * ys;
        *o = accumulate ? *o + acc[i] : acc[i];
      }
    }
  }
}

template <int TYPE, bool WIDE, int NS, int NE>
void launch_kq_ns(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y,
                  int64_t ys, bool accumulate, int n_rt, int n_tt, int n_big) {
  const size_t lds = NS * (size_t)KqLds<TYPE>::bytes;
  static bool attr = false;  // per instantiation: rings past 64 KB of dynamic LDS
  if (!attr) {
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_kq<TYPE, WIDE, NS, NE>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
          "hipFuncSetAttribute");
    attr = true;
  }
  hipLaunchKernelGGL((k_gemm_kq<TYPE, WIDE, NS, NE>), dim3((unsigned)((int64_t)n_rt * n_tt)), dim3(kThreads), lds, s,
                     static_cast<const uint8_t*>(w), rows, cols, x, n, y, ys, accumulate ? 1 : 0, n_rt, n_tt, n_big);
}

// Ring depth by grid size: one workgroup per CU takes an 8-stage ring (7 stages, about 130 KB, in flight), two per CU
// a 4-stage ring; larger grids (prefill) keep 3 stages and several workgroups per CU.
template <int TYPE, bool WIDE>
void launch_kq(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
               bool accumulate) {
  int n_rt = (int)((rows + kRowsT - 1) / kRowsT), n_big = n_rt;
  const int n_tt = (n + kTokT - 1) / kTokT;
  const int64_t cus = device_cus();
  // A short batch over slightly more than one 128-row tile per CU (the 14B gate|up, 34816 rows: 272 tiles) takes one
  // full tile per CU and covers the rest with 32-row tiles (one live wave), so that no CU runs two full tiles.
  // Measured at 17 tokens (bit-identical): Q6_K 34816 x 5120 65.3 -> 62.3 us, 40960 x 5120 66.4 -> 63.6, Q4_K
  // 34816 x 5120 50.5 -> 48.4; at 24 tokens Q6_K 34816 x 5120 78.2 -> 75.6. Q6_K tail tiles copying only their
  // 4 groups' quants and scales (4 instead of 6 copies per wave and stage): 61.9 -> 60.9 us, at 24 tokens 73.3 -> 70.8.
  if (n_tt == 1 && n_rt > cus && rows <= (kRowsT + 32) * cus) {
    n_big = (int)cus;
    n_rt = n_big + (int)((rows - kRowsT * cus) / 32);
  }
  const int64_t wgs = (int64_t)n_rt * n_tt;
  if (wgs <= cus)
    n <= 17 ? launch_kq_ns<TYPE, WIDE, 8, 9>(s, w, rows, cols, x, n, y, ys, accumulate, n_rt, n_tt, n_big)
            : launch_kq_ns<TYPE, WIDE, 8, 16>(s, w, rows, cols, x, n, y, ys, accumulate, n_rt, n_tt, n_big);
  else if (wgs <= 2 * cus)
    n <= 17 ? launch_kq_ns<TYPE, WIDE, 4, 9>(s, w, rows, cols, x, n, y, ys, accumulate, n_rt, n_tt, n_big)
            : launch_kq_ns<TYPE, WIDE, 4, 16>(s, w, rows, cols, x, n, y, ys, accumulate, n_rt, n_tt, n_big);
  else
    launch_kq_ns<TYPE, WIDE, 3, 16>(s, w, rows, cols, x, n, y, ys, accumulate, n_rt, n_tt, n_big);
}

}  // namespace

bool gemm_kq_supported(int type, int64_t rows, int64_t cols, int n) {
  return (type == kQ4_K || type == kQ6_K) && rows % 32 == 0 && cols % 256 == 0 && n > 8;
}

void gemm_kq(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n,
             float* y, int64_t ys, bool accumulate) {
  require(gemm_kq_supported(type, rows, cols, n), "gemm_kq: Q4_K/Q6_K, rows a multiple of 32, cols of 256, n > 8");
  if (type == kQ4_K)
    launch_kq<kQ4_K, false>(s, w, rows, cols, x, n, y, ys, accumulate);
  else if (wide && n > 16)
    launch_kq<kQ6_K, true>(s, w, rows, cols, x, n, y, ys, accumulate);
  else
    launch_kq<kQ6_K, false>(s, w, rows, cols, x, n, y, ys, accumulate);
  check_launch("gemm_kq");
}

}  // namespace mk
