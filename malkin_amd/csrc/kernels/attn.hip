// QK-norm + RoPE + int8 KV write, GQA attention over the int8 KV cache, KV row moves, greedy selection.
// Bit-identical to the reference:
//   qk_norm_rope_kv  model.cpp:370-392 (rmsnorm per head, NeoX RoPE as clang contracts it, quantize_i8 rows)
//   attention        kernels_avx512.cpp:228-267 (attend_t<D/16>) and 282-306 (other head sizes), model.cpp:204-247
//   move_kv_rows     model.cpp:432-440
//   argmax_top2      sampler.cpp:27-30 (first maximum), engine.cpp:309-318 (runner-up scan)
#include <mutex>
#include <utility>

#include "attn_dec.h"
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

// One wavefront per (token, head): heads [0, H) are query heads, [H, H+KV) key heads, [H+KV, H+2KV) value heads.
// Every global operand (the head's values, its norm weights, the RoPE row) is loaded up front.
constexpr int kQkMaxPer = 4;  // D <= 256: up to 4 values per lane

__global__ __launch_bounds__(64) void k_qk_norm_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                                        const float* __restrict__ v, int64_t stride, int H, int KV,
                                                        int D, const float* __restrict__ q_norm,
                                                        const float* __restrict__ k_norm, float eps,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t,
                                                        const int32_t* __restrict__ rpos,
                                                        const int32_t* __restrict__ seq,
                                                        const int32_t* __restrict__ kv_row, KvLayer kv, int n_ctx) {
  const int t = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
  extern __shared__ float sh[];  // D floats
  __shared__ float scale_s, amax_s[64];
  const bool is_q = hh < H, is_k = hh >= H && hh < H + KV, is_v = hh >= H + KV;
  const int head = is_q ? hh : (is_k ? hh - H : hh - H - KV);
  float* vec = is_q ? q + t * stride + (int64_t)head * D : (is_k ? k + t * stride + (int64_t)head * D : nullptr);
  const float* src = is_v ? v + t * stride + (int64_t)head * D : vec;
  const float* w = is_q ? q_norm : k_norm;
  const int64_t pos = rpos[t];
  float xv[kQkMaxPer], wv[kQkMaxPer], cv[kQkMaxPer], sv[kQkMaxPer];
#pragma unroll
  for (int c = 0; c < kQkMaxPer; ++c) {
    const int i = lane + 64 * c;
    if (i < D) {
      xv[c] = src[i];
      if (!is_v) wv[c] = w[i];
    }
    if (!is_v && i < D / 2) {
      cv[c] = cos_t[pos * (D / 2) + i];
      sv[c] = sin_t[pos * (D / 2) + i];
    }
  }
#pragma unroll
  for (int c = 0; c < kQkMaxPer; ++c)
    if (lane + 64 * c < D) sh[lane + 64 * c] = xv[c];
  __syncthreads();
  if (!is_v) {
    // rmsnorm (model.cpp:46-49) over D: 16 fma chains + halving tree.
    if (lane < 16) {
      float acc = 0.0f;
#pragma unroll 4
      for (int i = lane; i < D; i += 16) acc = fma_(sh[i], sh[i], acc);
      acc = reduce16_lanes(acc);
      if (lane == 0) scale_s = 1.0f / sqrtf(acc / (float)D + eps);
    }
    __syncthreads();
    const float s = scale_s;
#pragma unroll
    for (int c = 0; c < kQkMaxPer; ++c)
      if (lane + 64 * c < D) sh[lane + 64 * c] = xv[c] * s * wv[c];
    __syncthreads();
    // RoPE on pairs (i, i + D/2): clang contracts x0*c - x1*s to fma(x0, c, -(x1*s)), x0*s + x1*c to fma(x0, s, x1*c).
#pragma unroll
    for (int c = 0; c < kQkMaxPer; ++c) {
      const int i = lane + 64 * c;
      if (i < D / 2) {
        const float x0 = sh[i], x1 = sh[i + D / 2];
        sh[i] = fma_(x0, cv[c], -(x1 * sv[c]));
        sh[i + D / 2] = fma_(x0, sv[c], x1 * cv[c]);
      }
    }
    __syncthreads();
    if (is_q) {
      for (int i = lane; i < D; i += 64) vec[i] = sh[i];
      return;
    }
  }
  // quantize_i8 (quant.cpp:134-140) into the cache row.
  float amax = 0.0f;
  for (int i = lane; i < D; i += 64) amax = fmaxf(amax, fabsf(sh[i]));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  const int64_t row = ((int64_t)seq[t] * KV + head) * n_ctx + kv_row[t];
  int8_t* dst = (is_v ? kv.v : kv.k) + row * D;
  for (int i = lane; i < D; i += 64) dst[is_v ? i : kv_perm(i, D / 16)] = (int8_t)(int)__builtin_rintf(sh[i] * id);
  if (lane == 0) (is_v ? kv.vs : kv.ks)[row] = d;
}

// Attention of one query head per workgroup, attend_t semantics (D in {64,128,256}, G <= 16):
//   scores  the 16 lane chains of attend_t (mul, then fma over D/16 chunks), the halving tree, times
//           (kv_scale * scale). Permuted K rows (the device cache): 16 lanes per key, lane l holding the D/16 values
//           of chain l contiguously, so a wave reads 4 whole rows per instruction and the halving tree is a 16-lane
//           shuffle tree. Rows in element order: one key per thread, from 16-byte loads. The first round of K rows
//           is issued at entry;
//   softmax exact max, e = exp512(s - max); the 16 sequential lane sums + tree run on otherwise idle threads while
//           the P.V chains start;
//   P.V     one sequential fma chain per output element over all keys in order. V is staged a tile of keys at a
//           time into LDS, converted to fp32 and transposed to [d][key], so a chain step is one fma fed by 16-byte
//           LDS reads (a dependent fma takes 9 cycles on gfx950; an int8 convert in the chain nearly doubles that).
//           Lane i of each 16-lane row reads p of key i of the current 16-key group; DPP broadcasts it to the row.
//           The staging threads form NG groups; group c % NG owns chunk c, loads it into registers NG chunks ahead and
//           stores it to LDS while lanes 0..D-1 run the chains of chunk c - 1. Barriers order LDS only, so the staging
//           loads stay in flight across them (a V load takes about 1 us to return, i.e. some 250 chain steps). Chains run over whole 16-key groups: keys past the end have p = 0 and v = 0, and
//           fma(0, 0, acc) == acc.
constexpr int kAttnThreads = 1024;
constexpr int kSumThread = kAttnThreads - 16;  // threads [1008, 1024) are never stagers (see AttnTile)

template <int D>
struct AttnTile {
  static constexpr int chunk = 8192 / D;                 // keys per V tile: 32 KB of fp32 values
  static constexpr int stride = chunk + 4;               // floats per tile row [d]: 16-byte aligned, spreads banks
  static constexpr int tile = D * stride * 4;            // bytes per tile
  static constexpr int tasks = (chunk / 4) * (D / 16);   // staging task: 4 keys x 16 values
  static constexpr int groups = (kSumThread - D) / tasks;  // staging groups, one chunk in flight each
  static_assert(groups >= 2, "too few staging threads");
};

// LDS: two V tiles, q, scores, p, the token's tree-ancestor rows.
__host__ __device__ constexpr size_t attn_lds_bytes(int tile_bytes, int D, int nk_pad) {
  return 2 * (size_t)tile_bytes + 4 * ((size_t)D + 3 * (size_t)nk_pad);
}

// DC = D / 16 bytes of a permuted K row: the values of one reference lane.
template <int DC>
struct KLane;
template <>
struct KLane<4> {
  using T = uint32_t;
  __device__ static int8_t at(T w, int c) { return (int8_t)(w >> (8 * c)); }
};
template <>
struct KLane<8> {
  using T = uint2;
  __device__ static int8_t at(T w, int c) { return (int8_t)((c < 4 ? w.x : w.y) >> (8 * (c & 3))); }
};
template <>
struct KLane<16> {
  using T = uint4;
  __device__ static int8_t at(T w, int c) { return (int8_t)((&w.x)[c >> 2] >> (8 * (c & 3))); }
};

// One (token, query head) of k_attention / k_attention_long. LONG: the scores and P.V coefficients live in the
// global slot gsc [2][gcap] instead of LDS (any key count); the V tiles start after the softmax, and each chunk's
// coefficients and e values are staged into LDS with its V tile (the chains and the lane sums read LDS only).
template <int D, bool PERM, bool LONG>
__device__ __forceinline__ void attend_pair(int t, int h, const float* __restrict__ q, int64_t q_stride,
                                            float* __restrict__ out, int64_t out_stride, int G, float scale,
                                            const AttnAddr& a, const int32_t* __restrict__ seqs,
                                            const int32_t* __restrict__ n_keys, const int32_t* __restrict__ anc_off,
                                            const int32_t* __restrict__ anc, float* __restrict__ gsc, int gcap,
                                            BlockQ8* __restrict__ xq, int64_t xq_stride) {
  constexpr int DC = D / 16;
  using T = AttnTile<D>;
  const int tid = threadIdx.x;
  const int g = h / G;
  const int n0 = n_keys[t];
  const int e0 = anc_off ? anc_off[t] : 0, ne = anc_off ? anc_off[t + 1] - e0 : 0;
  const int nk = n0 + ne;
  const int nk_pad = attn_keys_pad(nk);
  extern __shared__ int4 smem4[];
  float* tiles = reinterpret_cast<float*>(smem4);                 // 2 x [D][stride] fp32
  float* qs = tiles + 2 * T::tile / 4;                           // D
  // LONG: per chunk (double-buffered) its P.V coefficients and e values, then the ancestors; the full arrays are
  // global.
  float* sc = LONG ? gsc : qs + D;                               // nk_pad: scores, then e^(s - max)
  float* pv = LONG ? gsc + gcap : sc + nk_pad;                   // nk_pad: e * v-scale, zero past nk
  float* pch = qs + D;                                           // LONG: [2][chunk] coefficients
  float* ech = pch + 2 * T::chunk;                               // LONG: [2][chunk] e values
  int* anc_s = reinterpret_cast<int*>(pv + nk_pad);              // !LONG, ne: KV rows of keys n0 .. nk - 1
  __shared__ float red[kAttnThreads / 64];
  __shared__ float inv_s;
  const int64_t sq = seqs[t];
  const int8_t* kb = a.k + sq * a.k_seq + g * a.k_head;
  const int8_t* vb = a.v + sq * a.k_seq + g * a.k_head;
  const char* ksb = a.ks + sq * a.s_seq + g * a.s_head;
  const char* vsb = a.vs + sq * a.s_seq + g * a.s_head;
  // Tree ancestors go to LDS first: a key row read from global memory would make every later load wait for all
  // earlier ones (the compiler's wait counts are per wave and in order), serialising the K and V prefetches.
  // LONG: ancestors are read from global memory (their count is not bounded by the LDS reservation).
  if (!LONG && ne > 0) {
    for (int i = tid; i < ne; i += kAttnThreads) anc_s[i] = anc[e0 + i];
    lds_barrier();
  }
  auto key_row = [&](int j) -> int64_t { return j < n0 ? j : LONG ? anc[e0 + j - n0] : anc_s[j - n0]; };

  // V staging: task = 4 consecutive keys x 16 consecutive values, written as 16 float4 of the transposed tile.
  constexpr int NG = T::groups;
  const bool stager = tid >= D && tid < D + NG * T::tasks;
  const int grp = (tid - D) / T::tasks, task = (tid - D) % T::tasks;
  auto mine = [&](int c) { return stager && grp == c % NG; };
  uint4 vreg[4];
  // LONG: the chunk's coefficients and e values ride with its V rows (2 chunk floats over the group's tasks).
  constexpr int PE = (2 * T::chunk + T::tasks - 1) / T::tasks;
  float pe[LONG ? PE : 1];
  auto load_chunk = [&](int c) {
    if (!mine(c)) return;
    const int kq = task % (T::chunk / 4), db = task / (T::chunk / 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = c * T::chunk + 4 * kq + i;
      vreg[i] = j < nk ? *reinterpret_cast<const uint4*>(vb + key_row(j) * a.k_row + 16 * db) : make_uint4(0, 0, 0, 0);
    }
    if constexpr (LONG) {
#pragma unroll
      for (int u = 0; u < PE; ++u) {
        const int idx = task + u * T::tasks, j = c * T::chunk + idx % T::chunk;
        pe[u] = idx < 2 * T::chunk && j < nk_pad ? (idx < T::chunk ? pv : sc)[j] : 0.0f;
      }
    }
  };
  auto store_chunk = [&](int c) {
    if (!mine(c)) return;
    const int kq = task % (T::chunk / 4), db = task / (T::chunk / 4);
    float* tile = tiles + (c & 1) * (T::tile / 4);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = (float)(int8_t)((&vreg[i].x)[v >> 2] >> (8 * (v & 3)));
      *reinterpret_cast<float4*>(tile + (16 * db + v) * T::stride + 4 * kq) = make_float4(f[0], f[1], f[2], f[3]);
    }
    if constexpr (LONG) {
#pragma unroll
      for (int u = 0; u < PE; ++u) {
        const int idx = task + u * T::tasks;
        if (idx < 2 * T::chunk) (idx < T::chunk ? pch : ech)[(c & 1) * T::chunk + idx % T::chunk] = pe[u];
      }
    }
  };
  const int chunks = (nk + T::chunk - 1) / T::chunk;
  // q first (its wait then covers it alone), then each staging group's first tile: in flight during the scores.
  const float* qh = q + t * q_stride + (int64_t)h * D;
  const float qv = tid < D ? qh[tid] : 0.0f;
  if (!LONG && stager && grp < chunks) load_chunk(grp);  // LONG: the V pipeline starts after the softmax

  if constexpr (PERM) {
    // 16 lanes per key: group grp of the workgroup takes keys grp, grp + 64, ...; KB keys per group in flight.
    // Loads are never predicated (past the last key they re-read it, unused), so the compiler's wait counts stay
    // exact and the next round's loads overlap this round's arithmetic.
    using KL = KLane<DC>;
    constexpr int NGR = kAttnThreads / 16, KB = DC >= 16 ? 4 : 8;
    const int gl = tid & 15, grp = tid >> 4;
    // A round's scales take one load per lane: lane b < 8 of the 16 holds the key scale of key b, lane 8 + b its
    // value scale (KB = 4: lanes 4-7 and 12-15 repeat keys 0-3); DPP broadcasts them at scoring time.
    struct Round {
      typename KL::T k[KB];
      float sv;
    };
    auto fetch = [&](Round& R, int r) {
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const int j = min((r * KB + b) * NGR + grp, nk - 1);
        R.k[b] = *reinterpret_cast<const typename KL::T*>(kb + key_row(j) * a.k_row + DC * gl);
      }
      const int js = min((r * KB + (gl & 7) % KB) * NGR + grp, nk - 1);
      R.sv = *reinterpret_cast<const float*>((gl < 8 ? ksb : vsb) + key_row(js) * a.s_row);
    };
    const int rounds = (nk + NGR * KB - 1) / (NGR * KB);
    Round RA, RB;
    fetch(RA, 0);
    if (tid < D) qs[tid] = qv;
    lds_barrier();
    float qr[DC];  // q of chain gl: q[16 c + gl]
#pragma unroll
    for (int c = 0; c < DC; ++c) qr[c] = qs[16 * c + gl];
    auto score = [&](const Round& R, int r) {
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const int j = (r * KB + b) * NGR + grp;
        if (j < nk) {  // uniform over the 16 lanes of the key
          float acc = qr[0] * (float)KL::at(R.k[b], 0);
#pragma unroll
          for (int c = 1; c < DC; ++c) acc = fma_(qr[c], (float)KL::at(R.k[b], c), acc);
          acc = reduce16_lanes(acc);
          const float ksv = bcast16(R.sv, b), vsv = bcast16(R.sv, 8 + b);
          if (gl == 0) {
            sc[j] = acc * (ksv * scale);
            pv[j] = vsv;
          }
        }
      }
    };
    for (int r = 0; r < rounds; r += 2) {
      fetch(RB, min(r + 1, rounds - 1));
      score(RA, r);
      if (r + 1 >= rounds) break;
      fetch(RA, min(r + 2, rounds - 1));
      score(RB, r + 1);
    }
  } else {
    // K row, key scale and value scale of key j.
    int4 kv[DC];
    float kscale = 0.0f, vscale = 0.0f;
    auto load_key = [&](int j) {
      const int64_t row = key_row(j);
      const int4* kr = reinterpret_cast<const int4*>(kb + row * a.k_row);
#pragma unroll
      for (int c = 0; c < DC; ++c) kv[c] = kr[c];
      kscale = *reinterpret_cast<const float*>(ksb + row * a.s_row);
      vscale = *reinterpret_cast<const float*>(vsb + row * a.s_row);
    };
    if (tid < nk) load_key(tid);
    if (tid < D) qs[tid] = qv;
    lds_barrier();

    // Scores (kernels_avx512.cpp:234-244).
    for (int j = tid; j < nk; j += kAttnThreads) {
      if (j != tid) load_key(j);
      float lanes[16];
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const int w[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
#pragma unroll
        for (int l = 0; l < 16; ++l) {
          const float kf = (float)(int8_t)(w[l >> 2] >> (8 * (l & 3)));
          lanes[l] = c == 0 ? qs[l] * kf : fma_(qs[16 * c + l], kf, lanes[l]);
        }
      }
      sc[j] = reduce16(lanes) * (kscale * scale);
      pv[j] = vscale;
    }
  }
  if constexpr (LONG) {
    __syncthreads();  // the scores are in global memory
  } else {
    store_chunk(0);
    if (NG < chunks) load_chunk(NG);
    lds_barrier();
  }

  // softmax_inplace (kernels_avx512.cpp:205-226).
  float m = -INFINITY;
  for (int j = tid; j < nk; j += kAttnThreads) m = fmaxf(m, sc[j]);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  lds_barrier();
  float mx = red[0];
  for (int i = 1; i < kAttnThreads / 64; ++i) mx = fmaxf(mx, red[i]);
  for (int j = tid; j < nk; j += kAttnThreads) {
    const float e = exp512(sc[j] - mx);
    sc[j] = e;
    pv[j] = e * pv[j];
  }
  for (int j = nk + tid; j < nk_pad; j += kAttnThreads) {
    pv[j] = 0.0f;
    if constexpr (LONG) sc[j] = 0.0f;
  }
  if constexpr (LONG) {
    __syncthreads();  // e and the coefficients are in global memory; now the V pipeline
    if (stager && grp < chunks) load_chunk(grp);
    store_chunk(0);
    if (NG < chunks) load_chunk(NG);
  }
  lds_barrier();

  // P.V (kernels_avx512.cpp:247-265): chunk c from tile c & 1 while chunk c + 1 is stored and c + 1 + NG loaded.
  // The chain waves are latency-bound: at raised priority they issue as soon as their operands are ready instead of
  // queueing behind the staging waves of their SIMD.
  if (tid < D) __builtin_amdgcn_s_setprio(3);
  float acc = 0.0f, lane_sum = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    if (tid < D) {
      const int j0 = c * T::chunk;
      const int len = min(T::chunk, nk_pad - j0);  // a multiple of 16
      const float4* vr = reinterpret_cast<const float4*>(tiles + (c & 1) * (T::tile / 4) + tid * T::stride);
      const float* pc = (LONG ? pch + (c & 1) * T::chunk : pv + j0) + (tid & 15);
      // Two register sets alternate: a 16-key group's LDS reads are issued while the previous group's chain runs
      // (past the last group they re-read it). The scheduling barriers keep the reads ahead of the chain.
      float4 a[4], b[4];
      float pa, pb;
      auto ld = [&](float4(&v)[4], float& p, int jj) {
        const int j = min(jj, len - 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = vr[j / 4 + i];
        p = pc[j];
      };
      auto chain = [&](const float4(&v)[4], float p) {
        acc = fma_bcast16<0>(p, v[0].x, acc);
        acc = fma_bcast16<1>(p, v[0].y, acc);
        acc = fma_bcast16<2>(p, v[0].z, acc);
        acc = fma_bcast16<3>(p, v[0].w, acc);
        acc = fma_bcast16<4>(p, v[1].x, acc);
        acc = fma_bcast16<5>(p, v[1].y, acc);
        acc = fma_bcast16<6>(p, v[1].z, acc);
        acc = fma_bcast16<7>(p, v[1].w, acc);
        acc = fma_bcast16<8>(p, v[2].x, acc);
        acc = fma_bcast16<9>(p, v[2].y, acc);
        acc = fma_bcast16<10>(p, v[2].z, acc);
        acc = fma_bcast16<11>(p, v[2].w, acc);
        acc = fma_bcast16<12>(p, v[3].x, acc);
        acc = fma_bcast16<13>(p, v[3].y, acc);
        acc = fma_bcast16<14>(p, v[3].z, acc);
        acc = fma_bcast16<15>(p, v[3].w, acc);
      };
      ld(a, pa, 0);
      for (int jj = 0; jj < len; jj += 32) {
        ld(b, pb, jj + 16);
        __builtin_amdgcn_sched_barrier(0);
        chain(a, pa);
        if (jj + 16 >= len) break;
        ld(a, pa, jj + 32);
        __builtin_amdgcn_sched_barrier(0);
        chain(b, pb);
      }
    } else if (tid >= kSumThread) {
      const int l = tid - kSumThread;
      // This chunk's part of lane l's sequential sum (chunks are whole 16-key groups): the reads are issued first;
      // keys past the end add +0, which leaves a sum of e >= 0 unchanged.
      const int j0 = c * T::chunk;
      float e[T::chunk / 16];
#pragma unroll
      for (int i = 0; i < T::chunk / 16; ++i) {
        const int j = j0 + l + 16 * i;
        e[i] = j < nk ? (LONG ? ech[(c & 1) * T::chunk + l + 16 * i] : sc[j]) : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < T::chunk / 16; ++i) lane_sum = lane_sum + e[i];
      if (c + 1 == chunks) {
        const float s = reduce16_lanes(lane_sum);
        if (l == 0) inv_s = 1.0f / s;
      }
    } else if (c + 1 < chunks) {
      store_chunk(c + 1);
      if (c + 1 + NG < chunks) load_chunk(c + 1 + NG);
    }
    lds_barrier();
  }
  if (tid < D) put_out(out + t * out_stride + (int64_t)h * D, xq, t * xq_stride, h * D, tid, acc * inv_s);
}

template <int D, bool PERM>
__global__ __launch_bounds__(kAttnThreads) void k_attention(const float* __restrict__ q, int64_t q_stride,
                                                            float* __restrict__ out, int64_t out_stride, int G,
                                                            float scale, AttnAddr a, const int32_t* __restrict__ seqs,
                                                            const int32_t* __restrict__ n_keys,
                                                            const int32_t* __restrict__ anc_off,
                                                            const int32_t* __restrict__ anc, int n, int H,
                                                            BlockQ8* __restrict__ xq, int64_t xq_stride) {
  // Workgroups are dealt to the 8 XCDs in turn (workgroup w on XCD w % 8). (token, head) pairs are numbered
  // KV-group-major (group, token, head in group) and XCD x takes a contiguous run of them: a KV group's K/V rows are
  // read into one XCD's L2, and in prefill every XCD gets tokens of all lengths.
  int t, h;
  if ((n * H) % 8 == 0) {
    const int pair = (int)(blockIdx.x % 8) * (n * H / 8) + (int)(blockIdx.x / 8);
    const int grp = pair / (n * G), rem = pair % (n * G);
    t = rem / G;
    h = grp * G + rem % G;
  } else {
    t = (int)blockIdx.x / H;
    h = (int)blockIdx.x % H;
  }
  attend_pair<D, PERM, false>(t, h, q, q_stride, out, out_stride, G, scale, a, seqs, n_keys, anc_off, anc, nullptr, 0,
                              xq, xq_stride);
}

// Rows with more keys than LDS holds: workgroup w owns the global slot w (2 gcap floats) and takes the (token,
// head) pairs w, w + grid, ... in turn.
template <int D, bool PERM>
__global__ __launch_bounds__(kAttnThreads) void k_attention_long(const float* __restrict__ q, int64_t q_stride,
                                                                 float* __restrict__ out, int64_t out_stride, int G,
                                                                 float scale, AttnAddr a,
                                                                 const int32_t* __restrict__ seqs,
                                                                 const int32_t* __restrict__ n_keys,
                                                                 const int32_t* __restrict__ anc_off,
                                                                 const int32_t* __restrict__ anc, int n, int H,
                                                                 float* __restrict__ gsc, int gcap,
                                                                 BlockQ8* __restrict__ xq, int64_t xq_stride) {
  float* slot = gsc + (size_t)blockIdx.x * 2 * (size_t)gcap;
  for (int pair = (int)blockIdx.x; pair < n * H; pair += (int)gridDim.x) {
    __syncthreads();  // the previous pair's LDS and slot are no longer read
    attend_pair<D, PERM, true>(pair / H, pair % H, q, q_stride, out, out_stride, G, scale, a, seqs, n_keys, anc_off,
                               anc, slot, gcap, xq, xq_stride);
  }
}

// GH query heads of one KV group for one token per workgroup (GH = G = 2..5, or GH = 1; D = 128, permuted K rows,
// the keys in LDS): verification trees and contexts past the decode kernel's LDS. With GH = G every K and V row is
// read, converted and staged once for the G heads instead of G times. Same arithmetic as attend_pair, head by head:
//   scores  16 lanes per key as in attend_pair; each lane holds the D/16 q values of its chain for every head and
//           runs G dot products on the K bytes it loaded once;
//   softmax per head, one pass over the keys for all heads (G maxima, one barrier);
//   P.V     V tiles staged once for the G heads. A chain lane owns one value d and the chains of up to three heads
//           (GH > 3: two head sets on four waves), so one LDS read of V feeds several independent chains;
//   sums    the 16 sequential lane sums per head advance chunk by chunk on the last 16 threads.
constexpr int kGrpMaxHeads = 5;

// V tiles of CK keys as int8, transposed to [value][key] (rows of CK + 16 bytes; a value row's 16-key blocks are
// stored XOR (value / 16) % 8 so that the staging writes spread over the banks), converted to fp32 by the chain lanes
// one 16-key group ahead of the fmas that use them.
template <int GH>
struct GrpCfg {
  static constexpr int D = 128, DC = 8;
  static constexpr int sets = GH <= 3 ? 1 : 2;           // head sets of the chain lanes
  static constexpr int h0 = (GH + sets - 1) / sets;      // heads of set 0 (set 1: GH - h0)
  static constexpr int chain = sets * D;                 // chain threads
  static constexpr int CK = 256, VS = CK + 16;           // keys per V tile, bytes per value row
  static constexpr int tile = D * VS;                    // bytes per tile
  static constexpr int tasks = (CK / 4) * (D / 16);      // staging task: 4 keys x 16 values
  static_assert(chain + tasks <= kSumThread, "too few staging threads");
};

// LDS: two V tiles, q of the GH heads, per head scores then e values and P.V coefficients, the token's ancestors.
__host__ __device__ constexpr size_t grp_lds_bytes(int GH, int nk_pad, int anc_cap) {
  return 2 * (size_t)GrpCfg<2>::tile + 4 * ((size_t)GH * 128 + 2 * (size_t)GH * nk_pad + (size_t)anc_cap);
}

template <int GH>
__global__ __launch_bounds__(kAttnThreads) void k_attention_grp(const float* __restrict__ q, int64_t q_stride,
                                                                float* __restrict__ out, int64_t out_stride, int G,
                                                                float scale, AttnAddr a,
                                                                const int32_t* __restrict__ seqs,
                                                                const int32_t* __restrict__ n_keys,
                                                                const int32_t* __restrict__ anc_off,
                                                                const int32_t* __restrict__ anc, int n, int KV,
                                                                int nk_pad, int anc_cap, BlockQ8* __restrict__ xq,
                                                                int64_t xq_stride) {
  using C = GrpCfg<GH>;
  constexpr int D = C::D, DC = C::DC, CK = C::CK, VS = C::VS;
  const int tid = threadIdx.x;
  // (group, token, head subset) numbered group-major; XCD x (workgroups x, x + 8, ...) takes a contiguous run, so a
  // group's K/V rows are read into one XCD's L2.
  const int hs = G / GH;  // head subsets per group
  int t, g, hsub;
  {
    const int total = n * KV * hs, w = (int)blockIdx.x;
    const int pair = total % 8 == 0 ? (w % 8) * (total / 8) + w / 8 : w;
    g = pair / (n * hs);
    t = (pair / hs) % n;
    hsub = pair % hs;
  }
  const int hfirst = g * G + hsub * GH;  // the workgroup's first query head
  const int n0 = n_keys[t];
  const int e0 = anc_off ? anc_off[t] : 0, ne = anc_off ? anc_off[t + 1] - e0 : 0;
  const int nk = n0 + ne;
  extern __shared__ int4 smem4[];
  uint8_t* tiles = reinterpret_cast<uint8_t*>(smem4);             // 2 x [D][VS] int8
  float* qs = reinterpret_cast<float*>(tiles + 2 * C::tile);     // [GH][D]
  float* sc = qs + GH * D;                                       // [GH][nk_pad]: scores, then e^(s - max)
  float* pv = sc + GH * nk_pad;                                  // [GH][nk_pad]: v-scale, then e * v-scale
  int* anc_s = reinterpret_cast<int*>(pv + GH * nk_pad);         // anc_cap: KV rows of keys n0 .. nk - 1
  __shared__ float red[GH][kAttnThreads / 64];
  __shared__ float inv_s[GH];
  const int64_t sq = seqs[t];
  const int8_t* kb = a.k + sq * a.k_seq + g * a.k_head;
  const int8_t* vb = a.v + sq * a.k_seq + g * a.k_head;
  const char* ksb = a.ks + sq * a.s_seq + g * a.s_head;
  const char* vsb = a.vs + sq * a.s_seq + g * a.s_head;
  // Ancestors to LDS (see attend_pair). They are rows of tokens of this batch, so at most anc_cap = n of them; the
  // index is clamped so that a longer list cannot read past the reservation.
  if (ne > 0) {
    for (int i = tid; i < min(ne, anc_cap); i += kAttnThreads) anc_s[i] = anc[e0 + i];
    lds_barrier();
  }
  auto key_row = [&](int j) -> int64_t { return j < n0 ? j : anc_s[min(j - n0, anc_cap - 1)]; };

  // V staging: task = (quad kq of 4 keys, segment sg of 16 values); every chunk's tasks go to the same threads,
  // which hold one chunk's rows in registers: chunk c + 2 is loaded right after chunk c + 1 is stored, a chunk's
  // chain time ahead of its use. Past the last key the loads re-read it: those keys have coefficient 0 and a finite
  // value, and fma(0, v, acc) == acc (the chain never holds -0).
  const int si = tid - C::chain;
  const bool stager = si >= 0 && si < C::tasks;
  const int ssg = si % (D / 16), skq = si / (D / 16);
  v4i vr[4];
  auto load_chunk = [&](int c) {
    if (!stager) return;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int j = min(c * CK + 4 * skq + x, nk - 1);
      vr[x] = *reinterpret_cast<const v4i*>(vb + key_row(j) * a.k_row + 16 * ssg);
    }
  };
  auto store_chunk = [&](int c) {  // 4 x 4 byte transposes into the [value][key] rows
    if (!stager) return;
    const int col = 16 * ((skq >> 2) ^ (ssg & 7)) + 4 * (skq & 3);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t A = (uint32_t)vr[0][u], B = (uint32_t)vr[1][u];
      const uint32_t Cw = (uint32_t)vr[2][u], E = (uint32_t)vr[3][u];
      const uint32_t t0 = __builtin_amdgcn_perm(B, A, 0x05010400u), t1 = __builtin_amdgcn_perm(B, A, 0x07030602u);
      const uint32_t t2 = __builtin_amdgcn_perm(E, Cw, 0x05010400u), t3 = __builtin_amdgcn_perm(E, Cw, 0x07030602u);
      uint8_t* row = tiles + (c & 1) * C::tile + (16 * ssg + 4 * u) * VS + col;
      *reinterpret_cast<uint32_t*>(row) = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
      *reinterpret_cast<uint32_t*>(row + VS) = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
      *reinterpret_cast<uint32_t*>(row + 2 * VS) = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
      *reinterpret_cast<uint32_t*>(row + 3 * VS) = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
    }
  };
  const int chunks = (nk + CK - 1) / CK;
  const float* qg = q + t * q_stride + (int64_t)hfirst * D;  // the workgroup's GH heads are contiguous
  float qv[(GH * D + kAttnThreads - 1) / kAttnThreads];
#pragma unroll
  for (int i = 0; i < (GH * D + kAttnThreads - 1) / kAttnThreads; ++i) {
    const int e = tid + i * kAttnThreads;
    qv[i] = e < GH * D ? qg[e] : 0.0f;
  }
  load_chunk(0);

  {
    // Scores (kernels_avx512.cpp:234-244): 16 lanes per key, group grp takes keys grp, grp + 64, ...; KB keys per
    // group in flight. Loads are never predicated (past the last key they re-read it, unused).
    using KL = KLane<DC>;
    constexpr int NGR = kAttnThreads / 16, KB = 8;
    const int gl = tid & 15, grp = tid >> 4;
    struct Round {
      typename KL::T k[KB];
      float sv;
    };
    // A key's row: its position below n0; a tree ancestor's KV row from LDS past it (TREE: the batch has ancestors,
    // a uniform choice, so the plain form has no per-key branch). Offsets in 32 bits: a head's rows span
    // n_ctx * (D + 4) bytes.
    auto row_of = [&]<bool TREE>(int j) __attribute__((always_inline)) -> uint32_t {
      if constexpr (TREE) return (uint32_t)(j < n0 ? j : anc_s[min(j - n0, anc_cap - 1)]);
      return (uint32_t)j;
    };
    auto fetch = [&]<bool TREE>(Round& R, int r) __attribute__((always_inline)) {
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const int j = min((r * KB + b) * NGR + grp, nk - 1);
        R.k[b] = *reinterpret_cast<const typename KL::T*>(kb + row_of.template operator()<TREE>(j) *
                                                                   (uint32_t)a.k_row + DC * gl);
      }
      const int js = min((r * KB + (gl & 7) % KB) * NGR + grp, nk - 1);
      R.sv = *reinterpret_cast<const float*>((gl < 8 ? ksb : vsb) +
                                             row_of.template operator()<TREE>(js) * (uint32_t)a.s_row);
    };
    const int rounds = (nk + NGR * KB - 1) / (NGR * KB);
    Round RA, RB;
    if (ne > 0)
      fetch.template operator()<true>(RA, 0);
    else
      fetch.template operator()<false>(RA, 0);
#pragma unroll
    for (int i = 0; i < (GH * D + kAttnThreads - 1) / kAttnThreads; ++i) {
      const int e = tid + i * kAttnThreads;
      if (e < GH * D) qs[e] = qv[i];
    }
    lds_barrier();
    float qr[GH][DC];  // q of chain gl for each head: q_h[16 c + gl]
#pragma unroll
    for (int h = 0; h < GH; ++h)
#pragma unroll
      for (int c = 0; c < DC; ++c) qr[h][c] = qs[h * D + 16 * c + gl];
    // One key: the GH dot products of the lane's chain (mul, then fma over the D/16 values), the halving trees of
    // all heads interleaved; lane 0 of the key stores the scores and (head 0's slot) the value scale.
    auto score = [&](const Round& R, int r) __attribute__((always_inline)) {
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const int j = (r * KB + b) * NGR + grp;
        if (j < nk) {  // uniform over the 16 lanes of the key
          float kf[DC];
#pragma unroll
          for (int c = 0; c < DC; ++c) kf[c] = (float)KL::at(R.k[b], c);
          float acc[GH];
#pragma unroll
          for (int h = 0; h < GH; ++h) {
            acc[h] = qr[h][0] * kf[0];
#pragma unroll
            for (int c = 1; c < DC; ++c) acc[h] = fma_(qr[h][c], kf[c], acc[h]);
          }
          reduce16_lanes_n(acc);
          const float ks2 = bcast16(R.sv, b) * scale, vsv = bcast16(R.sv, 8 + b);
          if (gl == 0) {
#pragma unroll
            for (int h = 0; h < GH; ++h) sc[h * nk_pad + j] = acc[h] * ks2;
            pv[j] = vsv;
          }
        }
      }
    };
    auto loop = [&]<bool TREE>() __attribute__((always_inline)) {
      for (int r = 0; r < rounds; r += 2) {
        fetch.template operator()<TREE>(RB, min(r + 1, rounds - 1));
        score(RA, r);
        if (r + 1 >= rounds) break;
        fetch.template operator()<TREE>(RA, min(r + 2, rounds - 1));
        score(RB, r + 1);
      }
    };
    if (ne > 0)
      loop.template operator()<true>();
    else
      loop.template operator()<false>();
  }
  store_chunk(0);
  if (1 < chunks) load_chunk(1);
  lds_barrier();

  // softmax_inplace (kernels_avx512.cpp:205-226), every head in one pass.
  {
    float m[GH];
#pragma unroll
    for (int h = 0; h < GH; ++h) m[h] = -INFINITY;
    for (int j = tid; j < nk; j += kAttnThreads)
#pragma unroll
      for (int h = 0; h < GH; ++h) m[h] = fmaxf(m[h], sc[h * nk_pad + j]);
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      for (int off = 32; off > 0; off >>= 1) m[h] = fmaxf(m[h], __shfl_xor(m[h], off));
      if ((tid & 63) == 0) red[h][tid >> 6] = m[h];
    }
    lds_barrier();
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      float mx = red[h][0];
      for (int i = 1; i < kAttnThreads / 64; ++i) mx = fmaxf(mx, red[h][i]);
      m[h] = mx;
    }
    for (int j = tid; j < nk; j += kAttnThreads) {
      const float vs = pv[j];  // the key's value scale (head 0's slot)
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        const float e = exp512(sc[h * nk_pad + j] - m[h]);
        sc[h * nk_pad + j] = e;
        pv[h * nk_pad + j] = e * vs;
      }
    }
    for (int j = nk + tid; j < attn_keys_pad(nk); j += kAttnThreads)
#pragma unroll
      for (int h = 0; h < GH; ++h) pv[h * nk_pad + j] = 0.0f;
  }
  lds_barrier();

  // P.V (kernels_avx512.cpp:247-265): chunk c from tile c & 1 while chunk c + 1 is stored and c + 2 loaded.
  const int nk16 = attn_keys_pad(nk);
  const int set = tid / D, d = tid % D;
  const int hb = set * C::h0;  // first head of this chain lane's set
  float acc[C::h0];
#pragma unroll
  for (int k = 0; k < C::h0; ++k) acc[k] = 0.0f;
  float lane_sum[GH];
#pragma unroll
  for (int h = 0; h < GH; ++h) lane_sum[h] = 0.0f;
  if (tid < C::chain) __builtin_amdgcn_s_setprio(3);
  for (int c = 0; c < chunks; ++c) {
    if (tid < C::chain) {
      const int j0 = c * CK;
      const int len = min(CK, nk16 - j0);  // a multiple of 16
      const uint8_t* vrow = tiles + (c & 1) * C::tile + d * VS;
      const int swz = (d >> 4) & 7;
      auto run = [&]<int NH>() __attribute__((always_inline)) {
        const float* pc = pv + hb * nk_pad + j0 + (tid & 15);
        // A 16-key group: its raw bytes and coefficients are read one group ahead; its values are converted before
        // its fmas (one convert feeds NH chains).
        v4i wa, wb;
        float pa[NH], pb[NH];
        auto ld = [&](v4i& w, float(&p)[NH], int jj) {
          const int j = min(jj, len - 16);
          w = *reinterpret_cast<const v4i*>(vrow + 16 * ((j >> 4) ^ swz));
#pragma unroll
          for (int k = 0; k < NH; ++k) p[k] = pc[k * nk_pad + j];
        };
        auto chain = [&](const v4i& w, const float(&p)[NH]) {
          float f[16];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            f[4 * q] = i8_to_f32<0>((uint32_t)w[q]);
            f[4 * q + 1] = i8_to_f32<1>((uint32_t)w[q]);
            f[4 * q + 2] = i8_to_f32<2>((uint32_t)w[q]);
            f[4 * q + 3] = i8_to_f32<3>((uint32_t)w[q]);
          }
          [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
            ((
                 [&] {
#pragma unroll
                   for (int k = 0; k < NH; ++k) acc[k] = fma_bcast16<I>(p[k], f[I], acc[k]);
                 }()),
             ...);
          }(std::make_integer_sequence<int, 16>{});
        };
        ld(wa, pa, 0);
        for (int jj = 0; jj < len; jj += 32) {
          ld(wb, pb, jj + 16);
          __builtin_amdgcn_sched_barrier(0);
          chain(wa, pa);
          if (jj + 16 >= len) break;
          ld(wa, pa, jj + 32);
          __builtin_amdgcn_sched_barrier(0);
          chain(wb, pb);
        }
      };
      if constexpr (C::sets == 1)
        run.template operator()<GH>();
      else if (set == 0)
        run.template operator()<C::h0>();
      else
        run.template operator()<GH - C::h0>();
    } else if (tid >= kSumThread) {
      // this chunk's part of lane l's sequential sum, per head (chunks are whole 16-key groups): a head's reads are
      // issued first; keys past the end add +0, which leaves a sum of e >= 0 unchanged.
      const int l = tid - kSumThread, j0 = c * CK;
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        float e[CK / 16];
#pragma unroll
        for (int i = 0; i < CK / 16; ++i) {
          const int j = j0 + l + 16 * i;
          e[i] = j < nk ? sc[h * nk_pad + j] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < CK / 16; ++i) lane_sum[h] = lane_sum[h] + e[i];
      }
      if (c + 1 == chunks) {
#pragma unroll
        for (int h = 0; h < GH; ++h) {
          const float sm = reduce16_lanes(lane_sum[h]);
          if (l == 0) inv_s[h] = 1.0f / sm;
        }
      }
    } else if (c + 1 < chunks) {
      store_chunk(c + 1);
      if (c + 2 < chunks) load_chunk(c + 2);
    }
    lds_barrier();
  }
  if (tid < C::chain) {
    const int nh = set == 0 ? C::h0 : GH - C::h0;
    float* o = out + t * out_stride + (int64_t)(hfirst + hb) * D + d;
#pragma unroll
    for (int k = 0; k < C::h0; ++k)
      if (k < nh) put_out(o + k * D - d, xq, t * xq_stride, (hfirst + hb + k) * D, d, acc[k] * inv_s[hb + k]);
  }
}

// Attention of many query rows at once (prefill and other long plain batches), attend_t semantics for D in {64, 128}
// and G <= 16, bit-identical to k_attention. A workgroup takes the 16 / G consecutive tokens of one token block and
// the G query heads of one KV group: up to 16 query rows that share every K and V row they read, so each key is
// loaded and converted once per 16 rows instead of once per row.
//   scores  one thread per key: its K row converted to fp32 in registers once, then for each row the 16 lane chains
//           (mul, then fma over the D/16 chunks), the halving tree, times (kv_scale * scale). q is uniform over the
//           workgroup and is read through the scalar unit;
//   softmax 16 threads per row: the row's exact max (keys < n_keys of its token), then the 16 sequential lane sums
//           of e = exp512(s - max), each thread one lane l (keys l, l + 16, ...), and the halving tree; the row's
//           P.V coefficient e * v_scale replaces the score in LDS, 0 past the row's last key;
//   P.V     one sequential fma chain per (row, value) over all keys in order; a lane owns 2 rows x D/32 values. V is
//           staged a tile of keys at a time into LDS as fp32 (double-buffered, one 16-byte load per thread per tile)
//           and read as D/32 consecutive floats per key; the row's coefficients come from LDS once per 16 keys and
//           are broadcast by DPP. Keys past a row's end have coefficient 0 and fma(0, v, acc) == acc.
// Tokens of a block that belong to different sequences are handled one sequence at a time (the rows of the other
// sequences sit out that pass).
constexpr int kRowsThreads = 256;
constexpr int kRowsMax = 16;       // query rows per workgroup
constexpr int kRowsMinTokens = 16; // shorter batches take the per-token kernel (decode, small multi-sequence batches)

template <int D>
struct RowsCfg {
  static constexpr int DC = D / 16;
  static constexpr int ck = 4096 / D;      // keys per V tile: one 16-byte load per thread
  static constexpr int stride = D + 4;     // floats per tile row
  static constexpr int tile = ck * stride; // floats per tile
  static constexpr int dl = D / 32;        // P.V values per lane
};

// LDS: two V tiles, scores [16][nk_pad], v scales [nk_pad].
__host__ __device__ constexpr size_t rows_lds_bytes(int D, int nk_pad) {
  return 4 * (2 * (size_t)(4096 / D) * (size_t)(D + 4) + (size_t)(kRowsMax + 1) * (size_t)nk_pad);
}

template <int D, bool PERM>
__global__ __launch_bounds__(kRowsThreads) void k_attention_rows(const float* __restrict__ q, int64_t q_stride,
                                                                 float* __restrict__ out, int64_t out_stride, int G,
                                                                 float scale, AttnAddr a,
                                                                 const int32_t* __restrict__ seqs,
                                                                 const int32_t* __restrict__ n_keys, int n, int KV,
                                                                 int nk_pad, BlockQ8* __restrict__ xq,
                                                                 int64_t xq_stride) {
  using C = RowsCfg<D>;
  constexpr int DC = C::DC;
  const int tid = threadIdx.x;
  const int TQ = kRowsMax / G, nblk = (n + TQ - 1) / TQ;
  // Workgroup -> (KV group, token block). XCD x (workgroups x, x + 8, ...) takes a contiguous run of
  // (group, block) pairs, so a group's K/V rows are read into one L2; within a group the blocks with the most keys
  // start first.
  int g, blk;
  {
    const int total = nblk * KV, w = (int)blockIdx.x;
    const int pair = total % 8 == 0 ? (w % 8) * (total / 8) + w / 8 : w;
    g = pair / nblk;
    blk = nblk - 1 - pair % nblk;
  }
  const int t0 = blk * TQ, tq = min(TQ, n - t0), R = tq * G;
  extern __shared__ int4 smem4[];
  float* tiles = reinterpret_cast<float*>(smem4);  // 2 x [ck][stride]
  float* sc = tiles + 2 * C::tile;                 // [16][nk_pad]: scores, then P.V coefficients
  float* vsc = sc + kRowsMax * nk_pad;             // [nk_pad]: v scales
  __shared__ int seq_s[kRowsMax], nk_s[kRowsMax];
  __shared__ float inv_s[kRowsMax];
  // Row r: token t0 + r / G, query head g * G + r % G.
  if (tid < kRowsMax) {
    const int t = t0 + min(tid / G, tq - 1);
    const int sv = seqs[t], kv = n_keys[t];
    seq_s[tid] = tid < R ? sv : -1;
    nk_s[tid] = tid < R ? kv : 0;
  }
  lds_barrier();

  const int LR = tid >> 4, dl = tid & 15;
  const int ra = 2 * (LR >> 1), rb = ra + 1;               // P.V rows of this lane
  const int d0 = (LR & 1) * (D / 2) + dl * C::dl;          // P.V values d0 .. d0 + dl - 1
  const int kk = tid / (D / 16), seg = tid % (D / 16);     // V staging: key kk of the tile, bytes 16 seg ..
  const uint32_t all = R >= 32 ? ~0u : (1u << R) - 1;
  uint32_t done = 0;
  while (done != all) {
    // The pass's sequence: that of the first row not done; its rows and their longest key range.
    const int s = __builtin_amdgcn_readfirstlane(seq_s[__builtin_ctz(~done)]);
    uint32_t act = 0;
    int nkb = 1;
    for (int r = 0; r < R; ++r) {
      const int sr = __builtin_amdgcn_readfirstlane(seq_s[r]);
      if (sr == s) {
        act |= 1u << r;
        nkb = max(nkb, __builtin_amdgcn_readfirstlane(nk_s[r]));
      }
    }
    nkb = min(nkb, nk_pad);  // nk_pad covers max_keys, which bounds every token's keys
    const int nkb_pad = attn_keys_pad(nkb);
    const int8_t* kb = a.k + (int64_t)s * a.k_seq + g * a.k_head;
    const int8_t* vb = a.v + (int64_t)s * a.k_seq + g * a.k_head;
    const char* ksb = a.ks + (int64_t)s * a.s_seq + g * a.s_head;
    const char* vsb = a.vs + (int64_t)s * a.s_seq + g * a.s_head;

    // Scores (kernels_avx512.cpp:234-244). Loads are never predicated: past the last key they re-read it, unused.
    for (int j0 = 0; j0 < nkb; j0 += kRowsThreads) {
      const int j = min(j0 + tid, nkb - 1);
      const bool live = j0 + tid < nkb;
      v4i kw[D / 16];
#pragma unroll
      for (int u = 0; u < D / 16; ++u) kw[u] = *reinterpret_cast<const v4i*>(kb + (int64_t)j * a.k_row + 16 * u);
      const float ksv = *reinterpret_cast<const float*>(ksb + (int64_t)j * a.s_row);
      const float vsv = *reinterpret_cast<const float*>(vsb + (int64_t)j * a.s_row);
      float kf[16][DC];  // kf[l][c] = k[16 c + l]
#pragma unroll
      for (int l = 0; l < 16; ++l)
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const int e = PERM ? DC * l + c : 16 * c + l;  // byte of element 16 c + l
          kf[l][c] = (float)(int8_t)(kw[e >> 4][(e >> 2) & 3] >> (8 * (e & 3)));
        }
      if (live) vsc[j] = vsv;
      const float kss = ksv * scale;
      for (int r = 0; r < R; ++r) {
        if (!((act >> r) & 1)) continue;
        const float* qr = q + (int64_t)(t0 + r / G) * q_stride + (int64_t)(g * G + r % G) * D;
        float lanes[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) lanes[l] = qr[l] * kf[l][0];
#pragma unroll
        for (int c = 1; c < DC; ++c)
#pragma unroll
          for (int l = 0; l < 16; ++l) lanes[l] = fma_(qr[16 * c + l], kf[l][c], lanes[l]);
        const float sres = reduce16(lanes) * kss;
        if (live) sc[r * nk_pad + j] = sres;
      }
    }
    lds_barrier();

    // softmax_inplace (kernels_avx512.cpp:205-226): thread (row LR, lane dl).
    {
      const bool on = LR < R && ((act >> LR) & 1);
      const int nkr = on ? nk_s[LR] : 0;
      float* srow = sc + LR * nk_pad;
      float m = -INFINITY;
      for (int j = dl; j < nkr; j += 16) m = fmaxf(m, srow[j]);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 16));
      float sum = 0.0f;
      if (on) {
        for (int j = dl; j < nkb_pad; j += 16) {
          const bool in = j < nkr;
          const float e = in ? exp512(srow[j] - m) : 0.0f;
          sum = sum + e;  // past the row's end e = +0: the sum is unchanged
          srow[j] = in ? e * vsc[j] : 0.0f;
        }
      }
      sum = reduce16_lanes(sum);
      if (dl == 0) inv_s[LR] = 1.0f / sum;
    }

    // P.V (kernels_avx512.cpp:247-265).
    v4i vr;
    auto vload = [&](int c) {
      const int j = min(c * C::ck + kk, nkb - 1);
      vr = *reinterpret_cast<const v4i*>(vb + (int64_t)j * a.k_row + 16 * seg);
    };
    auto vstore = [&](int c) {
      float* dst = tiles + (c & 1) * C::tile + kk * C::stride + 16 * seg;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t x = (uint32_t)vr[w];
        *reinterpret_cast<float4*>(dst + 4 * w) =
            make_float4((float)(int8_t)x, (float)(int8_t)(x >> 8), (float)(int8_t)(x >> 16), (float)(int8_t)(x >> 24));
      }
    };
    const int nch = (nkb_pad + C::ck - 1) / C::ck;
    vload(0);
    vstore(0);
    vload(1);
    lds_barrier();
    float acc0[C::dl], acc1[C::dl];
#pragma unroll
    for (int k = 0; k < C::dl; ++k) acc0[k] = acc1[k] = 0.0f;
    for (int c = 0; c < nch; ++c) {
      const float* tile = tiles + (c & 1) * C::tile + d0;
      const int j0 = c * C::ck;
      const int len = min(C::ck, nkb_pad - j0);  // a multiple of 16
      for (int jj = 0; jj < len; jj += 16) {
        const float pa = sc[ra * nk_pad + j0 + jj + dl], pb = sc[rb * nk_pad + j0 + jj + dl];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p0 = bcast16(pa, i), p1 = bcast16(pb, i);
          float v[C::dl];
          if constexpr (C::dl == 4) {
            const float4 t = *reinterpret_cast<const float4*>(tile + (jj + i) * C::stride);
            v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
          } else {
            const float2 t = *reinterpret_cast<const float2*>(tile + (jj + i) * C::stride);
            v[0] = t.x, v[1] = t.y;
          }
#pragma unroll
          for (int k = 0; k < C::dl; ++k) {
            acc0[k] = fma_(p0, v[k], acc0[k]);
            acc1[k] = fma_(p1, v[k], acc1[k]);
          }
        }
      }
      if (c + 1 < nch) vstore(c + 1);
      lds_barrier();
      vload(c + 2);
    }
    auto put = [&](int r, const float* acc) {
      if (r < R && ((act >> r) & 1)) {
        const int64_t tr = t0 + r / G;
        const int hd = (g * G + r % G) * D;
        float* o = out + tr * out_stride + hd + d0;
        const float inv = inv_s[r];
        float v[C::dl];
#pragma unroll
        for (int k = 0; k < C::dl; ++k) o[k] = v[k] = acc[k] * inv;
        // A Q8 block of the row is 32 / dl consecutive lanes of this lane's 16-lane group (same row).
        if (xq) quantize_block_lanes_n<C::dl>(v, (d0 & 31) / C::dl, xq + tr * xq_stride + (hd + d0) / 32);
      }
    };
    put(ra, acc0);
    put(rb, acc1);
    done |= act;
    lds_barrier();  // the next pass rewrites sc, vsc and the tiles
  }
}

// Other head sizes or G > 16: the per-head path of attend_gqa (kernels_avx512.cpp:296-305), one query head per
// workgroup, byte loads.
__global__ __launch_bounds__(256) void k_attention_generic(const float* __restrict__ q, int64_t q_stride,
                                                           float* __restrict__ out, int64_t out_stride, int G, int D,
                                                           float scale, AttnAddr a,
                                                           const int32_t* __restrict__ seqs,
                                                           const int32_t* __restrict__ n_keys,
                                                           const int32_t* __restrict__ anc_off,
                                                           const int32_t* __restrict__ anc, BlockQ8* __restrict__ xq,
                                                           int64_t xq_stride) {
  const int t = blockIdx.x, h = blockIdx.y, g = h / G, tid = threadIdx.x;
  extern __shared__ float sm[];
  float* qs = sm;
  float* sc = qs + D;
  __shared__ float red[256];
  __shared__ float inv_s;
  const int n0 = n_keys[t];
  const int e0 = anc_off ? anc_off[t] : 0, ne = anc_off ? anc_off[t + 1] - e0 : 0;
  const int nk = n0 + ne;
  float* pv = sc + nk;
  const int64_t sq = seqs[t];
  const int8_t* kb = a.k + sq * a.k_seq + g * a.k_head;
  const int8_t* vb = a.v + sq * a.k_seq + g * a.k_head;
  const char* ksb = a.ks + sq * a.s_seq + g * a.s_head;
  const char* vsb = a.vs + sq * a.s_seq + g * a.s_head;
  const float* qh = q + t * q_stride + (int64_t)h * D;
  for (int i = tid; i < D; i += 256) qs[i] = qh[i];
  __syncthreads();
  for (int j = tid; j < nk; j += 256) {
    const int64_t row = j < n0 ? j : anc[e0 + j - n0];
    const int8_t* kr = kb + row * a.k_row;
    const float kscale = *reinterpret_cast<const float*>(ksb + row * a.s_row);
    auto kat = [&](int e) { return (float)kr[a.k_perm ? kv_perm(e, D / 16) : e]; };
    float lanes[16];
    for (int l = 0; l < 16; ++l) lanes[l] = qs[l] * kat(l);
    for (int c = 16; c < D; c += 16)
      for (int l = 0; l < 16; ++l) lanes[l] = fma_(qs[c + l], kat(c + l), lanes[l]);
    sc[j] = reduce16(lanes) * kscale * scale;  // (dot * kv_scale) * scale
  }
  __syncthreads();
  float m = -INFINITY;
  for (int j = tid; j < nk; j += 256) m = fmaxf(m, sc[j]);
  red[tid] = m;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
    __syncthreads();
  }
  const float mx = red[0];
  __syncthreads();
  for (int j = tid; j < nk; j += 256) sc[j] = exp512(sc[j] - mx);
  __syncthreads();
  if (tid < 16) {
    float s = 0.0f;
    for (int j = tid; j < nk; j += 16) s = s + sc[j];
    s = reduce16_lanes(s);
    if (tid == 0) inv_s = 1.0f / s;
  }
  __syncthreads();
  const float inv = inv_s;
  for (int j = tid; j < nk; j += 256) {
    const int64_t row = j < n0 ? j : anc[e0 + j - n0];
    pv[j] = sc[j] * inv * *reinterpret_cast<const float*>(vsb + row * a.s_row);  // (p * inv) * v-scale
  }
  __syncthreads();
  for (int d = tid; d < D; d += 256) {
    float acc = 0.0f;
    for (int j = 0; j < nk; ++j) {
      const int64_t r = j < n0 ? j : anc[e0 + j - n0];
      acc = fma_(pv[j], (float)vb[r * a.k_row + d], acc);
    }
    // With xq, D % 32 == 0: a Q8 block is 32 consecutive threads, all in the loop or all past it.
    put_out(out + t * out_stride + (int64_t)h * D, xq, t * xq_stride, h * D, d, acc);
  }
}

__global__ void k_move_kv(int8_t* k8, int8_t* v8, float* ks, float* vs, int n_seq, int KV, int D, int n_ctx, int seq,
                          int from, int to) {
  const int il = blockIdx.x, g = blockIdx.y;
  const int64_t base = (((int64_t)il * n_seq + seq) * KV + g) * n_ctx;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    k8[(base + to) * D + i] = k8[(base + from) * D + i];
    v8[(base + to) * D + i] = v8[(base + from) * D + i];
  }
  if (threadIdx.x == 0) {
    ks[base + to] = ks[base + from];
    vs[base + to] = vs[base + from];
  }
}

// Total order "better": larger value, then smaller index.
__device__ __forceinline__ bool better(float v1, int i1, float v2, int i2) {
  return v1 > v2 || (v1 == v2 && i1 < i2);
}

struct Top2 {
  float v1, v2;
  int i1, i2;
};

__device__ __forceinline__ void push(Top2& t, float v, int i) {
  if (better(v, i, t.v1, t.i1)) {
    t.v2 = t.v1;
    t.i2 = t.i1;
    t.v1 = v;
    t.i1 = i;
  } else if (better(v, i, t.v2, t.i2)) {
    t.v2 = v;
    t.i2 = i;
  }
}

constexpr int kSelT = 256;
constexpr int kSelParts = 64;  // workgroups per logits row

__device__ __forceinline__ void block_top2(Top2& t, Top2* red) {
  red[threadIdx.x] = t;
  __syncthreads();
  for (int st = kSelT / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) {
      Top2 a = red[threadIdx.x];
      const Top2 b = red[threadIdx.x + st];
      push(a, b.v1, b.i1);
      push(a, b.v2, b.i2);
      red[threadIdx.x] = a;
    }
    __syncthreads();
  }
  t = red[0];
}

// Top-1 under (value desc, index asc) is std::max_element's first maximum; top-2 is the best of the rest under the
// same order, which is what the reference's strict-'>' runner-up scan returns. Pass 1: kSelParts workgroups per row
// each reduce a slice; pass 2 merges the slices (the order is total, so the merge is associative).
__global__ __launch_bounds__(kSelT) void k_top2_part(const float* __restrict__ logits, int n, Top2* __restrict__ part) {
  const int row = blockIdx.y, p = blockIdx.x;
  const float* l = logits + (int64_t)row * n;
  const int per = (n + kSelParts - 1) / kSelParts, lo = p * per, hi = min(n, lo + per);
  Top2 t{-INFINITY, -INFINITY, 0x7fffffff, 0x7fffffff};
  for (int i = lo + threadIdx.x; i < hi; i += kSelT) push(t, l[i], i);
  __shared__ Top2 red[kSelT];
  block_top2(t, red);
  if (threadIdx.x == 0) part[row * kSelParts + p] = t;
}

__global__ __launch_bounds__(kSelParts) void k_top2_merge(const Top2* __restrict__ part, int32_t* top1,
                                                          int32_t* top2) {
  const int row = blockIdx.x;
  __shared__ Top2 red[kSelParts];
  red[threadIdx.x] = part[row * kSelParts + threadIdx.x];
  __syncthreads();
  for (int st = kSelParts / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) {
      Top2 a = red[threadIdx.x];
      const Top2 b = red[threadIdx.x + st];
      push(a, b.v1, b.i1);
      push(a, b.v2, b.i2);
      red[threadIdx.x] = a;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    top1[row] = red[0].i1;
    if (top2) top2[row] = red[0].i2;
  }
}

__global__ void k_greedy_advance(const int32_t* top1, int32_t* ids, int32_t* rpos, int32_t* kv_row, int32_t* n_keys,
                                 int32_t* out_tokens, int32_t* counter) {
  const int32_t tok = *top1;
  out_tokens[*counter] = tok;
  *counter += 1;
  ids[0] = tok;
  rpos[0] += 1;
  kv_row[0] += 1;
  n_keys[0] += 1;
}

// dst[dst_idx[i]] = src[src_idx[i]] for i < n (identity where an index array is null; a negative index skips i).
__global__ void k_move_ids(int32_t* __restrict__ dst, const int32_t* __restrict__ dst_idx,
                           const int32_t* __restrict__ src, const int32_t* __restrict__ src_idx, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int d = dst_idx ? dst_idx[i] : i, s = src_idx ? src_idx[i] : i;
  if (d >= 0 && s >= 0) dst[d] = src[s];
}

}  // namespace

void move_ids(hipStream_t s, int32_t* dst, const int32_t* dst_idx, const int32_t* src, const int32_t* src_idx,
              int n) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_move_ids, dim3((n + 255) / 256), dim3(256), 0, s, dst, dst_idx, src, src_idx, n);
  check_launch("move_ids");
}

void greedy_advance(hipStream_t s, const int32_t* top1, int32_t* ids, int32_t* rpos, int32_t* kv_row, int32_t* n_keys,
                    int32_t* out_tokens, int32_t* counter) {
  hipLaunchKernelGGL(k_greedy_advance, dim3(1), dim3(1), 0, s, top1, ids, rpos, kv_row, n_keys, out_tokens, counter);
  check_launch("greedy_advance");
}

void qk_norm_rope_kv(hipStream_t s, float* q, float* k, const float* v, int64_t stride, int n, int H, int KV, int D,
                     const float* q_norm, const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                     const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const KvLayer& kv, int n_ctx) {
  if (n <= 0) return;
  require(D % 16 == 0 && D <= 64 * kQkMaxPer, "qk_norm_rope_kv: head_dim must be a multiple of 16, at most 256");
  hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3(n, H + 2 * KV), dim3(64), D * sizeof(float), s, q, k, v, stride, H, KV,
                     D, q_norm, k_norm, eps, cos_t, sin_t, rpos, seq, kv_row, kv, n_ctx);
  check_launch("qk_norm_rope_kv");
}

namespace {

bool dec_ok(int G, int D, const AttnAddr& a, int max_keys) {
  return G <= 16 && (D == 64 || D == 128) && a.k_perm && attn_aligned(a) && dec_fits(D, max_keys);
}

template <bool FUSE>
void launch_dec(hipStream_t s, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int H, int D,
                int G, float scale, const AttnAddr& a, const int32_t* seq, const int32_t* n_keys, int max_keys,
                const DecFuse& f, BlockQ8* xq, int64_t xq_stride) {
  const size_t lds = dec_lds_bytes(D, attn_keys_pad(max_keys));
  auto go = [&](auto kernel) {
    static bool attr = false;
    if (!attr) {
      check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024 - 1024),
            "hipFuncSetAttribute");
      attr = true;
    }
    hipLaunchKernelGGL(kernel, dim3(n * H), dim3(kDecThreads), lds, s, q, q_stride, out, out_stride, G, scale, a, seq,
                       n_keys, n, H, f, xq, xq_stride);
  };
  const int slots = dec_slots(D, max_keys, FUSE);
  if (D == 64) {
    slots == 1   ? go(k_attention_dec<64, 1, FUSE>)
    : slots == 2 ? go(k_attention_dec<64, 2, FUSE>)
                 : go(k_attention_dec<64, 3, FUSE>);
  } else {
    slots == 1   ? go(k_attention_dec<128, 1, FUSE>)
    : slots == 2 ? go(k_attention_dec<128, 2, FUSE>)
                 : go(k_attention_dec<128, 3, FUSE>);
  }
}

}  // namespace

bool attention_decode_fused(hipStream_t s, const float* qkv, int64_t stride, float* out, int64_t out_stride, int n,
                            int H, int KV, int D, float scale, const AttnAddr& a, const float* q_norm,
                            const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                            const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys,
                            const KvLayer& kv, int n_ctx, int max_keys, BlockQ8* xq, int64_t xq_stride) {
  if (n <= 0) return true;
  require(!xq || D % 32 == 0, "attention_decode_fused: Q8 rows need head_dim % 32 == 0");
  if (H % KV != 0 || !dec_ok(H / KV, D, a, max_keys)) return false;
  const DecFuse f{qkv, stride, q_norm, k_norm, eps, cos_t, sin_t, rpos, kv_row, kv, n_ctx, KV};
  launch_dec<true>(s, nullptr, 0, out, out_stride, n, H, D, H / KV, scale, a, seq, n_keys, max_keys, f, xq,
                   xq_stride);
  check_launch("attention_decode_fused");
  return true;
}

size_t attention_scratch_bytes(int D, int max_keys, int pairs) {
  const int tile = D == 64 ? AttnTile<64>::tile : D == 128 ? AttnTile<128>::tile : AttnTile<256>::tile;
  const int nk_pad = attn_keys_pad(max_keys);
  if (attn_lds_bytes(tile, D, nk_pad) <= 160 * 1024 - 1024) return 0;
  // D = 128 over the device cache: the grouped kernel with one head per workgroup holds more keys in LDS
  if (D == 128 && grp_lds_bytes(1, nk_pad, std::min(pairs, nk_pad)) <= 160 * 1024 - 1024) return 0;
  return (size_t)std::min(pairs, 1024) * 2 * (size_t)nk_pad * sizeof(float);
}

// Heads per workgroup of the grouped kernel for this batch (0: not used). All G heads of a KV group (G = 2..5) when one
// workgroup per (token, head) would take more than one round of the CUs: a grouped workgroup costs about twice a
// single-head one (2057 keys, G = 5: 62 vs 31 us), so with fewer pairs than CUs one head per workgroup is faster.
int grp_heads(int n, int H, int G, int D, const AttnAddr& a, const int32_t* anc_off, int max_keys) {
  if (D != 128 || !a.k_perm || !attn_aligned(a) || G > 16) return 0;
  const int nk_pad = attn_keys_pad(max_keys), anc_cap = anc_off ? std::min(n, nk_pad) : 0;
  const size_t limit = 160 * 1024 - 1024;
  if (G >= 2 && G <= kGrpMaxHeads && (int64_t)n * H > device_cus() && grp_lds_bytes(G, nk_pad, anc_cap) <= limit)
    return G;
  return grp_lds_bytes(1, nk_pad, anc_cap) <= limit ? 1 : 0;
}

void attention(hipStream_t s, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int H, int KV,
               int D, float scale, const AttnAddr& a, const int32_t* seq, const int32_t* n_keys,
               const int32_t* anc_off, const int32_t* anc, int max_keys, void* scratch, size_t scratch_bytes,
               BlockQ8* xq, int64_t xq_stride) {
  if (n <= 0) return;
  require(D % 16 == 0 && D <= 256 && H % KV == 0 && max_keys > 0, "attention: unsupported head layout");
  require(!xq || D % 32 == 0, "attention: Q8 rows need head_dim % 32 == 0");
  const int G = H / KV;
  const bool aligned = attn_aligned(a);
  if (!anc_off && n >= kRowsMinTokens && G <= 16 && (D == 64 || D == 128) && aligned &&
      rows_lds_bytes(D, attn_keys_pad(max_keys)) <= 160 * 1024 - 1024) {
    const int nk_pad = attn_keys_pad(max_keys);
    const size_t lds = rows_lds_bytes(D, nk_pad);
    auto go = [&](auto kernel) {
      static bool attr = false;
      if (!attr) {
        check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024 - 1024),
              "hipFuncSetAttribute");
        attr = true;
      }
      const int TQ = kRowsMax / G;
      hipLaunchKernelGGL(kernel, dim3(((n + TQ - 1) / TQ) * KV), dim3(kRowsThreads), lds, s, q, q_stride, out,
                         out_stride, G, scale, a, seq, n_keys, n, KV, nk_pad, xq, xq_stride);
    };
    if (D == 64)
      a.k_perm ? go(k_attention_rows<64, true>) : go(k_attention_rows<64, false>);
    else
      a.k_perm ? go(k_attention_rows<128, true>) : go(k_attention_rows<128, false>);
  } else if (!anc_off && dec_ok(G, D, a, max_keys)) {
    launch_dec<false>(s, q, q_stride, out, out_stride, n, H, D, G, scale, a, seq, n_keys, max_keys, DecFuse{}, xq,
                      xq_stride);
  } else if (grp_heads(n, H, G, D, a, anc_off, max_keys) > 0) {
    // Grouped workgroups (trees, keys past the decode kernel's LDS): all heads of a KV group per workgroup where one
    // workgroup per (token, head) would take more than one round of the CUs, else one head per workgroup.
    const int GH = grp_heads(n, H, G, D, a, anc_off, max_keys);
    const int nk_pad = attn_keys_pad(max_keys), anc_cap = anc_off ? std::min(n, nk_pad) : 0;
    const size_t lds = grp_lds_bytes(GH, nk_pad, anc_cap);
    auto go = [&](auto kernel) {
      static bool done = false;
      if (!done) {
        check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024 - 1024),
              "hipFuncSetAttribute");
        done = true;
      }
      hipLaunchKernelGGL(kernel, dim3(n * KV * (G / GH)), dim3(kAttnThreads), lds, s, q, q_stride, out, out_stride, G,
                         scale, a, seq, n_keys, anc_off, anc, n, KV, nk_pad, anc_cap, xq, xq_stride);
    };
    switch (GH) {
      case 1: go(k_attention_grp<1>); break;
      case 2: go(k_attention_grp<2>); break;
      case 3: go(k_attention_grp<3>); break;
      case 4: go(k_attention_grp<4>); break;
      default: go(k_attention_grp<5>); break;
    }
  } else if (G <= 16 && (D == 64 || D == 128 || D == 256) && aligned) {
    const int tile = D == 64 ? AttnTile<64>::tile : D == 128 ? AttnTile<128>::tile : AttnTile<256>::tile;
    const int nk_pad = attn_keys_pad(max_keys);
    const size_t lds = attn_lds_bytes(tile, D, nk_pad);
    auto attr = [&](auto kernel, bool& done) {
      if (!done) {
        check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024 - 1024),
              "hipFuncSetAttribute");
        done = true;
      }
    };
    if (lds <= 160 * 1024 - 1024) {
      auto go = [&](auto kernel) {
        static bool done = false;
        attr(kernel, done);
        hipLaunchKernelGGL(kernel, dim3(n * H), dim3(kAttnThreads), lds, s, q, q_stride, out, out_stride, G, scale, a,
                           seq, n_keys, anc_off, anc, n, H, xq, xq_stride);
      };
      if (D == 64)
        a.k_perm ? go(k_attention<64, true>) : go(k_attention<64, false>);
      else if (D == 128)
        a.k_perm ? go(k_attention<128, true>) : go(k_attention<128, false>);
      else
        a.k_perm ? go(k_attention<256, true>) : go(k_attention<256, false>);
    } else {
      // More keys than LDS holds: scores and coefficients in global slots of the caller's scratch.
      const size_t slot = 2 * (size_t)nk_pad * sizeof(float);
      const int slots = (int)std::min<size_t>({(size_t)n * H, scratch_bytes / slot, (size_t)1024});
      require(scratch && slots >= 1, "attention: too many keys for the scratch buffer (mk_reserve_scratch)");
      const int chunk = D == 64 ? AttnTile<64>::chunk : D == 128 ? AttnTile<128>::chunk : AttnTile<256>::chunk;
      const size_t lds_long = 2 * (size_t)tile + 4 * ((size_t)D + 4 * (size_t)chunk);
      auto go = [&](auto kernel) {
        static bool done = false;
        attr(kernel, done);
        hipLaunchKernelGGL(kernel, dim3(slots), dim3(kAttnThreads), lds_long, s, q, q_stride, out, out_stride, G,
                           scale, a, seq, n_keys, anc_off, anc, n, H, static_cast<float*>(scratch), nk_pad, xq,
                           xq_stride);
      };
      if (D == 64)
        a.k_perm ? go(k_attention_long<64, true>) : go(k_attention_long<64, false>);
      else if (D == 128)
        a.k_perm ? go(k_attention_long<128, true>) : go(k_attention_long<128, false>);
      else
        a.k_perm ? go(k_attention_long<256, true>) : go(k_attention_long<256, false>);
    }
  } else {
    const size_t lds = (size_t)(D + 2 * (size_t)max_keys) * sizeof(float);
    require(lds <= 60 * 1024, "attention: too many keys for one workgroup");
    const bool ref_order = G <= 16 && (D == 64 || D == 128 || D == 256);
    require(!ref_order, "attention: K/V rows must be 16-byte aligned");
    hipLaunchKernelGGL(k_attention_generic, dim3(n, H), dim3(256), lds, s, q, q_stride, out, out_stride, G, D, scale,
                       a, seq, n_keys, anc_off, anc, xq, xq_stride);
  }
  check_launch("attention");
}

void move_kv_rows(hipStream_t s, int8_t* k8, int8_t* v8, float* ks, float* vs, int n_layer, int n_seq, int KV, int D,
                  int n_ctx, int seq, int from, int to) {
  if (from == to) return;
  hipLaunchKernelGGL(k_move_kv, dim3(n_layer, KV), dim3(128), 0, s, k8, v8, ks, vs, n_seq, KV, D, n_ctx, seq, from,
                     to);
  check_launch("move_kv");
}

size_t argmax_scratch_bytes(int rows) { return (size_t)rows * kSelParts * sizeof(Top2); }

void argmax_top2(hipStream_t s, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2,
                 void* scratch, size_t scratch_bytes) {
  if (rows <= 0) return;
  require(n_vocab >= 2, "argmax_top2: need at least two logits");
  require(argmax_scratch_bytes(rows) <= scratch_bytes, "argmax_top2: too many rows for the context scratch");
  Top2* part = static_cast<Top2*>(scratch);
  hipLaunchKernelGGL(k_top2_part, dim3(kSelParts, rows), dim3(kSelT), 0, s, logits, n_vocab, part);
  hipLaunchKernelGGL(k_top2_merge, dim3(rows), dim3(kSelParts), 0, s, part, top1, top2);
  check_launch("argmax_top2");
}

}  // namespace mk

// ---- allocation-free greedy selection (mk_argmax_top2_noalloc) ----
// k_top2_part's per-row partial results for callers that cannot allocate device memory: a file-scope array of
// kNoAllocSelectRows rows (256 KiB), one copy per GPU the library runs on, held until the process ends. In host code
// this name is only a stand-in; its device address comes from hipGetSymbolAddress (noalloc_select_scratch).
static __device__ __align__(256) unsigned char scratch[mk::kNoAllocSelectRows * mk::kSelParts * sizeof(mk::Top2)];

namespace mk {

namespace {
constexpr int kMaxDevices = 64;
}

// Device address of `scratch` on the stream's device, resolved once per device with that device current.
static void* noalloc_select_scratch(hipStream_t s) {
  int dev = 0;
  if (s)
    check(hipStreamGetDevice(s, &dev), "hipStreamGetDevice");
  else
    check(hipGetDevice(&dev), "hipGetDevice");
  require(dev >= 0 && dev < kMaxDevices, "mk_argmax_top2_noalloc: device index out of range");
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    int cur = 0;
    check(hipGetDevice(&cur), "hipGetDevice");
    if (cur != dev) check(hipSetDevice(dev), "hipSetDevice");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    check(e, "hipGetSymbolAddress(scratch)");
    addr[dev] = p;
  }
  return addr[dev];
}

void argmax_top2_noalloc(hipStream_t s, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2) {
  require(rows <= kNoAllocSelectRows, "mk_argmax_top2_noalloc: more than 256 rows (its static scratch holds 256)");
  // k_top2_part writes every (row, part) entry it covers before k_top2_merge reads it: nothing needs clearing.
  argmax_top2(s, logits, rows, n_vocab, top1, top2, noalloc_select_scratch(s),
              (size_t)kNoAllocSelectRows * kSelParts * sizeof(Top2));
}

}  // namespace mk
