// Decode attention (one query head of one token per workgroup over the int8 device KV cache), shared by the attention
// launches (attn.hip) and the persistent decode kernel (decode.hip). Bit-identical to the reference's attend_t
// (kernels_avx512.cpp:228-267) with the fused QK-norm / RoPE / KV write of model.cpp:370-392.
#pragma once

#include "ops.h"

namespace mk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int attn_keys_pad(int nk) { return (nk + 15) & ~15; }

// Attention of one query head of one token per workgroup for plain tokens (decode steps and other short plain
// batches), attend_t semantics for D in {64, 128} and G <= 16, bit-identical to k_attention, over the permuted K
// rows of the device cache. Its keys' V rows are staged once, transposed to [value][key] int8 in LDS, while the
// scores are computed, so the P.V chains run without further barriers:
//   scores  as in k_attention (16 lanes per key, KB keys per 16-lane group in flight, the scales of a round in one
//           load per lane, broadcast by DPP);
//   V       a staging task = 4 keys x 16 values: four 16-byte loads issued at entry (the D/16 tasks of a key quad on
//           consecutive lanes, so each load instruction reads whole rows), a 4 x 4 byte transpose per word
//           (v_perm_b32), four-key words written to the [value][key] rows. Rows are 16 bytes longer than a multiple of
//           128, so the 16-byte reads of the chains (lane = value) fall in distinct banks, and the 16-key blocks of
//           row i sit at block b ^ ((i / 16) % 8), so the writes of the D/16 segments of a quad do too;
//   P.V     lane i runs the chain of value i: per 16 keys one 16-byte LDS read of its row, a DPP-broadcast p per key
//           folded into the fma, the int8 convert off the chain (SDWA). Reads run one 16-key group ahead. Keys past
//           the end have p = 0 and finite v, and fma(0, v, acc) == acc;
//   sum     16 otherwise idle threads run the 16 sequential lane sums of softmax_inplace during the chains.
constexpr int kDecThreads = 1024;  // threads per workgroup of k_attention_dec (the body takes any multiple of 256)
constexpr int kDecMaxTasks = 3;    // V staging tasks per thread of k_attention_dec

__host__ __device__ constexpr int dec_vstride(int nk_pad) { return ((nk_pad + 127) & ~127) + 16; }
// LDS: the transposed V rows, scores, p, q.
__host__ __device__ constexpr size_t dec_lds_bytes(int D, int nk_pad) {
  return (size_t)D * (size_t)dec_vstride(nk_pad) + 4 * (2 * (size_t)nk_pad + (size_t)D);
}
// V staging threads: with the fused QK-norm / RoPE / KV-write step its three waves stage nothing (the others
// transpose V while they run).
__host__ __device__ constexpr int dec_stagers(bool fuse, int nt = kDecThreads) { return fuse ? nt - 3 * 64 : nt; }
__host__ __device__ constexpr int dec_slots(int D, int nk, bool fuse, int nt = kDecThreads) {
  return (((nk + 3) / 4) * (D / 16) + dec_stagers(fuse, nt) - 1) / dec_stagers(fuse, nt);
}
__host__ __device__ constexpr bool dec_fits(int D, int nk, int nt = kDecThreads, int max_tasks = kDecMaxTasks) {
  return dec_lds_bytes(D, attn_keys_pad(nk)) <= 160 * 1024 - 1024 &&
         ((nk + 3) / 4) * (D / 16) <= max_tasks * dec_stagers(true, nt);
}

// The fused QK-norm / RoPE / KV-write step of k_attention_dec (model.cpp:370-392, the arithmetic of
// k_qk_norm_rope_kv): one wave per role (0: query head h, 1: key head g, 2: value head g), D/64 values per lane.
// Role 0 leaves q in qs; roles 1 and 2 leave the quantized rows (K permuted) and their scales in LDS and, in the
// group's writer workgroup, in the cache row kv_row[t] of the token's sequence.
// 16-byte K/V row loads and 4-byte scale loads are legal for this cache layout.
inline bool attn_aligned(const AttnAddr& a) {
  return a.k_row % 16 == 0 && a.k_head % 16 == 0 && a.k_seq % 16 == 0 && reinterpret_cast<uintptr_t>(a.k) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(a.v) % 16 == 0 && a.s_row % 4 == 0 && reinterpret_cast<uintptr_t>(a.ks) % 4 == 0 &&
         reinterpret_cast<uintptr_t>(a.vs) % 4 == 0;
}

struct DecFuse {
  const float* qkv;  // token t: the H query heads, then KV key heads, then KV value heads (raw), at qkv + t * stride
  int64_t stride;
  const float* q_norm;
  const float* k_norm;
  float eps;
  const float* cos_t;  // [n_pos][D / 2]
  const float* sin_t;
  const int32_t* rpos;
  const int32_t* kv_row;
  KvLayer kv;
  int n_ctx, KV;
};

template <int D, int role, bool COH>
__device__ __forceinline__ void fuse_qkv(const DecFuse& f, int t, int h, int g, int lane, int H, int64_t sq, int jo,
                                         bool writer, float* qs, float* kscratch, int8_t* own_k, int8_t* own_v,
                                         float* own_sc) {
  constexpr int NPL = D / 64, DC = D / 16;
  const float* row = f.qkv + t * f.stride + (int64_t)(role == 0 ? h * D : role == 1 ? (H + g) * D : (H + f.KV + g) * D);
  const float* w = role == 0 ? f.q_norm : f.k_norm;
  const int64_t pos = f.rpos[t];
  float x[NPL], wv[NPL], cv = 0.0f, sv = 0.0f;
#pragma unroll
  for (int u = 0; u < NPL; ++u) x[u] = COH ? ld_coh(row + lane + 64 * u) : row[lane + 64 * u];
  if constexpr (role < 2) {
#pragma unroll
    for (int u = 0; u < NPL; ++u) wv[u] = w[lane + 64 * u];
    if (lane < D / 2) {
      cv = f.cos_t[pos * (D / 2) + lane];
      sv = f.sin_t[pos * (D / 2) + lane];
    }
    // rmsnorm over D (model.cpp:46-49): lane l < 16 runs the chain over x[l], x[l + 16], ..., then the halving tree.
    float* sh = role == 0 ? qs : kscratch;  // D floats of LDS per role
#pragma unroll
    for (int u = 0; u < NPL; ++u) sh[lane + 64 * u] = x[u];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    float acc = 0.0f;
    if (lane < 16) {
#pragma unroll
      for (int c = 0; c < DC; ++c) acc = fma_(sh[16 * c + lane], sh[16 * c + lane], acc);
    }
    acc = reduce16_lanes(acc);
    const float tot = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, acc)));
    const float s = 1.0f / sqrtf(tot / (float)D + f.eps);
#pragma unroll
    for (int u = 0; u < NPL; ++u) x[u] = x[u] * s * wv[u];
    // NeoX RoPE on pairs (i, i + D/2) as clang contracts it: fma(x0, c, -(x1 * s)), fma(x0, s, x1 * c).
    if constexpr (NPL == 2) {  // the pair (lane, lane + 64) is this lane's own two values
      const float x0 = x[0], x1 = x[1];
      x[0] = fma_(x0, cv, -(x1 * sv));
      x[1] = fma_(x0, sv, x1 * cv);
    } else {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      sh[lane] = x[0];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      const float other = sh[lane ^ 32];
      const float cp = __shfl(cv, lane & 31), sp = __shfl(sv, lane & 31);  // the pair's angle (lane i < 32 loaded it)
      x[0] = lane < 32 ? fma_(x[0], cp, -(other * sp)) : fma_(other, sp, x[0] * cp);
    }
    if constexpr (role == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
      for (int u = 0; u < NPL; ++u) qs[lane + 64 * u] = x[u];
      return;
    }
  }
  // quantize_i8 (quant.cpp:134-140) of the key (after norm and RoPE) or the raw value.
  float amax = 0.0f;
#pragma unroll
  for (int u = 0; u < NPL; ++u) amax = fmaxf(amax, fabsf(x[u]));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  const int64_t crow = (sq * f.KV + g) * f.n_ctx + jo;
  int8_t* dst = (role == 1 ? f.kv.k : f.kv.v) + crow * D;
  int8_t* own = role == 1 ? own_k : own_v;
#pragma unroll
  for (int u = 0; u < NPL; ++u) {
    const int i = lane + 64 * u;
    const int8_t qv = (int8_t)(int)__builtin_rintf(x[u] * id);
    const int at = role == 1 ? kv_perm(i, DC) : i;
    own[at] = qv;
    if (writer) dst[at] = qv;
  }
  if (lane == 0) {
    own_sc[role - 1] = d;
    if (writer) (role == 1 ? f.kv.ks : f.kv.vs)[crow] = d;
  }
}

// The body of k_attention_dec for workgroup blk, NT threads. COH (inside the persistent decode kernel): the raw q/k/v
// rows are read and the BlockQ8 output rows written with device-coherent accesses, and there is no fp32 output; wait()
// is called by the three fuse waves before they read the raw rows (the K and V loads of the cached keys are already
// in flight).
template <int D, int NSLOT, bool FUSE, bool COH, int NT = kDecThreads, typename Wait>
__device__ __forceinline__ void attend_dec(int blk, const float* __restrict__ q, int64_t q_stride,
                                           float* __restrict__ out, int64_t out_stride, int G, float scale,
                                           const AttnAddr& a, const int32_t* __restrict__ seqs,
                                           const int32_t* __restrict__ n_keys, int n, int H, const DecFuse& f,
                                           BlockQ8* __restrict__ xq, int64_t xq_stride, const Wait& wait) {
  constexpr int DC = D / 16;
  const int tid = threadIdx.x;
  int t, h;
  if ((n * H) % 8 == 0) {
    const int pair = (int)((unsigned)blk % 8) * (n * H / 8) + (int)((unsigned)blk / 8);
    const int grp = pair / (n * G), rem = pair % (n * G);
    t = rem / G;
    h = grp * G + rem % G;
  } else {
    t = blk / H;
    h = blk % H;
  }
  const int g = h / G;
  const int nk = n_keys[t];
  const int nk_pad = attn_keys_pad(nk);
  const int vstride = dec_vstride(nk_pad);
  extern __shared__ int4 smem4[];
  uint8_t* vt = reinterpret_cast<uint8_t*>(smem4);          // [D][vstride] int8: V transposed
  float* sc = reinterpret_cast<float*>(vt + D * vstride);   // nk_pad: scores, then e^(s - max)
  float* pv = sc + nk_pad;                                  // nk_pad: v scales, then e * v-scale, 0 past nk
  float* qs = pv + nk_pad;                                  // D
  __shared__ float red[NT / 64];
  __shared__ float inv_s;
  const int64_t sq = seqs[t];
  const int8_t* kb = a.k + sq * a.k_seq + g * a.k_head;
  const int8_t* vb = a.v + sq * a.k_seq + g * a.k_head;
  const char* ksb = a.ks + sq * a.s_seq + g * a.s_head;
  const char* vsb = a.vs + sq * a.s_seq + g * a.s_head;
  float qv = 0.0f;
  if constexpr (!FUSE) qv = tid < D ? q[t * q_stride + (int64_t)h * D + tid] : 0.0f;
  // FUSE: this token's own K and V rows (key jo), made here from the raw projections.
  __shared__ __align__(16) int8_t own_k[FUSE ? D : 16], own_v[FUSE ? D : 16];
  __shared__ float own_sc[2];
  const int jo = FUSE ? f.kv_row[t] : -1;

  // Scores (kernels_avx512.cpp:234-244): LPK = D/16 lanes per key, each with one 16-byte load of the permuted row,
  // i.e. CPL = 16/LPK of the reference's lane chains (chains CPL m .. CPL m + CPL - 1 in lane m). KB keys per group
  // and round (512 keys per round); the round's key and value scales take one load per lane (lane b < KB: key scale
  // of key b, lane KB + b: its value scale). Loads are never predicated: past the last key they re-read it, unused.
  constexpr int LPK = D / 16, CPL = 16 / LPK, NGR = NT / LPK, KB = LPK / 2;
  const int gl = tid % LPK, grp = tid / LPK;
  struct Round {
    v4i k[KB];
    float sv;
  };
  auto fetch = [&](Round& R, int r) {
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      const int j = min((r * KB + b) * NGR + grp, nk - 1);
      R.k[b] = *reinterpret_cast<const v4i*>(kb + (int64_t)j * a.k_row + 16 * gl);
    }
    const int js = min((r * KB + gl % KB) * NGR + grp, nk - 1);
    R.sv = *reinterpret_cast<const float*>((gl < KB ? ksb : vsb) + (int64_t)js * a.s_row);
  };
  const int rounds = (nk + NGR * KB - 1) / (NGR * KB);
  // The first two rounds' K rows are issued here, before anything waits: a load issued later would be waited for
  // together with everything issued before it (the wait counts are in order).
  Round RA, RB;
  fetch(RA, 0);
  fetch(RB, min(1, rounds - 1));

  // V staging: task k = (quad kq = k / (D/16) of 4 keys, segment sg = k % (D/16) of 16 values), NSLOT tasks per
  // staging thread (st = tid less the fuse roles' waves). Past the last task the loads re-read it (the same rows:
  // no extra lines), unused.
  constexpr int SEG = D / 16, NST = dec_stagers(FUSE, NT);
  const int ntask = ((nk + 3) / 4) * SEG;
  const int st = tid - (NT - NST);
  v4i vr[NSLOT][4];
  if (st >= 0) {
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
      const int tk = min(st + NST * i, ntask - 1);
      const int sg = tk % SEG, kq = tk / SEG;
#pragma unroll
      for (int x = 0; x < 4; ++x)
        vr[i][x] = *reinterpret_cast<const v4i*>(vb + (int64_t)min(4 * kq + x, nk - 1) * a.k_row + 16 * sg);
    }
  }

  __shared__ float kscr[FUSE ? D : 1];  // the key role's rmsnorm scratch
  if constexpr (FUSE) {
    // One wave per role; the staging waves transpose V meanwhile (below).
    const int wv = tid >> 6;
    float* ksc = kscr;
    if (wv < 3) wait();
    if (wv == 0)
      fuse_qkv<D, 0, COH>(f, t, h, g, tid & 63, H, (int64_t)seqs[t], jo, h % G == 0, qs, ksc, own_k, own_v, own_sc);
    else if (wv == 1)
      fuse_qkv<D, 1, COH>(f, t, h, g, tid & 63, H, (int64_t)seqs[t], jo, h % G == 0, qs, ksc, own_k, own_v, own_sc);
    else if (wv == 2)
      fuse_qkv<D, 2, COH>(f, t, h, g, tid & 63, H, (int64_t)seqs[t], jo, h % G == 0, qs, ksc, own_k, own_v, own_sc);
  } else {
    if (tid < D) qs[tid] = qv;
  }

  // V: 4 x 4 byte transposes into the [value][key] rows; rows of segment sg hold their 16-key blocks XOR sg % 8.
  // The token's own key (FUSE) is written over after the barrier, once its row exists.
  if (st >= 0) {
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
      const int tk = st + NST * i;
      const int sg = tk % SEG, kq = tk / SEG;
      if (tk < ntask) {
        const int col = 16 * ((kq >> 2) ^ (sg & 7)) + 4 * (kq & 3);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t A = (uint32_t)vr[i][0][u], B = (uint32_t)vr[i][1][u];
          const uint32_t C = (uint32_t)vr[i][2][u], E = (uint32_t)vr[i][3][u];
          const uint32_t t0 = __builtin_amdgcn_perm(B, A, 0x05010400u), t1 = __builtin_amdgcn_perm(B, A, 0x07030602u);
          const uint32_t t2 = __builtin_amdgcn_perm(E, C, 0x05010400u), t3 = __builtin_amdgcn_perm(E, C, 0x07030602u);
          uint8_t* row = vt + (16 * sg + 4 * u) * vstride + col;
          *reinterpret_cast<uint32_t*>(row) = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
          *reinterpret_cast<uint32_t*>(row + vstride) = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
          *reinterpret_cast<uint32_t*>(row + 2 * vstride) = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
          *reinterpret_cast<uint32_t*>(row + 3 * vstride) = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
        }
      }
    }
  }
  lds_barrier();
  if (FUSE && tid < D) {  // value tid of the token's own key jo
    const int kq = jo >> 2;
    vt[tid * vstride + 16 * ((kq >> 2) ^ ((tid >> 4) & 7)) + 4 * (kq & 3) + (jo & 3)] = (uint8_t)own_v[tid];
  }
  float qr[CPL][DC];  // qr[k][c] = q[16 c + CPL gl + k]
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int c = 0; c < DC; ++c) qr[k][c] = qs[16 * c + CPL * gl + k];
  auto score = [&](const Round& R, int r) {
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      const int j = (r * KB + b) * NGR + grp;
      if (j < nk) {  // uniform over the LPK lanes of the key
        v4i kw = R.k[b];
        if (FUSE && j == jo) kw = *reinterpret_cast<const v4i*>(own_k + 16 * gl);
        float sl[CPL];
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
#pragma unroll
          for (int c = 0; c < DC; ++c) {
            const int e = k * DC + c;  // byte of chain CPL gl + k, value c
            const float kf = (float)(int8_t)((uint32_t)kw[e >> 2] >> (8 * (e & 3)));
            sl[k] = c == 0 ? qr[k][0] * kf : fma_(qr[k][c], kf, sl[k]);
          }
        }
        // The halving tree of _mm512_reduce_add_ps over the 16 chains: pairs 8, 4, 2, 1 chains apart, across lanes
        // while the distance spans whole lanes, then within lane 0.
#pragma unroll
        for (int k = 0; k < CPL; ++k) sl[k] = sl[k] + shl16<8 / CPL>(sl[k]);
#pragma unroll
        for (int k = 0; k < CPL; ++k) sl[k] = sl[k] + shl16<(4 / CPL > 0 ? 4 / CPL : 1)>(sl[k]);
        float tot;
        if constexpr (CPL == 2) {
#pragma unroll
          for (int k = 0; k < 2; ++k) sl[k] = sl[k] + shl16<1>(sl[k]);
          tot = sl[0] + sl[1];
        } else {  // CPL == 4: the second step above crossed one lane; the last two are in-lane
          tot = (sl[0] + sl[2]) + (sl[1] + sl[3]);
        }
        float ksv = shl16_k(R.sv, b), vsv = shl16_k(R.sv, KB + b);  // valid in lane 0 of the key
        if (FUSE && j == jo) ksv = own_sc[0], vsv = own_sc[1];
        if (gl == 0) {
          sc[j] = tot * (ksv * scale);
          pv[j] = vsv;
        }
      }
    }
  };
  if constexpr (NT == kDecThreads) {
    score(RA, 0);
    if (rounds > 1) score(RB, 1);
    for (int r = 2; r < rounds; ++r) {  // more than 1024 keys (D = 128)
      fetch(RA, r);
      score(RA, r);
    }
  } else {
    // Fewer threads, more rounds: each register set is refilled two rounds ahead as soon as it has been scored
    // (unpredicated: past the last round the loads re-read the last key, and score skips keys past the end).
    score(RA, 0);
    fetch(RA, 2);
    score(RB, 1);
    fetch(RB, 3);
    for (int r = 2; r < rounds; r += 2) {
      score(RA, r);
      fetch(RA, r + 2);
      score(RB, r + 1);
      fetch(RB, r + 3);
    }
  }
  lds_barrier();

  // softmax_inplace (kernels_avx512.cpp:205-226).
  float m = -INFINITY;
  for (int j = tid; j < nk; j += NT) m = fmaxf(m, sc[j]);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  lds_barrier();
  float mx = red[0];
  for (int i = 1; i < NT / 64; ++i) mx = fmaxf(mx, red[i]);
  for (int j = tid; j < nk_pad; j += NT) {
    if (j < nk) {
      const float e = exp512(sc[j] - mx);
      sc[j] = e;
      pv[j] = e * pv[j];
    } else {
      pv[j] = 0.0f;
    }
  }
  lds_barrier();

  // P.V (kernels_avx512.cpp:247-265).
  float acc = 0.0f;
  if (tid < D) {
    __builtin_amdgcn_s_setprio(3);
    const uint8_t* vrow = vt + tid * vstride;
    const int swz = (tid >> 4) & 7;
    const float* pc = pv + (tid & 15);
    auto ld = [&](v4i& v, float& p, int jj) {
      const int j = min(jj, nk_pad - 16);
      v = *reinterpret_cast<const v4i*>(vrow + 16 * ((j >> 4) ^ swz));
      p = pc[j];
    };
    // One 16-key group: the chain over the group's converted values fc (coefficients p), with the converts of the
    // next group's raw bytes w into fn issued in the fmas' latency, one per step.
    auto group = [&](const float (&fc)[16], float p, const v4i& w, float (&fn)[16]) {
      acc = fma8_bcast16_cvt<0>(p, fc, acc, (uint32_t)w[0], (uint32_t)w[1], fn);
      acc = fma8_bcast16_cvt<8>(p, fc, acc, (uint32_t)w[2], (uint32_t)w[3], fn);
    };
    // Group g's values are converted during group g - 1's chain; its raw bytes are read during group g - 2's.
    v4i ra, rb;
    float pa, pb, qa, qb;
    float fa[16], fb[16];
    ld(ra, pa, 0);
    ld(rb, pb, 16);
    {
      const uint32_t w[4] = {(uint32_t)ra[0], (uint32_t)ra[1], (uint32_t)ra[2], (uint32_t)ra[3]};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        fa[4 * k] = i8_to_f32<0>(w[k]);
        fa[4 * k + 1] = i8_to_f32<1>(w[k]);
        fa[4 * k + 2] = i8_to_f32<2>(w[k]);
        fa[4 * k + 3] = i8_to_f32<3>(w[k]);
      }
    }
    for (int jj = 0; jj < nk_pad; jj += 32) {
      ld(ra, qa, jj + 32);
      __builtin_amdgcn_sched_barrier(0);
      group(fa, pa, rb, fb);
      if (jj + 16 >= nk_pad) break;
      ld(rb, qb, jj + 48);
      __builtin_amdgcn_sched_barrier(0);
      group(fb, pb, ra, fa);
      pa = qa;
      pb = qb;
    }
  } else if (tid >= NT - 16) {
    const int l = tid - (NT - 16);
    float s = 0.0f;
    for (int j = l; j < nk; j += 16) s = s + sc[j];
    s = reduce16_lanes(s);
    if (l == 0) inv_s = 1.0f / s;
  }
  lds_barrier();
  if (tid < D) {
    if constexpr (COH)
      put_q8_coh(xq + t * xq_stride + (h * D) / 32, tid, acc * inv_s);
    else
      put_out(out + t * out_stride + (int64_t)h * D, xq, t * xq_stride, h * D, tid, acc * inv_s);
  }
}

template <int D, int NSLOT, bool FUSE>
__global__ __launch_bounds__(kDecThreads) void k_attention_dec(const float* __restrict__ q, int64_t q_stride,
                                                               float* __restrict__ out, int64_t out_stride, int G,
                                                               float scale, AttnAddr a,
                                                               const int32_t* __restrict__ seqs,
                                                               const int32_t* __restrict__ n_keys, int n, int H,
                                                               DecFuse f, BlockQ8* __restrict__ xq,
                                                               int64_t xq_stride) {
  attend_dec<D, NSLOT, FUSE, false>((int)blockIdx.x, q, q_stride, out, out_stride, G, scale, a, seqs, n_keys, n, H, f,
                                    xq, xq_stride, [] {});
}

}  // namespace
}  // namespace mk
