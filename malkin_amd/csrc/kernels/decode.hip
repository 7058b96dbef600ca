// Persistent decode kernel: the layers [l0, l1) of a one-token decode step (model.cpp:355-417 at n = 1) in one
// launch, bit-identical to the per-layer launches it replaces (k_gemv's Q8_0 arithmetic with its rmsnorm, quantize,
// residual and silu*up prologues / epilogues, and k_attention_dec's body).
//
// A decode layer is five dependent steps: q|k|v GEMV, attention, attn_output GEMV, gate|up GEMV, down GEMV. As one
// kernel each, every step pays a kernel boundary (ramp and tail) and its weight stream starts only after the previous
// kernel has drained. Here one 512-thread workgroup per CU stays resident over all the layers and the steps hand off
// through device-coherent counters. Before a GEMV sub-unit waits for a step's input it already has the loads of its
// first two weight chunks of that step in flight, and the attention workgroups have their cached K and V rows in
// flight, so each hand-off overlaps with weight traffic, and the attn_output weights stream in while attention runs
// on H of the CUs.
//
// Workgroup = two GEMV sub-units of 256 threads (wave 0: the sequential row chains; waves 1-3: the exact int dots
// and per-block terms of R = 8-row packed groups, 48 blocks per chunk, two chunks of weights in registers), or, in
// the attention step, one query head. A GEMV step's row groups are dealt to sub-units (w - wlo) + nw * sub of the
// nw workgroups taking part, so every workgroup gets an equal share first.
//
// Hand-off: a step's outputs are written with coherent stores (sc1: past the per-XCD caches); each workgroup then
// (after s_waitcnt) adds one to its XCD's counter for the step (8 counters per step, 128 bytes apart); a reader polls
// the 8 counters until each holds the workgroup count of its XCD. Every workgroup signals every step, immediately
// where it has no work in it. An activation buffer is overwritten only by a step that waited, directly or through
// another step, for a step that every reader of its previous contents signalled after reading, so one buffer per
// activation suffices. Every wait is bounded: past spin_max polls the workgroup sets the error word and goes on, and
// later waits end at once; the host checks the word after the launch. The last workgroup to leave resets the
// counters for the next launch.
#include <algorithm>
#include <cmath>

#include "attn_dec.h"
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kDT = 512;                  // threads per workgroup (two waves per SIMD: 256 VGPRs each)
constexpr int kSubs = kDT / 256;          // GEMV sub-units per workgroup
constexpr int kR = 8;                     // rows per packed group
constexpr int kChunk = 48;                // blocks per chunk (k_gemv's measured best at one token)
constexpr int kWk = 192;                  // worker lanes per sub-unit
constexpr int kP = kChunk * kR / kWk;     // (row, block) pairs per worker lane and chunk
constexpr int kG = 8;                     // blocks per chain step group
constexpr int kLane = (kChunk + kG) * 2 + 4;  // term floats per row: the chunk's (dot, scale) pairs + read-ahead + pad
constexpr int kSlot = kR * kLane;
constexpr int kSteps = 5;                 // per layer
constexpr int kCtr = 32;                  // words per counter (128 bytes)
constexpr int kMaxSlots = 8;              // V staging tasks per attention thread (keys up to LDS capacity)
static_assert(kChunk * kR % kWk == 0 && kChunk % kG == 0, "chunk shape");

struct Raw8 {
  uint4 a, b;
  uint32_t s;
};

// A pointer read from the argument block points to global memory: saying so lets loads and stores through it (and
// through pointers derived from it) use global instructions with a scalar base instead of flat ones.
template <typename T>
__device__ __forceinline__ T* glob(T* p) {
  return (T*)((__attribute__((address_space(1))) T*)p);
}


// A GEMV step over one packed Q8_0 weight (rows x nu blocks), taken by workgroups [wlo, wlo + nw).
struct Gs {
  const uint8_t* W;
  int rows, nu, nc, ng;
  int wlo, nw;
  __device__ int su_of(int w, int sub) const { return w >= wlo && w < wlo + nw ? (w - wlo) + nw * sub : -1; }
  __device__ int nq_of(int su) const {
    return su < 0 || su >= ng ? 0 : ((ng - 1 - su) / (kSubs * nw) + 1) * nc;
  }
};

__device__ __forceinline__ Gs make_gs(const void* W, int rows, int cols, int wlo, int nw) {
  Gs g;
  g.W = static_cast<const uint8_t*>(W);
  g.rows = rows;
  g.nu = cols / 32;
  g.nc = (g.nu + kChunk - 1) / kChunk;
  g.ng = rows / kR;
  g.wlo = wlo;
  g.nw = nw;
  return g;
}

// Chunk p of sub-unit su's share of step S: its pairs (row f % 8, block f / 8 of the chunk) for f = wi + 192 k.
// Blocks past the row's end re-read its last block (unused).
// Offsets as in PackedQ8_0 (layout.h), in 32 bits: a packed weight here is far below 4 GB.
__device__ __forceinline__ void load_chunk(Raw8 (&r)[kP], const Gs& S, int su, int p, int wi) {
  const uint32_t g = (uint32_t)(su + (p / S.nc) * (kSubs * S.nw));
  const int cc = p % S.nc;
  const uint8_t* W = glob(S.W);
  const uint32_t scales0 = (uint32_t)S.ng * (uint32_t)S.nu * 256u;
#pragma unroll
  for (int k = 0; k < kP; ++k) {
    const int f = wi + k * kWk;
    const uint32_t gu = g * (uint32_t)S.nu + (uint32_t)min(cc * kChunk + f / kR, S.nu - 1);
    const uint32_t q = gu * 256u + (uint32_t)(f % kR) * 16u;
    r[k].a = *reinterpret_cast<const uint4*>(W + q);
    r[k].b = *reinterpret_cast<const uint4*>(W + q + 128u);
    r[k].s = *reinterpret_cast<const uint16_t*>(W + scales0 + gu * 16u + (uint32_t)(f % kR) * 2u);
  }
}

// Position p of a sub-unit's load stream in step S (nq chunks): chunk p of S, then the first two chunks of the next
// GEMV step N (nn chunks there, as sub-unit sun), or where there are none a re-read of S's last chunk. Every path
// issues the same loads, so the compiler's wait counts stay exact.
__device__ __forceinline__ void load_pos(Raw8 (&r)[kP], const Gs& S, int su, int nq, const Gs& N, int sun, int nn,
                                         int p, int wi) {
  if (p < nq)
    load_chunk(r, S, su, p, wi);
  else if (nn > 0)
    load_chunk(r, N, sun, p - nq, wi);
  else
    load_chunk(r, S, su, nq - 1, wi);
}

// The per-model constants of the kernel, in device memory (written once per model): they are read where used through
// an opaque pointer (opaque below) rather than held in registers across the kernel.
struct DecodeArgs {
  const DecodeLayer* layers;
  int E, H, KV, F;
  int n_ctx, n_seq;
  float eps, scale;
  int8_t* k8;
  int8_t* v8;
  float* ks;
  float* vs;
  float* x;         // [E] residual stream
  float* qkv;       // [(H + 2 KV) D]
  BlockQ8* att;     // [H D / 32]
  float* h;         // [F]
  const float* cos_t;
  const float* sin_t;
  const int32_t* rpos;
  const int32_t* seq;
  const int32_t* kv_row;
  const int32_t* n_keys;
  unsigned* sync;   // [steps][8] counters, then the exit counter and the error word
  unsigned spin_max;
};

// 16 coherent bytes at byte offset off of the array at base (wave-uniform base; sc1 buffer load).
__device__ __forceinline__ float4 ld_coh16(const void* base, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7FFFFFFF,
                                                                     0x00020000);
  typedef int v4i_t __attribute__((ext_vector_type(4)));
  const v4i_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16);
  return make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
}

// A copy of p the compiler cannot see through: a field read through it is loaded where it is used (a scalar load,
// a scalar-cache hit) instead of being hoisted and kept in registers over the whole kernel.
// The argument block is constant during a launch: reads through the constant address space are scalar loads.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* opaque(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  asm volatile("" : "+s"(lo), "+s"(hi));
  return (const __attribute__((address_space(4))) T*)((uint64_t)hi << 32 | lo);
}


// Counters of step sid (8, one per XCD), the exit counter and the error word; n_steps = (l1 - l0) * kSteps.
__device__ __forceinline__ unsigned* step_ctr(const DecodeArgs* P, int sid, int x) {
  return glob(opaque(P)->sync) + ((size_t)sid * 8 + x) * kCtr;
}
__device__ __forceinline__ unsigned* exit_ctr(const DecodeArgs* P, int n_steps) {
  return glob(opaque(P)->sync) + (size_t)n_steps * 8 * kCtr;
}
__device__ __forceinline__ unsigned* err_word(const DecodeArgs* P, int n_steps) {
  return exit_ctr(P, n_steps) + kCtr;
}

// One wave waits until every workgroup has signalled step sid (bounded; see the file comment).
__device__ __forceinline__ void poll_step(const DecodeArgs* P, int n_steps, int sid) {
  if (sid < 0) return;
  const int lane = threadIdx.x & 63;
  const unsigned G = gridDim.x;
  const unsigned per = G / 8 + ((unsigned)(lane & 7) < G % 8 ? 1u : 0u);
  const unsigned* c = step_ctr(P, sid, lane & 7);
  unsigned* err = err_word(P, n_steps);
  const unsigned spin_max = opaque(P)->spin_max;
  for (unsigned it = 0; it < spin_max; ++it) {
    const bool ok = lane >= 8 || ld_coh_u32(c) >= per;
    if (__all(ok)) return;
    if ((it & 63) == 63 && ld_coh_u32(err) != 0) return;
  }
  if (lane == 0) st_coh_u32(err, 1u);
}

// The whole workgroup waits for step sid (wave 0 polls).
__device__ __forceinline__ void wait_step(const DecodeArgs* P, int n_steps, int sid) {
  if ((threadIdx.x >> 6) == 0) poll_step(P, n_steps, sid);
  lds_barrier();
}

// Signals step sid once every wave that stored outputs has waited for its stores (s_waitcnt before the call).
__device__ __forceinline__ void signal_step(const DecodeArgs* P, int sid) {
  lds_barrier();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(step_ctr(P, sid, blockIdx.x & 7), 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
}

enum : int { kInNorm = 0, kInQ8 = 1, kInF32 = 2 };
enum : int { kOutStore = 0, kOutAcc = 1, kOutSilu = 2 };

// LDS of a GEMV step: the input's BlockQ8 row (xs), four sub-units' double-buffered term slots, and an fp32 staging
// area (the rmsnorm's transposed row, or an fp32 input row read with coalesced loads before it is quantized).
struct GemvLds {
  int* xs;
  float* res;
  float* tr;
};
__host__ __device__ constexpr size_t gemv_stage_floats(int max_cols, int E) {
  return (size_t)16 * sumsq_tstride(E / 16) > (size_t)max_cols ? (size_t)16 * sumsq_tstride(E / 16) : (size_t)max_cols;
}
__host__ __device__ constexpr size_t gemv_xs_bytes(int max_cols) { return ((size_t)(max_cols / 32) * 40 + 15) & ~15; }
__host__ __device__ constexpr size_t gemv_lds_bytes(int max_cols, int E) {
  return gemv_xs_bytes(max_cols) + (size_t)kSubs * 2 * kSlot * 4 + gemv_stage_floats(max_cols, E) * 4;
}
__device__ __forceinline__ GemvLds gemv_lds(int max_cols) {
  extern __shared__ int smem[];
  GemvLds l;
  l.xs = smem;
  l.res = reinterpret_cast<float*>(smem + gemv_xs_bytes(max_cols) / 4);
  l.tr = l.res + kSubs * 2 * kSlot;
  return l;
}

// The loader threads' share of n4 16-byte pieces of the coherent array in: batches of kLB pieces per thread, all of a
// batch's loads issued before the first is used (one memory round trip per batch), then use(i4, piece).
constexpr int kLB = 8;
template <typename F>
__device__ __forceinline__ void load_pieces(const void* in, int n4, int li, int loaders, F&& use) {
  for (int base = 0; base < n4; base += kLB * loaders) {
    float4 v[kLB];
#pragma unroll
    for (int k = 0; k < kLB; ++k) v[k] = ld_coh16(in, 16u * (uint32_t)min(base + li + k * loaders, n4 - 1));
#pragma unroll
    for (int k = 0; k < kLB; ++k)
      if (base + li + k * loaders < n4) use(base + li + k * loaders, v[k]);
  }
}

// The input row of a GEMV step into xs as BlockQ8, by the whole workgroup (ends with a barrier):
//   kInNorm  rmsnorm(x) * nw, quantized (model.cpp:46-49, 362-364, 403-405; k_gemv's kProNorm arithmetic);
//   kInQ8    BlockQ8 blocks as they are;
//   kInF32   fp32 values, quantized (quantize_acts; k_gemv's kProF32).
// Its global loads are made by the chain waves (wave 0 of each sub-unit) alone: the workers have the step's first
// weight chunks in flight, and a wave's loads complete in issue order, so a load of theirs would wait for those.
template <int IN>
__device__ __forceinline__ void gemv_input(const GemvLds& l, const void* in, const float* nw, float eps, int cols) {
  const int tid = threadIdx.x, wv = tid >> 6;
  const bool loader = (wv & 3) == 0;
  const int li = (wv >> 2) * 64 + (tid & 63);  // loader index
  constexpr int kLoaders = kSubs * 64;
  const int nq8 = cols / 32;
  BlockQ8* xb = reinterpret_cast<BlockQ8*>(l.xs);
  if constexpr (IN == kInNorm) {
    const int per = cols / 16, tstride = sumsq_tstride(per), padded = sumsq_padded(per);
    // tr[c][j] = x[16 j + c] (the 16 lane chains' values in order), zero past the row.
    if (loader)
      load_pieces(in, cols / 4, li, kLoaders, [&](int i4, const float4& v) {
        const int i = 4 * i4, j = i >> 4, c = i & 15;
        l.tr[c * tstride + j] = v.x;
        l.tr[(c + 1) * tstride + j] = v.y;
        l.tr[(c + 2) * tstride + j] = v.z;
        l.tr[(c + 3) * tstride + j] = v.w;
      });
    for (int i = cols + tid; i < 16 * padded; i += kDT) l.tr[(i & 15) * tstride + (i >> 4)] = 0.0f;
    __shared__ float scale_s;
    lds_barrier();
    if (tid < 16) {
      float acc = sumsq_lane_chain(l.tr + tid * tstride, per);
      acc = reduce16_lanes(acc);
      if (tid == 0) scale_s = 1.0f / sqrtf(acc / (float)cols + eps);
    }
    lds_barrier();
    const float sc = scale_s;
    for (int c16 = tid; c16 < per; c16 += kDT) {
      float wv[16], yv[16];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 w4 = reinterpret_cast<const float4*>(nw + 16 * c16)[k];
        wv[4 * k] = w4.x, wv[4 * k + 1] = w4.y, wv[4 * k + 2] = w4.z, wv[4 * k + 3] = w4.w;
      }
#pragma unroll
      for (int c = 0; c < 16; ++c) yv[c] = l.tr[c * tstride + c16] * sc * wv[c];
      quantize_half_block(yv, c16 & 1, true, xb + c16 / 2);
    }
  } else if constexpr (IN == kInQ8) {
    // nq8 * 40 bytes: whole 16-byte pieces (nq8 even), and the odd one's last 8 bytes by a 4-byte pair.
    if (loader) {
      load_pieces(in, nq8 * 10 / 4, li, kLoaders,
                  [&](int i4, const float4& v) { reinterpret_cast<float4*>(l.xs)[i4] = v; });
      for (int i = (nq8 * 10 / 4) * 4 + li; i < nq8 * 10; i += kLoaders)
        l.xs[i] = (int)ld_coh_u32(static_cast<const uint32_t*>(in) + i);
    }
  } else {
    // Coalesced coherent loads into the staging area, then 16 consecutive values per lane from LDS.
    if (loader)
      load_pieces(in, cols / 4, li, kLoaders,
                  [&](int i4, const float4& v) { reinterpret_cast<float4*>(l.tr)[i4] = v; });
    lds_barrier();
    for (int c16 = tid; c16 < 2 * nq8; c16 += kDT) {
      float v[16];
      const float4* p4 = reinterpret_cast<const float4*>(l.tr + 16 * c16);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 a = p4[k];
        v[4 * k] = a.x, v[4 * k + 1] = a.y, v[4 * k + 2] = a.z, v[4 * k + 3] = a.w;
      }
      quantize_half_block(v, c16 & 1, true, xb + c16 / 2);
    }
  }
  lds_barrier();
}

// Worker terms of chunk c (blocks c * 48 ...): per pair the exact int dot and dw * dx, zero past the row.
__device__ __forceinline__ void gemv_dots(const Raw8 (&raw)[kP], float* slot, const int* xs, int c, int nu, int wi) {
#pragma unroll
  for (int k = 0; k < kP; ++k) {
    const int f = wi + k * kWk;
    const int ul = f / kR, r = f % kR;
    const int u = c * kChunk + ul;
    const bool live = u < nu;
    const float dw = half_to_float((uint16_t)raw[k].s);
    const int* xq = xs + (live ? u : 0) * 10;
    *reinterpret_cast<float2*>(slot + r * kLane + ul * 2) =
        live ? make_float2((float)dot8(raw[k].a, raw[k].b, xq), dw * xd(xq)) : make_float2(0.0f, 0.0f);
  }
}

// One GEMV step of this workgroup (step id sid, its input step sid - 1). ra / rb are the sub-unit's register sets
// and pf says which holds chunk 0 of this step (0: ra, 1: rb, -1: not loaded). N: the sub-unit's next GEMV step
// (n_ok false: none), whose first two chunks the loop loads after this step's last. Returns pf for N.
template <int IN, int OUT>
__device__ __forceinline__ int gemv_step(const DecodeArgs* P, int n_steps, int sid, const Gs& S, const Gs& N,
                                         bool n_ok, Raw8 (&ra)[kP], Raw8 (&rb)[kP], int pf, const void* in,
                                         const float* nw, int cols, int max_cols, float* y) {
  const int tid = threadIdx.x, w = blockIdx.x, wv = tid >> 6, sub = wv >> 2;
  const bool worker = (wv & 3) != 0;
  const int wi = (tid & 255) - 64;
  const int su = S.su_of(w, sub), nq = S.nq_of(su);
  const int nq_wg = S.nq_of(S.su_of(w, 0));
  const int sun = n_ok ? N.su_of(w, sub) : -1, nn = n_ok ? N.nq_of(sun) : 0;
  const int pf_next = nn > 0 ? (nq > 0 ? (nq & 1) : 0) : -1;
  if (worker) {
    if (nq > 0) {
      if (pf < 0) {
        load_pos(ra, S, su, nq, N, sun, nn, 0, wi);
        load_pos(rb, S, su, nq, N, sun, nn, 1, wi);
      } else if (pf == 1) {
        const Raw8 t0 = ra[0], t1 = ra[1];
        ra[0] = rb[0], ra[1] = rb[1];
        rb[0] = t0, rb[1] = t1;
      }
    } else if (nn > 0) {
      load_chunk(ra, N, sun, 0, wi);
      load_chunk(rb, N, sun, 1, wi);
    }
  }
  if (nq_wg == 0) {
    signal_step(P, sid);
    return pf_next;
  }
  wait_step(P, n_steps, sid - 1);
  const GemvLds l = gemv_lds(max_cols);
  gemv_input<IN>(l, in, nw, opaque(P)->eps, cols);

  float* slots = l.res + sub * 2 * kSlot;
  const int cr = tid & 255;
  const bool chain_lane = !worker && cr < kR && nq > 0;
  float acc = 0.0f, xr = 0.0f;
  // Chain lane cr runs row cr of the chunk's group over the chunk's blocks in order (k_gemv's chain, Q8_0, one token).
  auto chain = [&](int q) {
    if (!chain_lane) return;
    const int c = q % S.nc;
    const int g = su + (q / S.nc) * (kSubs * S.nw);
    if (OUT == kOutAcc && c == 0) xr = ld_coh(y + g * kR + cr);  // the residual, read early
    const int cn = min(kChunk, S.nu - c * kChunk);
    const float4* e = reinterpret_cast<const float4*>(slots + (q & 1) * kSlot + cr * kLane);
    float4 T0[4], T1[4];
    auto fetch = [&](float4(&T)[4], int ul0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) T[i] = e[ul0 / 2 + i];
    };
    auto step = [&](const float4(&T)[4]) {
      const float* v = reinterpret_cast<const float*>(T);
#pragma unroll
      for (int i = 0; i < kG; ++i) acc = fma_(v[2 * i], v[2 * i + 1], acc);
    };
    fetch(T0, 0);
    for (int ul0 = 0;;) {
      fetch(T1, ul0 + kG);
      __builtin_amdgcn_sched_barrier(0);
      step(T0);
      __builtin_amdgcn_sched_barrier(0);
      if ((ul0 += kG) >= cn) break;
      fetch(T0, ul0 + kG);
      __builtin_amdgcn_sched_barrier(0);
      step(T1);
      __builtin_amdgcn_sched_barrier(0);
      if ((ul0 += kG) >= cn) break;
    }
    if (c == S.nc - 1) {
      if constexpr (OUT == kOutSilu) {
        // Rows cr and cr + 4 of a group are gate and up of output 4 g + cr.
        const float up = __shfl_down(acc, 4, 8);
        if (cr < 4) {
          const float ex = exp512(0.0f - acc);
          st_coh(y + g * (kR / 2) + cr, (acc / (1.0f + ex)) * up);
        }
      } else if constexpr (OUT == kOutAcc) {
        st_coh(y + g * kR + cr, xr + acc);
      } else {
        st_coh(y + g * kR + cr, acc);
      }
      acc = 0.0f;
    }
  };

  if (!worker) __builtin_amdgcn_s_setprio(2);
  for (int q = 0; q < nq_wg; q += 2) {
    if (worker) {
      if (q < nq) {
        gemv_dots(ra, slots + (q & 1) * kSlot, l.xs, q % S.nc, S.nu, wi);
        load_pos(ra, S, su, nq, N, sun, nn, q + 2, wi);
      }
    } else if (q > 0 && q - 1 < nq) {
      chain(q - 1);
    }
    lds_barrier();
    if (q + 1 < nq_wg) {
      if (worker) {
        if (q + 1 < nq) {
          gemv_dots(rb, slots + ((q + 1) & 1) * kSlot, l.xs, (q + 1) % S.nc, S.nu, wi);
          load_pos(rb, S, su, nq, N, sun, nn, q + 3, wi);
        }
      } else if (q < nq) {
        chain(q);
      }
      lds_barrier();
    }
  }
  if (nq == nq_wg) chain(nq - 1);
  if (!worker) {
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's output stores have completed
  }
  signal_step(P, sid);
  return pf_next;
}

template <int D, int NSLOT>
__global__ __launch_bounds__(kDT) void k_decode_layers(const DecodeArgs* __restrict__ P, int l0, int l1) {
  const int w = blockIdx.x, tid = threadIdx.x;
  const int G = (int)gridDim.x;
  const int n_steps = (l1 - l0) * kSteps;
  Raw8 ra[kP], rb[kP];
  int pf = -1;
  for (int il = l0; il < l1; ++il) {
    const int s0 = (il - l0) * kSteps;
    const bool last = il + 1 == l1;
    const int E = opaque(P)->E, H = opaque(P)->H, KV = opaque(P)->KV, F = opaque(P)->F;
    const int QKV = (H + 2 * KV) * D, HD = H * D, max_cols = max(max(E, HD), F);
    const bool is_att = w < H;  // one attention workgroup per query head (one token)
    const DecodeLayer* L = glob(opaque(P)->layers) + il;

    // q|k|v = W_qkv . rmsnorm(x); the attention workgroups load nothing ahead across their attention step (they load
    // their attn_output chunks right after it).
    pf = gemv_step<kInNorm, kOutStore>(P, n_steps, s0, make_gs(glob(opaque(L)->qkv), QKV, E, 0, G),
                                       make_gs(glob(opaque(L)->wo), E, HD, 0, G), !is_att, ra, rb, pf,
                                       glob(opaque(P)->x), glob(opaque(L)->attn_norm), E, max_cols,
                                       glob(opaque(P)->qkv));

    // Attention: QK-norm, RoPE, the KV row write and attention of one query head; BlockQ8 output rows.
    if (is_att) {
      const auto* Q = opaque(P);
      const size_t lrow = (size_t)il * Q->n_seq * KV * Q->n_ctx;
      const KvLayer kv{glob(Q->k8) + lrow * D, glob(Q->v8) + lrow * D, glob(Q->ks) + lrow, glob(Q->vs) + lrow};
      const int64_t rows = Q->n_ctx;
      const AttnAddr a{kv.k,  kv.v, reinterpret_cast<const char*>(kv.ks), reinterpret_cast<const char*>(kv.vs),
                       (int64_t)KV * rows * D, rows * D, D, (int64_t)KV * rows * 4, rows * 4, 4, 1};
      const DecFuse f{glob(Q->qkv), 0, glob(opaque(L)->q_norm), glob(opaque(L)->k_norm), Q->eps, glob(Q->cos_t),
                      glob(Q->sin_t), glob(Q->rpos), glob(Q->kv_row), kv, Q->n_ctx, KV};
      attend_dec<D, NSLOT, true, true, kDT>(w, nullptr, 0, nullptr, 0, H / KV, Q->scale, a, glob(Q->seq),
                                            glob(Q->n_keys), 1, H, f, glob(Q->att), 0,
                                            [&] { poll_step(P, n_steps, s0); });
      __builtin_amdgcn_s_waitcnt(0);
      // Nothing was loaded ahead for the next GEMV step; clearing the register sets here also ends their lifetime
      // before the attention code (which needs the registers) on this path.
      ra[0] = ra[1] = rb[0] = rb[1] = Raw8{};
      pf = -1;
    }
    signal_step(P, s0 + 1);

    // x += W_o . att
    pf = gemv_step<kInQ8, kOutAcc>(P, n_steps, s0 + 2, make_gs(glob(opaque(L)->wo), E, HD, 0, G),
                                   make_gs(glob(opaque(L)->gate_up), 2 * F, E, 0, G), true, ra, rb, pf,
                                   glob(opaque(P)->att), nullptr, HD, max_cols, glob(opaque(P)->x));
    // h = silu(gate) * up of W_gate|up . rmsnorm(x)
    pf = gemv_step<kInNorm, kOutSilu>(P, n_steps, s0 + 3, make_gs(glob(opaque(L)->gate_up), 2 * F, E, 0, G),
                                      make_gs(glob(opaque(L)->down), E, F, 0, G), true, ra, rb, pf,
                                      glob(opaque(P)->x), glob(opaque(L)->ffn_norm), E, max_cols,
                                      glob(opaque(P)->h));
    // x += W_down . h; then the next layer's q|k|v
    const void* next_qkv = last ? glob(opaque(L)->qkv) : glob(opaque(L + 1)->qkv);
    pf = gemv_step<kInF32, kOutAcc>(P, n_steps, s0 + 4, make_gs(glob(opaque(L)->down), E, F, 0, G),
                                    make_gs(next_qkv, QKV, E, 0, G), !last, ra, rb, pf, glob(opaque(P)->h), nullptr,
                                    F, max_cols, glob(opaque(P)->x));
  }

  // The last workgroup to leave resets the counters (every workgroup has finished its waits by then, and its signals
  // have completed: s_waitcnt before the exit count).
  __builtin_amdgcn_s_waitcnt(0);
  if ((tid >> 6) == 0) {
    unsigned old = 0;
    if (tid == 0) old = __hip_atomic_fetch_add(exit_ctr(P, n_steps), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old == (unsigned)G - 1) {
      unsigned* sync = glob(opaque(P)->sync);
      for (int i = tid; i < n_steps * 8; i += 64) st_coh_u32(sync + (size_t)i * kCtr, 0u);
      if (tid == 0) st_coh_u32(exit_ctr(P, n_steps), 0u);
    }
  }
}

}  // namespace

size_t decode_sync_bytes(int n_layer) { return ((size_t)n_layer * kSteps * 8 + 2) * kCtr * sizeof(unsigned); }
size_t decode_error_word(int n_layer) { return ((size_t)n_layer * kSteps * 8 + 1) * kCtr; }

bool decode_layers_supported(const DecodeDims& d, int max_keys) {
  if (d.D != 128 || d.KV <= 0 || d.H % d.KV != 0 || d.H / d.KV > 16 || d.E % 32 != 0 || d.F % 32 != 0) return false;
  // Every sub-unit that takes part in a GEMV step has at least two chunks (the prefetch of the next step's first
  // two chunks relies on it): more than 48 blocks per row.
  if (d.E / 32 <= kChunk || (d.H * d.D) / 32 <= kChunk || d.F / 32 <= kChunk) return false;
  if (max_keys <= 0 || max_keys > d.n_ctx || !dec_fits(d.D, max_keys, kDT, kMaxSlots)) return false;
  const int max_cols = std::max(std::max(d.E, d.H * d.D), d.F);
  const size_t lds = std::max(gemv_lds_bytes(max_cols, d.E), dec_lds_bytes(d.D, attn_keys_pad(max_keys)));
  // The attention step takes H of the workgroups (one per CU).
  return lds <= 160 * 1024 - 1024 && device_cus() >= d.H;
}

size_t decode_args_bytes() { return sizeof(DecodeArgs); }

void decode_set_args(void* dev, const DecodeDims& d, const DecodeBufs& b) {
  DecodeArgs A{};
  A.layers = b.layers;
  A.E = d.E, A.H = d.H, A.KV = d.KV, A.F = d.F;
  A.n_ctx = d.n_ctx, A.n_seq = d.n_seq;
  A.eps = d.eps;
  A.scale = 1.0f / std::sqrt(static_cast<float>(d.D));  // model.cpp:208
  A.k8 = b.kv0.k, A.v8 = b.kv0.v, A.ks = b.kv0.ks, A.vs = b.kv0.vs;
  A.x = b.x, A.qkv = b.qkv, A.att = static_cast<BlockQ8*>(b.att), A.h = b.h;
  A.cos_t = b.cos_t, A.sin_t = b.sin_t, A.rpos = b.rpos, A.seq = b.seq, A.kv_row = b.kv_row, A.n_keys = b.n_keys;
  A.sync = b.sync;
  A.spin_max = b.spin_max;
  check(hipMemcpy(dev, &A, sizeof A, hipMemcpyHostToDevice), "hipMemcpy");
}

void decode_layers(hipStream_t s, const void* dev_args, const DecodeDims& d, int l0, int l1, int max_keys) {
  require(decode_layers_supported(d, max_keys), "decode_layers: unsupported shape");
  require(l0 >= 0 && l1 > l0, "decode_layers: bad layer range");
  const int max_cols = std::max(std::max(d.E, d.H * d.D), d.F);
  const size_t lds = std::max(gemv_lds_bytes(max_cols, d.E), dec_lds_bytes(d.D, attn_keys_pad(max_keys)));
  const int cus = device_cus();
  const DecodeArgs* P = static_cast<const DecodeArgs*>(dev_args);
  auto go = [&](auto kernel) {
    static bool attr = false;
    if (!attr) {
      check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024 - 1024),
            "hipFuncSetAttribute");
      attr = true;
    }
    int per_cu = 0;
    check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kDT, lds),
          "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    // Every workgroup waits for the others: the whole grid (one workgroup per CU) must be resident at once.
    require(per_cu >= 1, "decode_layers: the kernel does not fit on a CU");
    hipLaunchKernelGGL(kernel, dim3(cus), dim3(kDT), lds, s, P, l0, l1);
  };
  const int slots = dec_slots(d.D, max_keys, true, kDT);
  if (slots <= 2)
    go(k_decode_layers<128, 2>);
  else if (slots <= 4)
    go(k_decode_layers<128, 4>);
  else if (slots <= 6)
    go(k_decode_layers<128, 6>);
  else
    go(k_decode_layers<128, kMaxSlots>);
  check_launch("decode_layers");
}

}  // namespace mk
