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
constexpr int kG = 8;                     // blocks per chain step group
constexpr int kLane = (kChunk + kG) * 2 + 4;  // term floats per row: the chunk's (dot, scale) pairs + read-ahead + pad
constexpr int kSlot = kR * kLane;
constexpr int kSteps = 5;                 // per layer
constexpr int kCtr = 32;                  // words per counter (128 bytes)
constexpr int kMaxSlots = 8;              // V staging tasks per attention thread (keys up to LDS capacity)
constexpr int kMaxRing = 4;               // weight chunk slots per sub-unit (3 where LDS is short), filled by direct
                                          // global -> LDS copies
constexpr int kStaticLds = 8 * 1024;      // bound on the kernel's static LDS (checked against the build in the tests)
constexpr int kChunkQ = kChunk * 256;     // quant bytes of a chunk (one 8-row group, 48 blocks)
constexpr int kChunkBytes = kChunkQ + kChunk * 16;  // + its scales
constexpr int kCopies = 5;                // copies per worker wave and chunk: 4 x 1 KB of quants, 256 B of scales
constexpr int kWarm = 3;                  // chunks after the ring's first brought into L2 while the input is prepared
static_assert(kChunk == 3 * 16 && kChunk % kG == 0, "three worker waves take 16 blocks of a chunk each");

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

// Direct global -> LDS copies (as lds_copy16 / lds_copy4 in common.h) from a scalar base and a 32-bit lane offset:
// lane i reads sbase + voff_i and writes LDS l + 16 i (4 i). sbase and l are wave-uniform here but derived from the
// thread index, so they are taken from the first lane.
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const T*>((uint64_t)hi << 32 | lo);
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy16s(const void* sbase, uint32_t voff, uint32_t l) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform_ptr(sbase)),
               "s"(__builtin_amdgcn_readfirstlane(l)) : "m0");
}
__device__ __forceinline__ void copy4s(const void* sbase, uint32_t voff, uint32_t l) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(uniform_ptr(sbase)),
               "s"(__builtin_amdgcn_readfirstlane(l)) : "m0");
}
#pragma clang diagnostic pop

// Worker wave ww (0..2) of sub-unit su copies its share of chunk p of step S into the LDS slot: quants 1 KB pieces
// 4 ww .. 4 ww + 3 (piece k = blocks 4k .. 4k + 3 of the chunk, 256 bytes each, in the packed order: lo plane, hi
// plane), and scales 256-byte piece ww (blocks 16 ww .. 16 ww + 15). The quants of a row's last chunk run on into
// the next group's blocks, or for the last group into the scales stream (at least a chunk long: decode_ring checks
// it), never used; scale reads past the row's end re-read its last block. Offsets as in PackedQ8_0 (layout.h), in 32
// bits: a packed weight here is far below 4 GB. slot: the LDS address of the slot. WARM: the same reads, every one
// into the 1 KB at slot (never read): they only bring the chunk into the L2 cache ahead of its real copies.
template <bool WARM = false>
__device__ __forceinline__ void copy_chunk(const Gs& S, int su, int p, int ww, int lane, uint32_t slot) {
  const uint32_t g = (uint32_t)(su + (p / S.nc) * (kSubs * S.nw));
  const int u0 = (p % S.nc) * kChunk;
  const uint8_t* W = glob(S.W);
  const uint8_t* q = W + (g * (uint32_t)S.nu + (uint32_t)u0) * 256u;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    copy16s(q, (uint32_t)((4 * ww + j) * 1024 + lane * 16), WARM ? slot : slot + (4 * ww + j) * 1024);
  const uint8_t* sc = W + (uint32_t)S.ng * (uint32_t)S.nu * 256u + g * (uint32_t)S.nu * 16u;
  const uint32_t u = (uint32_t)min(u0 + 16 * ww + lane / 4, S.nu - 1);
  copy4s(sc, u * 16u + (uint32_t)(lane % 4) * 4u, WARM ? slot : slot + kChunkQ + ww * 256);
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

// LDS of a GEMV step: the input's BlockQ8 row (xs), the two sub-units' double-buffered term slots, an fp32 staging
// area (the rmsnorm's transposed row, or a batch of an fp32 input row read with coalesced loads before it is
// quantized), and the sub-units' weight rings (RING chunk slots each). Only the rings stay live across steps.
struct GemvLds {
  int* xs;
  float* res;
  float* tr;
  uint8_t* ring;
};
constexpr int kLB = 8;                          // 16-byte pieces per loader thread and batch
constexpr int kLoaders = kSubs * 64;            // the chain waves
constexpr int kStageF = kLB * kLoaders * 4;     // fp32 values per input batch
__host__ __device__ constexpr size_t gemv_xs_bytes(int max_cols) { return ((size_t)(max_cols / 32) * 40 + 15) & ~15; }
__host__ __device__ constexpr size_t gemv_stage_floats(int E) { return (size_t)E > (size_t)kStageF ? E : kStageF; }
__host__ __device__ constexpr size_t gemv_ring_offset(int max_cols, int E) {
  return gemv_xs_bytes(max_cols) + (size_t)kSubs * 2 * kSlot * 4 + gemv_stage_floats(E) * 4;
}
__host__ __device__ constexpr size_t gemv_lds_bytes(int max_cols, int E, int ring) {
  return gemv_ring_offset(max_cols, E) + (size_t)kSubs * ring * kChunkBytes;
}
__device__ __forceinline__ GemvLds gemv_lds(int max_cols, int E) {
  extern __shared__ int smem[];
  GemvLds l;
  l.xs = smem;
  l.res = reinterpret_cast<float*>(smem + gemv_xs_bytes(max_cols) / 4);
  l.tr = l.res + kSubs * 2 * kSlot;
  l.ring = reinterpret_cast<uint8_t*>(smem) + gemv_ring_offset(max_cols, E);
  return l;
}

// The loader threads' share of n4 16-byte pieces of the coherent array in (from piece p0): batches of kLB pieces per
// thread, all of a batch's loads issued before the first is used (one memory round trip per batch), then
// use(i4, piece) with i4 counted from p0.
template <typename F>
__device__ __forceinline__ void load_pieces(const void* in, int p0, int n4, int li, F&& use) {
  for (int base = 0; base < n4; base += kLB * kLoaders) {
    float4 v[kLB];
#pragma unroll
    for (int k = 0; k < kLB; ++k)
      v[k] = ld_coh16(in, 16u * (uint32_t)(p0 + min(base + li + k * kLoaders, n4 - 1)));
#pragma unroll
    for (int k = 0; k < kLB; ++k)
      if (base + li + k * kLoaders < n4) use(base + li + k * kLoaders, v[k]);
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
  const int nq8 = cols / 32;
  BlockQ8* xb = reinterpret_cast<BlockQ8*>(l.xs);
  if constexpr (IN == kInNorm) {
    // rmsnorm (model.cpp:46-49): the 16 lane chains of kern::dot_f32 (lane c: x[c], x[16 + c], ... in order) over a
    // transposed copy tt[c][j] = x[16 j + c] (sumsq_lane_chain's layout: four values per LDS read), then the halving
    // tree. The row is loaded in order into tr, transposed into tt (the xs and term-slot area, unused until the
    // quantization below), and tr is read again for the scaling. The norm weights are loaded first: they are ready
    // by the time the scaling needs them.
    const int per = cols / 16, tstride = sumsq_tstride(per), padded = sumsq_padded(per);
    float wv[16];
    const int c16 = tid;  // per <= kDT: one half-block per thread
    if (c16 < per) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 w4 = reinterpret_cast<const float4*>(nw + 16 * c16)[k];
        wv[4 * k] = w4.x, wv[4 * k + 1] = w4.y, wv[4 * k + 2] = w4.z, wv[4 * k + 3] = w4.w;
      }
    }
    if (loader)
      load_pieces(in, 0, cols / 4, li, [&](int i4, const float4& v) { reinterpret_cast<float4*>(l.tr)[i4] = v; });
    float* tt = reinterpret_cast<float*>(l.xs);
    lds_barrier();
    for (int i = tid; i < 16 * padded; i += kDT) tt[(i & 15) * tstride + (i >> 4)] = i < cols ? l.tr[i] : 0.0f;
    __shared__ float scale_s;
    lds_barrier();
    if (tid < 16) {
      float acc = sumsq_lane_chain(tt + tid * tstride, per);
      acc = reduce16_lanes(acc);
      if (tid == 0) scale_s = 1.0f / sqrtf(acc / (float)cols + eps);
    }
    lds_barrier();
    const float sc = scale_s;
    if (c16 < per) {
      float yv[16];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 x4 = reinterpret_cast<const float4*>(l.tr + 16 * c16)[k];
        yv[4 * k] = x4.x, yv[4 * k + 1] = x4.y, yv[4 * k + 2] = x4.z, yv[4 * k + 3] = x4.w;
      }
#pragma unroll
      for (int c = 0; c < 16; ++c) yv[c] = yv[c] * sc * wv[c];
      quantize_half_block(yv, c16 & 1, true, xb + c16 / 2);
    }
  } else if constexpr (IN == kInQ8) {
    // nq8 * 40 bytes: whole 16-byte pieces (nq8 even), and the odd one's last 8 bytes by a 4-byte pair.
    if (loader) {
      load_pieces(in, 0, nq8 * 10 / 4, li, [&](int i4, const float4& v) { reinterpret_cast<float4*>(l.xs)[i4] = v; });
      for (int i = (nq8 * 10 / 4) * 4 + li; i < nq8 * 10; i += kLoaders)
        l.xs[i] = (int)ld_coh_u32(static_cast<const uint32_t*>(in) + i);
    }
  } else {
    // Batches of kStageF values: coalesced coherent loads into the staging area, then 16 consecutive values per lane.
    for (int b0 = 0; b0 < cols; b0 += kStageF) {
      const int nb = min(kStageF, cols - b0);
      if (loader)
        load_pieces(in, b0 / 4, nb / 4, li, [&](int i4, const float4& v) { reinterpret_cast<float4*>(l.tr)[i4] = v; });
      lds_barrier();
      for (int c16 = tid; c16 < nb / 16; c16 += kDT) {
        float v[16];
        const float4* p4 = reinterpret_cast<const float4*>(l.tr + 16 * c16);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float4 a = p4[k];
          v[4 * k] = a.x, v[4 * k + 1] = a.y, v[4 * k + 2] = a.z, v[4 * k + 3] = a.w;
        }
        quantize_half_block(v, c16 & 1, true, xb + (b0 / 16 + c16) / 2);
      }
      lds_barrier();
    }
    return;
  }
  lds_barrier();
}

// Worker terms of chunk c (blocks c * 48 ...) from its ring slot: per (block, row) the exact int dot and dw * dx, zero
// past the row. Worker wave ww takes blocks 16 ww .. 16 ww + 15, four per step; lane l reads the 16 bytes at 16 l of
// the step's four blocks (block l / 16, plane (l / 8) % 2, row l % 8: whole 1 KB, no bank conflicts) and computes the
// int dot of its plane with its half of the block's Q8 activations; the lo-plane lane adds the hi lane's partial
// (lane + 8 of its 16-lane row) and writes the terms. Int sums are exact in any order.
// All of a call's LDS reads (16 per lane: within the 15 the LDS counter can track once the first is consumed) are
// issued before the first dot, so their latencies overlap.
__device__ __forceinline__ void gemv_dots(const uint8_t* slot, float* terms, const int* xs, int c, int nu, int ww,
                                          int lane) {
  const int r = lane & 7, h = (lane >> 3) & 1;
  uint4 w[4];
  uint2 x0[4], x1[4];
  uint16_t dh[4];
  float dx[4];
  bool live[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int ul = 16 * ww + 4 * k + (lane >> 4);
    const int u = c * kChunk + ul;
    live[k] = u < nu;
    const int* xq = xs + (live[k] ? u : 0) * 10;
    w[k] = *reinterpret_cast<const uint4*>(slot + ul * 256 + (lane & 15) * 16);
    x0[k] = *reinterpret_cast<const uint2*>(xq + 2 + 4 * h);
    x1[k] = *reinterpret_cast<const uint2*>(xq + 4 + 4 * h);
    dh[k] = *reinterpret_cast<const uint16_t*>(slot + kChunkQ + ul * 16 + r * 2);
    dx[k] = xd(xq);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int ul = 16 * ww + 4 * k + (lane >> 4);
    int part = dot4((int)w[k].x, (int)x0[k].x, 0);
    part = dot4((int)w[k].y, (int)x0[k].y, part);
    part = dot4((int)w[k].z, (int)x1[k].x, part);
    part = dot4((int)w[k].w, (int)x1[k].y, part);
    const int hi = __builtin_amdgcn_update_dpp(0, part, 0x108, 0xF, 0xF, false);  // row_shl:8
    const float2 t = live[k] ? make_float2((float)(part + hi), half_to_float(dh[k]) * dx[k]) : make_float2(0.0f, 0.0f);
    if (h == 0) *reinterpret_cast<float2*>(terms + r * kLane + ul * 2) = t;
  }
}

// Target of the copies that carry nothing: every worker wave issues kCopies copies per position of its copy stream,
// so that the explicit wait counts stay exact.
__shared__ __align__(16) uint8_t g_junk[1024];

// Where a sub-unit's weight ring (RING slots) stands between steps: base = slot of the next step's chunk 0; ready = the
// copies of that step's first RING - 1 chunks have been issued (by the previous step's last iterations).
struct Ring {
  int base;
  int ready;
};

// One GEMV step of this workgroup (step id sid; its input is step sid - 1's output). N: the sub-unit's next GEMV step
// (n_ok false: none), whose first chunks the last iterations copy into the ring. Returns the ring state for N.
template <int IN, int OUT, int RING>
__device__ __forceinline__ Ring gemv_step(const DecodeArgs* P, int n_steps, int sid, const Gs& S, const Gs& N,
                                          bool n_ok, Ring rs, const void* in, const float* nw, int cols,
                                          int max_cols, int E, float* y) {
  // Wave-uniform values are taken from the first lane, so that the copy addresses are scalar arithmetic.
  const int tid = threadIdx.x, w = blockIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), sub = wv >> 2;
  const bool worker = (wv & 3) != 0;
  const int ww = (wv & 3) - 1;
  const int su = S.su_of(w, sub), nq = S.nq_of(su);
  const int nq_wg = S.nq_of(S.su_of(w, 0));
  const int sun = n_ok ? N.su_of(w, sub) : -1, nn = n_ok ? N.nq_of(sun) : 0;
  const GemvLds l = gemv_lds(max_cols, E);
  uint8_t* ring = l.ring + sub * RING * kChunkBytes;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));
  auto slot = [&](int p) { return ring + ((rs.base + p) % RING) * kChunkBytes; };
  auto slot_lds = [&](int p) { return ring_lds + (uint32_t)(((rs.base + p) % RING) * kChunkBytes); };
  auto copy_junk = [&](const Gs& G) {
    const uint32_t junk = lds_addr(g_junk);
#pragma unroll
    for (int j = 0; j < 4; ++j) copy16s(glob(G.W), (uint32_t)lane * 16u, junk);
    copy4s(glob(G.W), (uint32_t)lane * 16u, junk);
  };
  // Position p of the sub-unit's copy stream: chunk p of S, then N's chunks, then nothing.
  auto issue = [&](int p) {
    if (p < nq)
      copy_chunk(S, su, p, ww, lane, slot_lds(p));
    else if (p - nq < nn)
      copy_chunk(N, sun, p - nq, ww, lane, slot_lds(p));
    else
      copy_junk(S);
  };
  if (worker) {
    if (nq > 0) {
      if (!rs.ready)
        for (int p = 0; p < RING - 1; ++p) issue(p);
      // The next kWarm chunks into L2 (or as many as there are; the rest of the kWarm * kCopies reads are junk
      // copies, which keep the first iteration's wait count exact).
      const uint32_t junk = lds_addr(g_junk);
      for (int p = RING - 1; p < RING - 1 + kWarm; ++p) {
        if (p < nq)
          copy_chunk<true>(S, su, p, ww, lane, junk);
        else
          copy_junk(S);
      }
    } else if (nn > 0) {
      for (int p = 0; p < RING - 1; ++p) {
        if (p < nn)
          copy_chunk(N, sun, p, ww, lane, slot_lds(p));
        else
          copy_junk(N);
      }
    }
  }
  const Ring next = nq > 0 ? Ring{(rs.base + nq) % RING, nn > 0} : Ring{rs.base, nn > 0};
  if (nq_wg == 0) {
    signal_step(P, sid);
    return next;
  }
  wait_step(P, n_steps, sid - 1);
  gemv_input<IN>(l, in, nw, opaque(P)->eps, cols);

  float* terms = l.res + sub * 2 * kSlot;
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
    const float4* e = reinterpret_cast<const float4*>(terms + (q & 1) * kSlot + cr * kLane);
    // The chunk's kChunk / kG groups of terms (4 float4 reads each, inside the row's slot whatever cn is), read three
    // groups ahead of the group being summed.
    constexpr int kNG = kChunk / kG, kAhead = 3;
    float4 T[kNG][4];
    auto fetch = [&](int g) {
#pragma unroll
      for (int i = 0; i < 4; ++i) T[g][i] = e[g * kG / 2 + i];
    };
#pragma unroll
    for (int g = 0; g < kAhead; ++g) fetch(g);
#pragma unroll
    for (int g = 0; g < kNG; ++g) {
      if (g + kAhead < kNG) fetch(g + kAhead);
      __builtin_amdgcn_sched_barrier(0);
      if (g * kG < cn) {
        const float* v = reinterpret_cast<const float*>(T[g]);
#pragma unroll
        for (int i = 0; i < kG; ++i) acc = fma_(v[2 * i], v[2 * i + 1], acc);
      }
      __builtin_amdgcn_sched_barrier(0);
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

  // Iteration q: the workers wait for their copies of chunk q (the RING - 2 chunks after it may be in flight), and
  // after the barrier refill the slot of chunk q - 1 (its dots are done) with position q + RING - 1 and compute
  // chunk q's terms, while the chain wave runs chunk q - 1's chains.
  if (!worker) __builtin_amdgcn_s_setprio(2);
  for (int q = 0; q < nq_wg; ++q) {
    if (worker && q < nq) {
      if (q == 0)
        wait_vm<kCopies * (RING - 2 + kWarm)>();
      else
        wait_vm<kCopies * (RING - 2)>();
    }
    lds_barrier();
    if (worker) {
      if (q < nq) {
        issue(q + RING - 1);
        gemv_dots(slot(q), terms + (q & 1) * kSlot, l.xs, q % S.nc, S.nu, ww, lane);
      }
    } else if (q > 0 && q - 1 < nq) {
      chain(q - 1);
    }
  }
  lds_barrier();
  if (nq == nq_wg) chain(nq - 1);
  if (!worker) {
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's output stores have completed
  }
  signal_step(P, sid);
  return next;
}

template <int D, int NSLOT, int RING>
__global__ __launch_bounds__(kDT) void k_decode_layers(const DecodeArgs* __restrict__ P, int l0, int l1) {
  const int w = blockIdx.x, tid = threadIdx.x;
  const int G = (int)gridDim.x;
  const int n_steps = (l1 - l0) * kSteps;
  Ring rs{0, 0};
  for (int il = l0; il < l1; ++il) {
    const int s0 = (il - l0) * kSteps;
    const bool last = il + 1 == l1;
    const int E = opaque(P)->E, H = opaque(P)->H, KV = opaque(P)->KV, F = opaque(P)->F;
    const int QKV = (H + 2 * KV) * D, HD = H * D, max_cols = max(max(E, HD), F);
    const bool is_att = w < H;  // one attention workgroup per query head (one token)
    const DecodeLayer* L = glob(opaque(P)->layers) + il;

    // q|k|v = W_qkv . rmsnorm(x); the attention workgroups load nothing ahead across their attention step (they load
    // their attn_output chunks right after it).
    rs = gemv_step<kInNorm, kOutStore, RING>(P, n_steps, s0, make_gs(glob(opaque(L)->qkv), QKV, E, 0, G),
                                       make_gs(glob(opaque(L)->wo), E, HD, 0, G), !is_att, rs, glob(opaque(P)->x),
                                       glob(opaque(L)->attn_norm), E, max_cols, E, glob(opaque(P)->qkv));

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
      rs.ready = 0;  // the attention's LDS overlaps the rings: nothing was copied ahead
    }
    signal_step(P, s0 + 1);

    // x += W_o . att
    rs = gemv_step<kInQ8, kOutAcc, RING>(P, n_steps, s0 + 2, make_gs(glob(opaque(L)->wo), E, HD, 0, G),
                                   make_gs(glob(opaque(L)->gate_up), 2 * F, E, 0, G), true, rs, glob(opaque(P)->att),
                                   nullptr, HD, max_cols, E, glob(opaque(P)->x));
    // h = silu(gate) * up of W_gate|up . rmsnorm(x)
    rs = gemv_step<kInNorm, kOutSilu, RING>(P, n_steps, s0 + 3, make_gs(glob(opaque(L)->gate_up), 2 * F, E, 0, G),
                                      make_gs(glob(opaque(L)->down), E, F, 0, G), true, rs, glob(opaque(P)->x),
                                      glob(opaque(L)->ffn_norm), E, max_cols, E, glob(opaque(P)->h));
    // x += W_down . h; then the next layer's q|k|v
    const void* next_qkv = last ? glob(opaque(L)->qkv) : glob(opaque(L + 1)->qkv);
    rs = gemv_step<kInF32, kOutAcc, RING>(P, n_steps, s0 + 4, make_gs(glob(opaque(L)->down), E, F, 0, G),
                                    make_gs(next_qkv, QKV, E, 0, G), !last, rs, glob(opaque(P)->h), nullptr, F,
                                    max_cols, E, glob(opaque(P)->x));
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

// One layer's attention and attn_output GEMV in one launch, between the per-step q|k|v and gate|up launches: the H
// attention workgroups run attention (their q|k|v input is complete: the previous launch has ended), while the others
// already copy their attn_output chunks into their rings; the GEMV step then waits for the attention step through the
// counters of the layer's steps 1 and 2 (the same counters, exit count and error word as k_decode_layers with all
// n_layer layers). Results as the attention and attn_output launches it replaces.
template <int D, int NSLOT, int RING>
__global__ __launch_bounds__(kDT) void k_decode_attn_wo(const DecodeArgs* __restrict__ P, int il, int n_layer) {
  const int w = blockIdx.x, tid = threadIdx.x;
  const int G = (int)gridDim.x;
  const int n_steps = n_layer * kSteps, s0 = il * kSteps;
  const int E = opaque(P)->E, H = opaque(P)->H, KV = opaque(P)->KV, F = opaque(P)->F;
  const int HD = H * D, max_cols = max(max(E, HD), F);
  const DecodeLayer* L = glob(opaque(P)->layers) + il;
  if (w < H) {
    const auto* Q = opaque(P);
    const size_t lrow = (size_t)il * Q->n_seq * KV * Q->n_ctx;
    const KvLayer kv{glob(Q->k8) + lrow * D, glob(Q->v8) + lrow * D, glob(Q->ks) + lrow, glob(Q->vs) + lrow};
    const int64_t rows = Q->n_ctx;
    const AttnAddr a{kv.k,  kv.v, reinterpret_cast<const char*>(kv.ks), reinterpret_cast<const char*>(kv.vs),
                     (int64_t)KV * rows * D, rows * D, D, (int64_t)KV * rows * 4, rows * 4, 4, 1};
    const DecFuse f{glob(Q->qkv), 0, glob(opaque(L)->q_norm), glob(opaque(L)->k_norm), Q->eps, glob(Q->cos_t),
                    glob(Q->sin_t), glob(Q->rpos), glob(Q->kv_row), kv, Q->n_ctx, KV};
    attend_dec<D, NSLOT, true, true, kDT>(w, nullptr, 0, nullptr, 0, H / KV, Q->scale, a, glob(Q->seq),
                                          glob(Q->n_keys), 1, H, f, glob(Q->att), 0, [] {});
    __builtin_amdgcn_s_waitcnt(0);
  }
  signal_step(P, s0 + 1);
  // x += W_o . att (no next step: the gate|up launch follows)
  const Gs wo = make_gs(glob(opaque(L)->wo), E, HD, 0, G);
  gemv_step<kInQ8, kOutAcc, RING>(P, n_steps, s0 + 2, wo, wo, false, Ring{0, 0}, glob(opaque(P)->att), nullptr, HD,
                                  max_cols, E, glob(opaque(P)->x));
  __builtin_amdgcn_s_waitcnt(0);
  if ((tid >> 6) == 0) {
    unsigned old = 0;
    if (tid == 0) old = __hip_atomic_fetch_add(exit_ctr(P, n_steps), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old == (unsigned)G - 1) {
      unsigned* sync = glob(opaque(P)->sync);
      for (int i = tid; i < 2 * 8; i += 64) st_coh_u32(sync + ((size_t)(s0 + 1) * 8 + i) * kCtr, 0u);
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
  // The attention step takes H of the workgroups (one per CU).
  return decode_ring(d, max_keys) >= 3 && device_cus() >= d.H;
}

// Weight ring depth for a model and key count: 4 slots where LDS allows, else 3 (0: the step does not fit). A step's
// copy stream runs ring - 1 chunks ahead, into the next GEMV step only: every sub-unit's share of a step (whole rows:
// at least one row's chunks) has at least ring - 1 chunks.
int decode_ring(const DecodeDims& d, int max_keys) {
  const int max_cols = std::max(std::max(d.E, d.H * d.D), d.F);
  // A row's last chunk of quants may run on into the scales stream (E rows is the smallest weight: at least a chunk)
  if ((size_t)d.E / 8 * (size_t)(d.E / 32) * 16 < (size_t)kChunkQ) return 0;
  // rmsnorm: one half-block per thread; the transposed row fits in the xs and term-slot area
  if (d.E / 16 > kDT ||
      (size_t)16 * sumsq_tstride(d.E / 16) * 4 > gemv_xs_bytes(max_cols) + (size_t)kSubs * 2 * kSlot * 4)
    return 0;
  const int min_cols = std::min(std::min(d.E, d.H * d.D), d.F);
  const int min_chunks = (min_cols / 32 + kChunk - 1) / kChunk;
  for (int ring = std::min(kMaxRing, min_chunks + 1); ring >= 3; --ring) {
    const size_t lds = std::max(gemv_lds_bytes(max_cols, d.E, ring), dec_lds_bytes(d.D, attn_keys_pad(max_keys)));
    if (lds + kStaticLds <= 160 * 1024) return ring;
  }
  return 0;
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

namespace {
// Launches a kernel of this file (all layers, or one layer's attention + attn_output) with the plan's LDS and the
// whole grid resident; select(slots, ring) returns the instantiation.
template <typename Sel, typename... Args>
void decode_launch(hipStream_t s, const DecodeDims& d, int max_keys, const char* what, Sel&& select, Args... args) {
  const int max_cols = std::max(std::max(d.E, d.H * d.D), d.F);
  const int ring = decode_ring(d, max_keys);
  const size_t lds = std::max(gemv_lds_bytes(max_cols, d.E, ring), dec_lds_bytes(d.D, attn_keys_pad(max_keys)));
  const int cus = device_cus();
  const auto kernel = select(dec_slots(d.D, max_keys, true, kDT), ring);
  check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024 - kStaticLds),
        "hipFuncSetAttribute");
  hipFuncAttributes fa{};
  check(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kernel)), "hipFuncGetAttributes");
  require(fa.sharedSizeBytes <= (size_t)kStaticLds, "decode: static LDS above its bound");
  int per_cu = 0;
  check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kDT, lds),
        "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  // Every workgroup waits for the others: the whole grid (one workgroup per CU) must be resident at once.
  require(per_cu >= 1, "decode: the kernel does not fit on a CU");
  hipLaunchKernelGGL(kernel, dim3(cus), dim3(kDT), lds, s, args...);
  check_launch(what);
}
}  // namespace

void decode_attn_wo(hipStream_t s, const void* dev_args, const DecodeDims& d, int layer, int n_layer, int max_keys) {
  require(decode_layers_supported(d, max_keys), "decode_attn_wo: unsupported shape");
  require(layer >= 0 && layer < n_layer, "decode_attn_wo: bad layer");
  using K = void (*)(const DecodeArgs*, int, int);
  auto select = [](int slots, int ring) -> K {
    if (slots <= 2) return ring == 4 ? k_decode_attn_wo<128, 2, 4> : k_decode_attn_wo<128, 2, 3>;
    if (slots <= 4) return ring == 4 ? k_decode_attn_wo<128, 4, 4> : k_decode_attn_wo<128, 4, 3>;
    if (slots <= 6) return ring == 4 ? k_decode_attn_wo<128, 6, 4> : k_decode_attn_wo<128, 6, 3>;
    return ring == 4 ? k_decode_attn_wo<128, kMaxSlots, 4> : k_decode_attn_wo<128, kMaxSlots, 3>;
  };
  decode_launch(s, d, max_keys, "decode_attn_wo", select, static_cast<const DecodeArgs*>(dev_args), layer, n_layer);
}

void decode_layers(hipStream_t s, const void* dev_args, const DecodeDims& d, int l0, int l1, int max_keys) {
  require(decode_layers_supported(d, max_keys), "decode_layers: unsupported shape");
  require(l0 >= 0 && l1 > l0, "decode_layers: bad layer range");
  const int max_cols = std::max(std::max(d.E, d.H * d.D), d.F);
  const int ring = decode_ring(d, max_keys);
  const size_t lds = std::max(gemv_lds_bytes(max_cols, d.E, ring), dec_lds_bytes(d.D, attn_keys_pad(max_keys)));
  const int cus = device_cus();
  const DecodeArgs* P = static_cast<const DecodeArgs*>(dev_args);
  auto go = [&](auto kernel) {
    static bool attr = false;
    if (!attr) {
      check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024 - kStaticLds),
            "hipFuncSetAttribute");
      attr = true;
    }
    hipFuncAttributes fa{};
    check(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kernel)), "hipFuncGetAttributes");
    require(fa.sharedSizeBytes <= (size_t)kStaticLds, "decode_layers: static LDS above its bound");
    int per_cu = 0;
    check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kDT, lds),
          "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    // Every workgroup waits for the others: the whole grid (one workgroup per CU) must be resident at once.
    require(per_cu >= 1, "decode_layers: the kernel does not fit on a CU");
    hipLaunchKernelGGL(kernel, dim3(cus), dim3(kDT), lds, s, P, l0, l1);
  };
  const int slots = dec_slots(d.D, max_keys, true, kDT);
  auto pick = [&](auto k4, auto k3) { ring == 4 ? go(k4) : go(k3); };
  if (slots <= 2)
    pick(k_decode_layers<128, 2, 4>, k_decode_layers<128, 2, 3>);
  else if (slots <= 4)
    pick(k_decode_layers<128, 4, 4>, k_decode_layers<128, 4, 3>);
  else if (slots <= 6)
    pick(k_decode_layers<128, 6, 4>, k_decode_layers<128, 6, 3>);
  else
    pick(k_decode_layers<128, kMaxSlots, 4>, k_decode_layers<128, kMaxSlots, 3>);
  check_launch("decode_layers");
}

}  // namespace mk
