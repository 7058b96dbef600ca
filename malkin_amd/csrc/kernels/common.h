// Device-side building blocks shared by the gfx950 kernels.
//
// Bit-exactness rules (the kernels reproduce the reference's AVX-512 fp32 arithmetic one rounding at a time):
//   * every source is compiled with -ffp-contract=off; fused multiply-adds are explicit __builtin_fmaf calls, placed
//     exactly where the reference uses _mm512_fmadd_ps / _mm512_fnmadd_ps (or where clang contracts its scalar code);
//   * '/' and sqrtf are correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt, the HIP default);
//   * fp32 denormals are kept (no flush-to-zero), as under the x86 default MXCSR.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mk {

// Activation block, byte-identical to the reference's BlockQ8 (quant.h:11-16).
struct BlockQ8 {
  float d;
  int16_t s[2];
  int8_t qs[32];
};
static_assert(sizeof(BlockQ8) == 40, "BlockQ8 is 40 bytes");

constexpr int kWave = 64;

__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// _mm512_reduce_add_ps as clang lowers it: halving tree (i, i+8), (i, i+4), (i, i+2), (0, 1).
__device__ __forceinline__ float reduce16(const float* v) {
  float a[8], b[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = v[i] + v[i + 8];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = a[i] + a[i + 4];
  const float c0 = b[0] + b[2], c1 = b[1] + b[3];
  return c0 + c1;
}

// Lane l gets lane l + K of its 16-lane row; lanes past the row's end keep their own value (the semantics of
// __shfl_down(v, K, 16)), by DPP row_shl: a register move instead of an LDS permute round trip.
template <int K>
__device__ __forceinline__ float shl16(float v) {
  const int x = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(x, x, 0x100 + K, 0xF, 0xF, false));
}

// shl16 with a shift that folds to a constant only after unrolling (0 = the lane's own value).
__device__ __forceinline__ float shl16_k(float v, int k) {
  const int x = __builtin_bit_cast(int, v);
  int r = x;
  switch (k) {
#define MK_SHL16_CASE(K) \
  case K:                \
    r = __builtin_amdgcn_update_dpp(x, x, 0x100 + K, 0xF, 0xF, false); \
    break;
    MK_SHL16_CASE(1) MK_SHL16_CASE(2) MK_SHL16_CASE(3) MK_SHL16_CASE(4) MK_SHL16_CASE(5) MK_SHL16_CASE(6)
    MK_SHL16_CASE(7) MK_SHL16_CASE(8) MK_SHL16_CASE(9) MK_SHL16_CASE(10) MK_SHL16_CASE(11) MK_SHL16_CASE(12)
    MK_SHL16_CASE(13) MK_SHL16_CASE(14) MK_SHL16_CASE(15)
#undef MK_SHL16_CASE
    default:
      break;
  }
  return __builtin_bit_cast(float, r);
}

// Workgroups are dealt to the 8 XCDs in turn (workgroup w runs on XCD w % 8, each XCD with its own L2). xcd_run
// numbers them so that XCD x takes one contiguous run of the items 0 .. total - 1, for any total (a bijection: XCD x
// holds total / 8 + (x < total % 8) workgroups, and its run starts after those of XCDs 0 .. x - 1). Items that share
// operands and are numbered next to each other then share an XCD and read those operands into its L2 once.
__device__ __forceinline__ int xcd_run(int w, int total) {
  const int x = w & 7, j = w >> 3;
  return x * (total >> 3) + min(x, total & 7) + j;
}

// The same tree over 16 consecutive lanes of a wavefront: lane l (l % 16 == 0 after the call holds the sum of lanes
// l..l+15). Valid in lanes whose 16-lane group is fully active.
__device__ __forceinline__ float reduce16_lanes(float v) {
  v = v + shl16<8>(v);
  v = v + shl16<4>(v);
  v = v + shl16<2>(v);
  v = v + shl16<1>(v);
  return v;
}

// reduce16_lanes of N values at once (N = 1..5), the halving steps interleaved across the values: one v_add_f32_dpp
// per value and step (lane l adds lane l + S's value: the same pairs as reduce16_lanes; a + b == b + a). A DPP read
// of a VGPR needs two wait states after a VALU write of it: before the first step, and between steps when fewer than
// three other instructions separate them (N < 3), an s_nop provides them.
template <int S, int N>
__device__ __forceinline__ void add_shl16_step(float (&v)[N]) {
  static_assert(N >= 2 && N <= 5, "2 to 5 values");
#define MK_ADD(I) "v_add_f32_dpp %" #I ", %" #I ", %" #I " row_shl:%" MK_NS " row_mask:0xf bank_mask:0xf\n\t"
  if constexpr (N == 2) {
#define MK_NS "2"
    asm("s_nop 1\n\t" MK_ADD(0) MK_ADD(1) : "+v"(v[0]), "+v"(v[1]) : "i"(S));
#undef MK_NS
  } else if constexpr (N == 3) {
#define MK_NS "3"
    asm("s_nop 1\n\t" MK_ADD(0) MK_ADD(1) MK_ADD(2) : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]) : "i"(S));
#undef MK_NS
  } else if constexpr (N == 4) {
#define MK_NS "4"
    asm("s_nop 1\n\t" MK_ADD(0) MK_ADD(1) MK_ADD(2) MK_ADD(3)
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "i"(S));
#undef MK_NS
  } else {
#define MK_NS "5"
    asm("s_nop 1\n\t" MK_ADD(0) MK_ADD(1) MK_ADD(2) MK_ADD(3) MK_ADD(4)
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]) : "i"(S));
#undef MK_NS
  }
#undef MK_ADD
}
template <int N>
__device__ __forceinline__ void reduce16_lanes_n(float (&v)[N]) {
  if constexpr (N == 1) {
    v[0] = reduce16_lanes(v[0]);
  } else {
    add_shl16_step<8>(v);
    add_shl16_step<4>(v);
    add_shl16_step<2>(v);
    add_shl16_step<1>(v);
  }
}

// Direct global -> LDS copies: lane i writes its 16 (or 4) bytes at the wave-uniform LDS address + 16 i (4 i). They
// are issued as inline assembly so that the compiler does not track them as LDS stores: it cannot tell a copy into a
// later pipeline stage from the stage being read and would wait for every copy in flight (vmcnt(0)) before each LDS
// read, which empties a prefetch ring. Kernels using them order them explicitly: a stage is read only after its own
// copies are waited for (s_waitcnt vmcnt) and a barrier, and a buffer is refilled only after the barrier that follows
// its last reads. M0 is named as clobbered (the copies set it); the compiler warns about clobbering a register it
// reserves, which is the intent here. On GFX9 an LDS DMA instruction reads M0 one wait state after an SALU write of
// it at the earliest (the hazard the compiler's own LDS DMA code respects): the s_nop between them is that state,
// without which a copy can land at the previous copy's LDS address.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ uint32_t lds_addr(const void* l) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)l;
}
__device__ __forceinline__ void lds_copy16(const void* g, void* l) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr(l)) : "m0");
}
__device__ __forceinline__ void lds_copy4(const void* g, void* l) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr(l)) : "m0");
}
#pragma clang diagnostic pop

// Ring staging with the copies above. ring_barrier: a plain s_barrier (the copies are waited for explicitly; a fenced
// barrier would make the compiler wait for every one in flight, prefetches included). wait_vm<N>: s_waitcnt vmcnt(N)
// (N < 64: bits 3:0 and 15:14), expcnt and lgkmcnt left at their maximum. wait_vm_stages<PER, KMAX>(k): vmcnt(k PER)
// for a runtime k in [0, KMAX], i.e. "at most k stages of PER copies each still in flight".
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
template <int PER, int KMAX>
__device__ __forceinline__ void wait_vm_stages(int k) {
  if constexpr (KMAX > 0) {
    if (k >= KMAX) {
      wait_vm<KMAX * PER>();
      return;
    }
    wait_vm_stages<PER, KMAX - 1>(k);
  } else {
    wait_vm<0>();
  }
}

// Workgroup barrier that orders LDS only. __syncthreads() also waits for every outstanding global load of the
// calling wave, which would turn loads issued ahead of a barrier (prefetches) into a full memory round trip.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Lane k of each 16-lane row, broadcast to the row (DPP row_newbcast, a register move). k must fold to a constant:
// call it from fully unrolled loops. Used where every lane needs the same value: gfx950 serialises 16-byte LDS reads
// that all lanes make at one address, and readlane would go through SGPRs.
__device__ __forceinline__ float bcast16(float x, int k) {
  const int v = __builtin_bit_cast(int, x);
  int r;
  switch (k) {
#define MK_BCAST16_CASE(K) \
  case K:                  \
    r = __builtin_amdgcn_update_dpp(0, v, 0x150 + K, 0xF, 0xF, true); \
    break;
    MK_BCAST16_CASE(0) MK_BCAST16_CASE(1) MK_BCAST16_CASE(2) MK_BCAST16_CASE(3) MK_BCAST16_CASE(4)
    MK_BCAST16_CASE(5) MK_BCAST16_CASE(6) MK_BCAST16_CASE(7) MK_BCAST16_CASE(8) MK_BCAST16_CASE(9)
    MK_BCAST16_CASE(10) MK_BCAST16_CASE(11) MK_BCAST16_CASE(12) MK_BCAST16_CASE(13) MK_BCAST16_CASE(14)
    default: MK_BCAST16_CASE(15)
#undef MK_BCAST16_CASE
  }
  return __builtin_bit_cast(float, r);
}

// fma(p, v, acc) with p = lane K of x's 16-lane row: the DPP row_newbcast broadcast folded into the fma, one VALU
// instruction per chain step (a dependent step takes 12 cycles, as a plain fma; a separate DPP move adds 5). For K = 0
// an s_nop provides the 2 wait states a DPP source needs after a VALU write of it; later K of the same x follow other
// instructions. The nop is not placed on every step: it adds its cycles to the chain's latency.
template <int K>
__device__ __forceinline__ float fma_bcast16(float x, float v, float acc) {
  if constexpr (K == 0)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf"
        : "+v"(acc)
        : "v"(x), "v"(v));
  else
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(x), "v"(v), "i"(K));
  return acc;
}

// fma_bcast16<K>, then the SDWA convert of byte B of w into cvt (as i8_to_f32<B>), as one pair of instructions: a
// chain that converts the next group of values while it runs the current one puts each convert, which does not
// depend on the chain, in the dependent fma's latency instead of in front of the fma that consumes it.
template <int K, int B>
__device__ __forceinline__ float fma_bcast16_cvt(float x, float v, float acc, uint32_t w, float& cvt) {
  if constexpr (K == 0)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_%5"
        : "+v"(acc), "=&v"(cvt)
        : "v"(x), "v"(v), "v"(w), "i"(B));
  else
    asm("v_fmac_f32_dpp %0, %2, %3 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_%5"
        : "+v"(acc), "=&v"(cvt)
        : "v"(x), "v"(v), "v"(w), "i"(B), "i"(K));
  return acc;
}

// Eight consecutive fma_bcast16_cvt steps (keys K0 .. K0 + 7 of a 16-key group: converts of the bytes of w0, then
// w1) in one asm statement, so that no wait states are placed between the steps: inside the statement only the DPP
// source x is read through DPP, and nothing in it writes x. K0 = 0 starts with the two wait states a DPP read of x
// needs after x is written.
template <int K0>
__device__ __forceinline__ float fma8_bcast16_cvt(float x, const float (&v)[16], float acc, uint32_t w0, uint32_t w1,
                                                  float (&cvt)[16]) {
  static_assert(K0 == 0 || K0 == 8, "two halves of a 16-key group");
  if constexpr (K0 == 0)
    asm("s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %17, %9 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_fmac_f32_dpp %0, %17, %10 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %2, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_fmac_f32_dpp %0, %17, %11 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %3, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_fmac_f32_dpp %0, %17, %12 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %4, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "v_fmac_f32_dpp %0, %17, %13 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %5, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_fmac_f32_dpp %0, %17, %14 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %6, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_fmac_f32_dpp %0, %17, %15 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %7, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_fmac_f32_dpp %0, %17, %16 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %8, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        : "+v"(acc), "=&v"(cvt[0]), "=&v"(cvt[1]), "=&v"(cvt[2]), "=&v"(cvt[3]), "=&v"(cvt[4]), "=&v"(cvt[5]),
          "=&v"(cvt[6]), "=&v"(cvt[7])
        : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]), "v"(x), "v"(w0),
          "v"(w1));
  else
    asm("v_fmac_f32_dpp %0, %17, %9 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_fmac_f32_dpp %0, %17, %10 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %2, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_fmac_f32_dpp %0, %17, %11 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %3, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_fmac_f32_dpp %0, %17, %12 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %4, sext(%18) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "v_fmac_f32_dpp %0, %17, %13 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %5, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_fmac_f32_dpp %0, %17, %14 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %6, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_fmac_f32_dpp %0, %17, %15 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %7, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_fmac_f32_dpp %0, %17, %16 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        "v_cvt_f32_i32_sdwa %8, sext(%19) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        : "+v"(acc), "=&v"(cvt[8]), "=&v"(cvt[9]), "=&v"(cvt[10]), "=&v"(cvt[11]), "=&v"(cvt[12]), "=&v"(cvt[13]),
          "=&v"(cvt[14]), "=&v"(cvt[15])
        : "v"(v[8]), "v"(v[9]), "v"(v[10]), "v"(v[11]), "v"(v[12]), "v"(v[13]), "v"(v[14]), "v"(v[15]), "v"(x),
          "v"(w0), "v"(w1));
  return acc;
}

// (float)(int8_t)(w >> 8 K): one SDWA convert of byte K (the compiler otherwise emits shift, extract and convert
// where the source word is live across a scheduling barrier).
template <int K>
__device__ __forceinline__ float i8_to_f32(uint32_t w) {
  float r;
  asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_%2" : "=v"(r) : "v"(w), "i"(K));
  return r;
}

// exp512 (kernels_avx512.cpp:186-202), one lane: max(x, -87), Cody-Waite reduction, degree-6 Taylor, scalef.
// This is the reference's own polynomial, not a library exponential.
__device__ __forceinline__ float exp512(float x) {
  x = fmaxf(x, -87.0f);
  const float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = fma_(-n, 0.693145751953125f, x);
  r = fma_(-n, 1.42860682030941723e-6f, r);
  float p = 1.0f / 720.0f;
  p = fma_(p, r, 1.0f / 120.0f);
  p = fma_(p, r, 1.0f / 24.0f);
  p = fma_(p, r, 1.0f / 6.0f);
  p = fma_(p, r, 0.5f);
  p = fma_(p, r, 1.0f);
  p = fma_(p, r, 1.0f);
  // _mm512_scalef_ps(p, n) with integral n: p * 2^n. Clamp the exponent so ldexp sees an in-range int; beyond +-300
  // the result saturates to inf / 0 exactly as scalef does.
  const float nc = fminf(fmaxf(n, -300.0f), 300.0f);
  return __builtin_ldexpf(p, (int)nc);
}

__device__ __forceinline__ float half_to_float(uint16_t h) {
  return __builtin_bit_cast(_Float16, h);
}

// Signed 8-bit dot of 4-byte groups: exact int32.
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// A BlockQ8 held in LDS as 10 words {d, s0 | s1 << 16, qs[32]}: the exact int dot of its 32 quants with 32 int8
// weights given as two 16-byte planes (lo = weights 0..15, hi = 16..31), and its fields.
__device__ __forceinline__ int dot8(const uint4& lo, const uint4& hi, const int* xq) {
  int ai = dot4((int)lo.x, xq[2], 0);
  ai = dot4((int)lo.y, xq[3], ai);
  ai = dot4((int)lo.z, xq[4], ai);
  ai = dot4((int)lo.w, xq[5], ai);
  ai = dot4((int)hi.x, xq[6], ai);
  ai = dot4((int)hi.y, xq[7], ai);
  ai = dot4((int)hi.z, xq[8], ai);
  ai = dot4((int)hi.w, xq[9], ai);
  return ai;
}
__device__ __forceinline__ float xd(const int* xq) { return __int_as_float(xq[0]); }
__device__ __forceinline__ int xs0(const int* xq) { return (int)(int16_t)(xq[1] & 0xFFFF); }
__device__ __forceinline__ int xs1(const int* xq) { return (int)(int16_t)((uint32_t)xq[1] >> 16); }

// _mm512_cvtps_epi32 under the default MXCSR (round to nearest even), then saturation to int8.
__device__ __forceinline__ int cvt_rne(float x) {
  if (!(x >= -2147483648.0f && x < 2147483648.0f)) return INT32_MIN;
  return (int)__builtin_rintf(x);
}

__device__ __forceinline__ int sat8(int v) { return v > 127 ? 127 : (v < -128 ? -128 : v); }

// One 32-value block of f32 activations -> BlockQ8 (kernels_avx512.cpp:66-80), held by 32 / N consecutive lanes
// (aligned to 32 / N): lane l of the block holds values N l .. N l + N - 1. Every lane of the block calls this. amax is
// an exact max and the half sums are exact integer sums, so the lane order of the reductions does not matter.
template <int N>
__device__ __forceinline__ void quantize_block_lanes_n(const float (&v)[N], int l, BlockQ8* out) {
  constexpr int LB = 32 / N;  // lanes per block
  static_assert(N == 1 || N == 2 || N == 4, "1, 2 or 4 values per lane");
  float amax = fabsf(v[0]);
#pragma unroll
  for (int k = 1; k < N; ++k) amax = fmaxf(amax, fabsf(v[k]));
#pragma unroll
  for (int off = LB / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, LB));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int s = 0;
  uint32_t packed = 0;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int q = cvt_rne(v[k] * id);
    s += q;
    packed |= (uint32_t)(uint8_t)(int8_t)sat8(q) << (8 * k);
  }
#pragma unroll
  for (int off = LB / 4; off > 0; off >>= 1) s += __shfl_xor(s, off, LB / 2);
  int8_t* o = reinterpret_cast<int8_t*>(out);
  if constexpr (N == 1) o[8 + l] = (int8_t)packed;
  else if constexpr (N == 2) *reinterpret_cast<uint16_t*>(o + 8 + 2 * l) = (uint16_t)packed;
  else *reinterpret_cast<uint32_t*>(o + 8 + 4 * l) = packed;
  if (l == 0) {
    *reinterpret_cast<float*>(o) = d;
    *reinterpret_cast<int16_t*>(o + 4) = (int16_t)s;
  } else if (l == LB / 2) {
    *reinterpret_cast<int16_t*>(o + 6) = (int16_t)s;
  }
}

// Device-coherent 4-byte accesses (relaxed atomics at agent scope: global loads and stores with sc1, which bypass the
// per-XCD caches). Data that one workgroup stores this way is read correctly by a workgroup on another XCD once the
// writer's stores have completed (s_waitcnt) before it signals, and the reader reads after seeing the signal.
__device__ __forceinline__ uint32_t ld_coh_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __builtin_bit_cast(float, ld_coh_u32(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void st_coh_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
  st_coh_u32(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v));
}

// quantize_block_lanes_n<1> (one value per lane, 32 lanes per block, l = d % 32) writing the block at blk0 + d / 32
// with coherent word stores: lane 0 the scale, lane 1 the two half sums, lanes 2..9 the quants of lanes 4 (l - 2) ..
// 4 (l - 2) + 3. The 32 lanes of a block must call this together.
__device__ __forceinline__ void put_q8_coh(BlockQ8* blk0, int d, float v) {
  const int l = d & 31;
  float amax = fabsf(v);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
  const float dq = amax / 127.0f;
  const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
  const int q = cvt_rne(v * id);
  int s = q;
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 16);
  const int b = (int)(uint32_t)(uint8_t)(int8_t)sat8(q);
  const int src = 4 * (l >= 2 && l < 10 ? l - 2 : 0);
  const uint32_t quad = (uint32_t)__shfl(b, src, 32) | (uint32_t)__shfl(b, src + 1, 32) << 8 |
                        (uint32_t)__shfl(b, src + 2, 32) << 16 | (uint32_t)__shfl(b, src + 3, 32) << 24;
  const int s_hi = __shfl(s, 16, 32);
  const uint32_t word = l == 0 ? __builtin_bit_cast(uint32_t, dq)
                        : l == 1 ? ((uint32_t)(uint16_t)(int16_t)s | (uint32_t)(uint16_t)(int16_t)s_hi << 16)
                                 : quad;
  if (l < 10) st_coh_u32(reinterpret_cast<uint32_t*>(blk0 + d / 32) + l, word);
}

// Value d of an attention output row (row[d] = v) and, with xq, its BlockQ8 row as quantize_acts writes it
// (model.cpp:398-401): column hd + d of the token's blocks at xq + xq_row (hd % 32 == 0). The 32 lanes that hold
// d = 32 b .. 32 b + 31 must call this together.
__device__ __forceinline__ void put_out(float* row, BlockQ8* xq, int64_t xq_row, int hd, int d, float v) {
  row[d] = v;
  if (xq) {
    const float one[1] = {v};
    quantize_block_lanes_n<1>(one, d & 31, xq + xq_row + (hd + d) / 32);
  }
}

// Half of one Q8 block (16 consecutive values, h = which half) -> its BlockQ8 bytes (kernels_avx512.cpp:66-80). The
// two halves sit on neighbouring lanes (h = lane & 1); every lane must call this, as the block max is exchanged between
// the pair. amax is an exact max and the half sums are exact integer sums, so their order does not matter.
__device__ __forceinline__ void quantize_half_block(const float (&v)[16], int h, bool store, BlockQ8* out) {
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < 16; ++c) amax = fmaxf(amax, fabsf(v[c]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int s = 0;
  uint32_t packed[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int q = cvt_rne(v[4 * k + c] * id);
      s += q;
      word |= (uint32_t)(uint8_t)(int8_t)sat8(q) << (8 * c);
    }
    packed[k] = word;
  }
  if (!store) return;
  uint8_t* o = reinterpret_cast<uint8_t*>(out);
  // BlockQ8 is 8-byte aligned (40-byte blocks), so its quants take two 8-byte stores per half.
  *reinterpret_cast<uint2*>(o + 8 + 16 * h) = make_uint2(packed[0], packed[1]);
  *reinterpret_cast<uint2*>(o + 16 + 16 * h) = make_uint2(packed[2], packed[3]);
  if (h == 0) {
    *reinterpret_cast<float*>(o) = d;
    *reinterpret_cast<int16_t*>(o + 4) = (int16_t)s;
  } else {
    *reinterpret_cast<int16_t*>(o + 6) = (int16_t)s;
  }
}


// Values per row of the transposed copy used by sumsq_lane_chain (per = n / 16, zero-padded to a multiple of 64), and
// its row stride in floats (4 more, against bank conflicts; rows stay 16-byte aligned).
__host__ __device__ constexpr int sumsq_padded(int per) { return (per + 63) & ~63; }
__host__ __device__ constexpr int sumsq_tstride(int per) { return sumsq_padded(per) + 4; }

// One lane chain of kern::dot_f32(x, x) (kernels_avx512.cpp:82-89): acc = fma(x_i, x_i, acc) over the lane's values
// in order, given as the lane's contiguous row tl of a transposed copy, zero-padded to a multiple of 64 values
// (fma(0, 0, acc) == acc: the sum of squares is never -0). 16 values per step in two alternating register sets: the
// next 16 are read while the current ones run, and the scheduling barriers keep the reads ahead of the fmas.
__device__ __forceinline__ float sumsq_lane_chain(const float* tl, int per) {
  const int nh = sumsq_padded(per) / 16;  // 16-value quarters of the padded row, an even count
  const float4* p4 = reinterpret_cast<const float4*>(tl);
  float acc = 0.0f;
  float4 a[4], b[4];
  auto ld = [&](float4(&r)[4], int h) {
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = p4[4 * h + k];
  };
  auto run = [&](const float4(&r)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc = fma_(r[k].x, r[k].x, acc);
      acc = fma_(r[k].y, r[k].y, acc);
      acc = fma_(r[k].z, r[k].z, acc);
      acc = fma_(r[k].w, r[k].w, acc);
    }
  };
  ld(a, 0);
  for (int h = 0; h < nh; h += 2) {
    ld(b, h + 1);
    __builtin_amdgcn_sched_barrier(0);
    run(a);
    ld(a, min(h + 2, nh - 1));  // past the end: the last quarter again, unused
    __builtin_amdgcn_sched_barrier(0);
    run(b);
  }
  return acc;
}


}  // namespace mk
