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

// The same tree over 16 consecutive lanes of a wavefront: lane l (l % 16 == 0 after the call holds the sum of lanes
// l..l+15). Valid in lanes whose 16-lane group is fully active.
__device__ __forceinline__ float reduce16_lanes(float v) {
  v = v + __shfl_down(v, 8, 16);
  v = v + __shfl_down(v, 4, 16);
  v = v + __shfl_down(v, 2, 16);
  v = v + __shfl_down(v, 1, 16);
  return v;
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

// _mm512_cvtps_epi32 under the default MXCSR (round to nearest even), then saturation to int8.
__device__ __forceinline__ int cvt_rne(float x) {
  if (!(x >= -2147483648.0f && x < 2147483648.0f)) return INT32_MIN;
  return (int)__builtin_rintf(x);
}

__device__ __forceinline__ int sat8(int v) { return v > 127 ? 127 : (v < -128 ? -128 : v); }

}  // namespace mk
