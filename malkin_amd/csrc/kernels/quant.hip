// Activation quantization and the per-token elementwise ops of Model::run, fused where the reference runs them
// back to back, each bit-identical to the reference:
//   quantize_q8     kernels_avx512.cpp:66-80 (kern::quantize_row_q8)
//   quantize_i8     quant.cpp:134-140
//   rmsnorm(_q8)    model.cpp:46-49 (+ quantize_acts, model.cpp:362-364, 403-405, 421-422)
//   silu_mul(_q8)   kernels_avx512.cpp:271-280 (+ quantize_acts, model.cpp:409-411)
//   dequantize_rows quant.cpp:70-128 (token embedding lookup, model.cpp:331-334)
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

constexpr int kT = 256;

// One element per thread; x has n * k elements, k % 32 == 0.
__global__ void k_quantize_q8(const float* __restrict__ x, int64_t total, BlockQ8* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const float v[1] = {x[i]};
  quantize_block_lanes_n<1>(v, (int)(i & 31), y + i / 32);
}

__global__ void k_quantize_i8(const float* __restrict__ x, int n, int8_t* __restrict__ q, float* __restrict__ d) {
  const int row = blockIdx.x;
  const float* xr = x + (int64_t)row * n;
  __shared__ float red[kT];
  float amax = 0.0f;
  for (int i = threadIdx.x; i < n; i += kT) amax = fmaxf(amax, fabsf(xr[i]));
  red[threadIdx.x] = amax;
  __syncthreads();
  for (int st = kT / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
    __syncthreads();
  }
  const float dd = red[0] / 127.0f, id = dd != 0.0f ? 1.0f / dd : 0.0f;
  for (int i = threadIdx.x; i < n; i += kT) q[(int64_t)row * n + i] = (int8_t)(int)__builtin_rintf(xr[i] * id);
  if (threadIdx.x == 0) d[row] = dd;
}

// rmsnorm of one row per workgroup; the sum of squares follows kern::dot_f32 (kernels_avx512.cpp:82-89): 16 lane
// accumulators, each a sequential fma chain over the elements i = l (mod 16), then the halving tree.
// Thread t owns the 16-element chunks t and t + 256 of the row (n <= 8192), held in registers from one round of 16-byte
// loads. The row goes to LDS transposed (chain lane l's elements contiguous), so a chain reads four elements per
// 16-byte access; the chain loads the next 32 elements while it runs the current 32. A chunk is half a Q8 block, so the
// quantized output needs one lane exchange per block.
template <bool kQuant>
__global__ __launch_bounds__(kT) void k_rmsnorm(const float* __restrict__ x, const int32_t* __restrict__ rows_idx,
                                                const float* __restrict__ w, int n, float eps, float* __restrict__ y,
                                                BlockQ8* __restrict__ xq) {
  extern __shared__ float4 sm4[];
  const int per = n / 16, tstride = sumsq_tstride(per);
  float* tr = reinterpret_cast<float*>(sm4);  // [16][tstride]; element i at (i % 16, i / 16)
  __shared__ float scale;
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* xr = x + (int64_t)(rows_idx ? rows_idx[r] : r) * n;
  constexpr int kPass = 2;
  float v[kPass][16], wv[kPass][16];
#pragma unroll
  for (int p = 0; p < kPass; ++p) {
    const int c16 = tid + p * kT;
    if (c16 < per) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 a = *reinterpret_cast<const float4*>(xr + 16 * c16 + 4 * k);
        const float4 b = *reinterpret_cast<const float4*>(w + 16 * c16 + 4 * k);
        v[p][4 * k] = a.x, v[p][4 * k + 1] = a.y, v[p][4 * k + 2] = a.z, v[p][4 * k + 3] = a.w;
        wv[p][4 * k] = b.x, wv[p][4 * k + 1] = b.y, wv[p][4 * k + 2] = b.z, wv[p][4 * k + 3] = b.w;
      }
    }
  }
  const int padded = sumsq_padded(per);
#pragma unroll
  for (int p = 0; p < kPass; ++p) {
    const int c16 = tid + p * kT;
    if (c16 < padded) {
#pragma unroll
      for (int c = 0; c < 16; ++c) tr[c * tstride + c16] = c16 < per ? v[p][c] : 0.0f;
    }
  }
  __syncthreads();
  if (tid < 16) {
    float acc = sumsq_lane_chain(tr + tid * tstride, per);
    acc = reduce16_lanes(acc);
    if (tid == 0) scale = 1.0f / sqrtf(acc / (float)n + eps);
  }
  __syncthreads();
  const float s = scale;
#pragma unroll
  for (int p = 0; p < kPass; ++p) {
    const int c16 = tid + p * kT;
    if (p * kT >= per) break;  // uniform: no chunk of this pass is in the row
    float yv[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) yv[c] = v[p][c] * s * wv[p][c];
    if (!kQuant) {
      if (c16 < per) {
        float* yr = y + (int64_t)r * n + 16 * c16;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          *reinterpret_cast<float4*>(yr + 4 * k) = make_float4(yv[4 * k], yv[4 * k + 1], yv[4 * k + 2], yv[4 * k + 3]);
      }
    } else {
      // n % 32 == 0, so both halves of a block are in the row or neither is.
      quantize_half_block(yv, c16 & 1, c16 < per, xq + (int64_t)r * (n / 32) + c16 / 2);
    }
  }
}

__global__ void k_silu_mul(int64_t n, float* __restrict__ g, const float* __restrict__ u) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = g[i];
  const float e = exp512(0.0f - x);
  g[i] = (x / (1.0f + e)) * u[i];
}

// Rows [gate(n) | up(n)] at stride 2n: gate = silu(gate) * up in place (kern::silu_mul per token).
__global__ void k_silu_mul_rows(float* __restrict__ gu, int64_t n, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  float* g = gu + (i / n) * 2 * n + i % n;
  const float x = *g;
  const float e = exp512(0.0f - x);
  *g = (x / (1.0f + e)) * g[n];
}

// gu row: [gate(n) | up(n)], or gate/up interleaved by 4 (row 8k + j: gate 4k + j for j < 4, else up 4k + j - 4)
// -> silu(gate) * up, quantized; one element per thread, n % 32 == 0.
// Row r (blockIdx.y), four consecutive outputs c .. c + 3 per thread (16-byte loads of gate and up), so that a Q8
// block is 8 consecutive lanes. Per element the arithmetic of kernels_avx512.cpp:271-280.
__global__ void k_silu_mul_q8(const float* __restrict__ gu, int64_t n, int interleave4, BlockQ8* __restrict__ xq) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // outputs 4q .. 4q + 3 of the row
  if (q >= n / 4) return;  // n % 32 == 0: whole 8-lane blocks leave together
  const int64_t r = blockIdx.y;
  const float* row = gu + r * 2 * n;
  // gate values 4q .. 4q + 3 and their up values: [gate | up] rows, or rows interleaved by 4 (8q: gate, 8q + 4: up)
  const float4 g4 = *reinterpret_cast<const float4*>(row + (interleave4 ? 8 * q : 4 * q));
  const float4 u4 = *reinterpret_cast<const float4*>(row + (interleave4 ? 8 * q + 4 : n + 4 * q));
  const float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w};
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float e = exp512(0.0f - g[k]);
    v[k] = (g[k] / (1.0f + e)) * u[k];
  }
  quantize_block_lanes_n<4>(v, (int)(q & 7), xq + r * (n / 32) + q / 8);
}

__global__ void k_add(int64_t n, float* __restrict__ x, const float* __restrict__ h) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] + h[i];
}

__global__ void k_fill(uint8_t* p, int v, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = (uint8_t)v;
}

// Four int32 words from the kernel arguments (small per-call metadata written in stream order, without a host copy).
__global__ void k_put4(int32_t* p, int a, int b, int c, int d) {
  if (threadIdx.x == 0) *reinterpret_cast<int4*>(p) = make_int4(a, b, c, d);
}

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& sc, int& m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// One thread per output element; every product below is exact in fp32, so the value has one rounding at most.
__global__ void k_dequant(int type, const uint8_t* __restrict__ src, size_t row_bytes, const int32_t* __restrict__ ids,
                          int64_t k, int64_t total, float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t t = i / k, e = i % k;
  const uint8_t* row = src + (size_t)ids[t] * row_bytes;
  float v = 0.0f;
  if (type == kF32) {
    v = reinterpret_cast<const float*>(row)[e];
  } else if (type == kF16) {
    v = half_to_float(reinterpret_cast<const uint16_t*>(row)[e]);
  } else if (type == kBF16) {
    v = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(row)[e] << 16);
  } else if (type == kQ5_K) {
    const uint8_t* b = row + (e / 256) * 176;
    const int within = (int)(e % 256), j = within / 32, l = within % 32;
    const float d = half_to_float((uint16_t)(b[0] | (b[1] << 8))), dmin = half_to_float((uint16_t)(b[2] | (b[3] << 8)));
    int sc, m;
    scale_min_k4(j, b + 4, sc, m);
    const uint8_t qb = b[48 + 32 * (j / 2) + l];
    const int q = ((j & 1) ? qb >> 4 : qb & 0xF) | (((b[16 + l] >> j) & 1) << 4);
    v = d * (float)sc * (float)q - dmin * (float)m;
  } else if (type == kQ8_0) {
    const uint8_t* b = row + (e / 32) * 34;
    v = half_to_float((uint16_t)(b[0] | (b[1] << 8))) * (float)(int8_t)b[2 + e % 32];
  } else if (type == kQ4_K) {
    const uint8_t* b = row + (e / 256) * 144;
    const int within = (int)(e % 256), j = within / 32, l = within % 32;
    const float d = half_to_float((uint16_t)(b[0] | (b[1] << 8))), dmin = half_to_float((uint16_t)(b[2] | (b[3] << 8)));
    int sc, m;
    scale_min_k4(j, b + 4, sc, m);
    const uint8_t qb = b[16 + 32 * (j / 2) + l];
    const int q = (j & 1) ? qb >> 4 : qb & 0xF;
    v = d * (float)sc * (float)q - dmin * (float)m;
  } else if (type == kQ6_K) {
    const uint8_t* b = row + (e / 256) * 210;
    const int k2 = (int)(e % 256), nn = k2 / 128, rem = k2 % 128, c = rem / 32, l = rem % 32;
    const uint8_t lo = b[64 * nn + l + (c & 1) * 32];
    const int nib = c >= 2 ? lo >> 4 : lo & 0xF;
    const int hb = (b[128 + 32 * nn + l] >> (2 * c)) & 3;
    const int q = (nib | (hb << 4)) - 32;
    const float d = half_to_float((uint16_t)(b[208] | (b[209] << 8)));
    v = d * (float)(int8_t)b[192 + k2 / 16] * (float)q;
  }
  dst[i] = v;
}

unsigned grid_for(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

}  // namespace

void quantize_q8(hipStream_t s, const float* x, int n, int64_t k, BlockQ8* xq) {
  require(k % 32 == 0, "quantize_q8: k must be a multiple of 32");
  const int64_t total = (int64_t)n * k;
  if (total == 0) return;
  hipLaunchKernelGGL(k_quantize_q8, dim3(grid_for(total, kT)), dim3(kT), 0, s, x, total, xq);
  check_launch("quantize_q8");
}

void quantize_i8_rows(hipStream_t s, const float* x, int rows, int n, int8_t* q, float* d) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_quantize_i8, dim3(rows), dim3(kT), 0, s, x, n, q, d);
  check_launch("quantize_i8");
}

void dequantize_rows(hipStream_t s, int type, const void* src, size_t row_bytes, const int32_t* ids, int n, int64_t k,
                     float* dst) {
  require(type == kF32 || type == kF16 || type == kBF16 || type == kQ8_0 || type == kQ4_K || type == kQ5_K ||
              type == kQ6_K,
          "dequantize: unsupported type");
  const int64_t total = (int64_t)n * k;
  if (total == 0) return;
  hipLaunchKernelGGL(k_dequant, dim3(grid_for(total, kT)), dim3(kT), 0, s, type, static_cast<const uint8_t*>(src),
                     row_bytes, ids, k, total, dst);
  check_launch("dequantize_rows");
}

static size_t rmsnorm_lds(int n) { return 16 * (size_t)sumsq_tstride(n / 16) * sizeof(float); }

void rmsnorm(hipStream_t s, const float* x, const float* w, int rows, int n, float eps, float* y,
             const int32_t* rows_idx) {
  if (rows <= 0) return;
  require(n % 16 == 0 && n <= 8192, "rmsnorm: n must be a multiple of 16, <= 8192");
  hipLaunchKernelGGL(k_rmsnorm<false>, dim3(rows), dim3(kT), rmsnorm_lds(n), s, x, rows_idx, w, n, eps, y, nullptr);
  check_launch("rmsnorm");
}

void rmsnorm_q8(hipStream_t s, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                BlockQ8* xq) {
  if (rows <= 0) return;
  require(n % 32 == 0 && n <= 8192, "rmsnorm_q8: n must be a multiple of 32, <= 8192");
  hipLaunchKernelGGL(k_rmsnorm<true>, dim3(rows), dim3(kT), rmsnorm_lds(n), s, x, rows_idx, w, n, eps, nullptr, xq);
  check_launch("rmsnorm_q8");
}

void silu_mul_rows(hipStream_t s, float* gu, int rows, int64_t n) {
  if (rows <= 0 || n <= 0) return;
  if (n % 16) throw Error(MK_ERR_UNSUPPORTED, "silu_mul: n must be a multiple of 16");
  const int64_t total = (int64_t)rows * n;
  hipLaunchKernelGGL(k_silu_mul_rows, dim3(grid_for(total, kT)), dim3(kT), 0, s, gu, n, total);
  check_launch("silu_mul_rows");
}

void silu_mul(hipStream_t s, int64_t n, float* g, const float* u) {
  // The reference's scalar tail (n % 16 != 0) calls libm's expf, which has no bit-exact device counterpart.
  if (n <= 0) return;
  if (n % 16) throw Error(MK_ERR_UNSUPPORTED, "silu_mul: n must be a multiple of 16");
  hipLaunchKernelGGL(k_silu_mul, dim3(grid_for(n, kT)), dim3(kT), 0, s, n, g, u);
  check_launch("silu_mul");
}

void silu_mul_q8(hipStream_t s, const float* gu, int rows, int64_t n, BlockQ8* xq, bool interleave4) {
  require(n % 32 == 0, "silu_mul_q8: n must be a multiple of 32");
  require(rows <= 65535, "silu_mul_q8: at most 65535 rows per call");
  if (rows <= 0 || n == 0) return;
  hipLaunchKernelGGL(k_silu_mul_q8, dim3(grid_for(n / 4, kT), rows), dim3(kT), 0, s, gu, n, interleave4 ? 1 : 0, xq);
  check_launch("silu_mul_q8");
}

void add(hipStream_t s, int64_t n, float* x, const float* h) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_add, dim3(grid_for(n, kT)), dim3(kT), 0, s, n, x, h);
  check_launch("add");
}

void put4(hipStream_t s, int32_t* p, int a, int b, int c, int d) {
  hipLaunchKernelGGL(k_put4, dim3(1), dim3(64), 0, s, p, a, b, c, d);
  check_launch("put4");
}

void fill(hipStream_t s, void* p, int v, size_t n) {
  if (n == 0) return;
  hipLaunchKernelGGL(k_fill, dim3(grid_for((int64_t)n, kT)), dim3(kT), 0, s, static_cast<uint8_t*>(p), v, n);
  check_launch("fill");
}

}  // namespace mk
