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

// One 32-value block of f32 activations -> BlockQ8, in one thread.
__device__ __forceinline__ void quantize_block(const float* v, BlockQ8* out) {
  float amax = 0.0f;
#pragma unroll
  for (int l = 0; l < 32; ++l) amax = fmaxf(amax, fabsf(v[l]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int s0 = 0, s1 = 0;
  int packed[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int l = 4 * w + b;
      const int q = cvt_rne(v[l] * id);
      if (l < 16)
        s0 += q;
      else
        s1 += q;
      word |= (uint32_t)(uint8_t)(int8_t)sat8(q) << (8 * b);
    }
    packed[w] = (int)word;
  }
  int* o = reinterpret_cast<int*>(out);
  o[0] = __float_as_int(d);
  o[1] = (int)((uint32_t)(uint16_t)(int16_t)s0 | ((uint32_t)(uint16_t)(int16_t)s1 << 16));
#pragma unroll
  for (int w = 0; w < 8; ++w) o[2 + w] = packed[w];
}

__global__ void k_quantize_q8(const float* __restrict__ x, int64_t nblocks, BlockQ8* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  float v[32];
  const float4* src = reinterpret_cast<const float4*>(x + i * 32);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const float4 f = src[w];
    v[4 * w] = f.x;
    v[4 * w + 1] = f.y;
    v[4 * w + 2] = f.z;
    v[4 * w + 3] = f.w;
  }
  quantize_block(v, y + i);
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
template <bool kQuant>
__global__ void k_rmsnorm(const float* __restrict__ x, const int32_t* __restrict__ rows_idx,
                          const float* __restrict__ w, int n, float eps, float* __restrict__ y,
                          BlockQ8* __restrict__ xq) {
  extern __shared__ float row[];  // n floats
  __shared__ float scale;
  const int r = blockIdx.x;
  const float* xr = x + (int64_t)(rows_idx ? rows_idx[r] : r) * n;
  for (int i = threadIdx.x; i < n; i += kT) row[i] = xr[i];
  __syncthreads();
  if (threadIdx.x < 16) {
    const int l = threadIdx.x;
    float acc = 0.0f;
    for (int i = l; i < n; i += 16) acc = fma_(row[i], row[i], acc);
    acc = reduce16_lanes(acc);
    if (l == 0) scale = 1.0f / sqrtf(acc / (float)n + eps);
  }
  __syncthreads();
  const float s = scale;
  if (!kQuant) {
    for (int i = threadIdx.x; i < n; i += kT) y[(int64_t)r * n + i] = row[i] * s * w[i];
    return;
  }
  for (int i = threadIdx.x; i < n; i += kT) row[i] = row[i] * s * w[i];
  __syncthreads();
  for (int b = threadIdx.x; b < n / 32; b += kT) quantize_block(row + 32 * b, xq + (int64_t)r * (n / 32) + b);
}

__global__ void k_silu_mul(int64_t n, float* __restrict__ g, const float* __restrict__ u) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = g[i];
  const float e = exp512(0.0f - x);
  g[i] = (x / (1.0f + e)) * u[i];
}

// gu row: [gate(n) | up(n)] -> silu(gate) * up, quantized; one thread per 32-value block.
__global__ void k_silu_mul_q8(const float* __restrict__ gu, int64_t n, int64_t nblocks, BlockQ8* __restrict__ xq) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  const int64_t per = n / 32, r = i / per, b = i % per;
  const float* g = gu + r * 2 * n + b * 32;
  const float* u = g + n;
  float v[32];
#pragma unroll
  for (int l = 0; l < 32; ++l) {
    const float x = g[l];
    const float e = exp512(0.0f - x);
    v[l] = (x / (1.0f + e)) * u[l];
  }
  quantize_block(v, xq + i);
}

__global__ void k_add(int64_t n, float* __restrict__ x, const float* __restrict__ h) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] + h[i];
}

__global__ void k_fill(uint8_t* p, int v, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = (uint8_t)v;
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
  const int64_t nb = (int64_t)n * (k / 32);
  if (nb == 0) return;
  hipLaunchKernelGGL(k_quantize_q8, dim3(grid_for(nb, kT)), dim3(kT), 0, s, x, nb, xq);
  check_launch("quantize_q8");
}

void quantize_i8_rows(hipStream_t s, const float* x, int rows, int n, int8_t* q, float* d) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_quantize_i8, dim3(rows), dim3(kT), 0, s, x, n, q, d);
  check_launch("quantize_i8");
}

void dequantize_rows(hipStream_t s, int type, const void* src, size_t row_bytes, const int32_t* ids, int n, int64_t k,
                     float* dst) {
  require(type == kF32 || type == kQ8_0 || type == kQ4_K || type == kQ6_K, "dequantize: unsupported type");
  const int64_t total = (int64_t)n * k;
  if (total == 0) return;
  hipLaunchKernelGGL(k_dequant, dim3(grid_for(total, kT)), dim3(kT), 0, s, type, static_cast<const uint8_t*>(src),
                     row_bytes, ids, k, total, dst);
  check_launch("dequantize_rows");
}

void rmsnorm(hipStream_t s, const float* x, const float* w, int rows, int n, float eps, float* y) {
  if (rows <= 0) return;
  require(n % 16 == 0, "rmsnorm: n must be a multiple of 16");
  hipLaunchKernelGGL(k_rmsnorm<false>, dim3(rows), dim3(kT), n * sizeof(float), s, x, nullptr, w, n, eps, y, nullptr);
  check_launch("rmsnorm");
}

void rmsnorm_q8(hipStream_t s, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                BlockQ8* xq) {
  if (rows <= 0) return;
  require(n % 32 == 0, "rmsnorm_q8: n must be a multiple of 32");
  hipLaunchKernelGGL(k_rmsnorm<true>, dim3(rows), dim3(kT), n * sizeof(float), s, x, rows_idx, w, n, eps, nullptr, xq);
  check_launch("rmsnorm_q8");
}

void silu_mul(hipStream_t s, int64_t n, float* g, const float* u) {
  // The reference's scalar tail (n % 16 != 0) calls libm's expf, which has no bit-exact device counterpart.
  if (n <= 0) return;
  if (n % 16) throw Error(MK_ERR_UNSUPPORTED, "silu_mul: n must be a multiple of 16");
  hipLaunchKernelGGL(k_silu_mul, dim3(grid_for(n, kT)), dim3(kT), 0, s, n, g, u);
  check_launch("silu_mul");
}

void silu_mul_q8(hipStream_t s, const float* gu, int rows, int64_t n, BlockQ8* xq) {
  require(n % 32 == 0, "silu_mul_q8: n must be a multiple of 32");
  const int64_t nb = (int64_t)rows * (n / 32);
  if (nb == 0) return;
  hipLaunchKernelGGL(k_silu_mul_q8, dim3(grid_for(nb, kT)), dim3(kT), 0, s, gu, n, nb, xq);
  check_launch("silu_mul_q8");
}

void add(hipStream_t s, int64_t n, float* x, const float* h) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_add, dim3(grid_for(n, kT)), dim3(kT), 0, s, n, x, h);
  check_launch("add");
}

void fill(hipStream_t s, void* p, int v, size_t n) {
  if (n == 0) return;
  hipLaunchKernelGGL(k_fill, dim3(grid_for((int64_t)n, kT)), dim3(kT), 0, s, static_cast<uint8_t*>(p), v, n);
  check_launch("fill");
}

}  // namespace mk
