/*
 * CPU oracle for the malkin token loop — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates the reference's AVX-512 arithmetic in plain C. An AVX-512 register is a float[16]; lane-wise ops map to
 * scalar ops on each element, _mm512_reduce_add_ps to or_reduce16. Build with -ffp-contract=off: every fused
 * multiply-add of the reference is an explicit fmaf() here, and nothing else is fused.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ---------------------------------------------------------------- scalars */

/* quant.cpp:21-25 (_Float16 -> float, exact) */
float or_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = sign;
    } else { /* subnormal: renormalise */
      int sh = 0;
      uint32_t mm = m;
      while (!(mm & 0x400)) mm <<= 1, ++sh;
      u = sign | ((uint32_t)(127 - 15 - sh + 1) << 23) | ((mm & 0x3FF) << 13);
    }
  } else if (e == 31) {
    u = sign | 0x7F800000u | (m << 13);
  } else {
    u = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* quant.cpp:27-32 (float -> _Float16, round to nearest even) */
uint16_t or_fp32_to_fp16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t a = u & 0x7FFFFFFF;
  if (a > 0x7F800000) return sign | 0x7E00; /* NaN */
  if (a >= 0x477FF000) return sign | 0x7C00; /* rounds to >= 65520: inf */
  if (a < 0x38800000) { /* below the smallest normal half: subnormal or zero */
    if (a < 0x33000000) return sign; /* < 2^-25: rounds to 0 (2^-25 exactly ties to even 0) */
    const uint32_t e = a >> 23, mant = (a & 0x7FFFFF) | 0x800000;
    const int shift = 126 - (int)e; /* value = mant * 2^(e-150); half subnormal unit 2^-24 */
    uint32_t q = mant >> (shift), rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return sign | (uint16_t)q;
  }
  uint32_t h = ((a >> 13) - (112u << 10));
  const uint32_t rem = a & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
  return sign | (uint16_t)h;
}

/* gguf.cpp:60-95 */
size_t or_row_size(int type, int64_t k) {
  switch (type) {
    case OR_F32:
      return (size_t)k * 4;
    case OR_F16:
    case OR_BF16:
      return (size_t)k * 2;
    case OR_Q8_0:
      return (size_t)(k / 32) * 34;
    case OR_Q4_K:
      return (size_t)(k / 256) * 144;
    case OR_Q5_K:
      return (size_t)(k / 256) * 176;
    case OR_Q6_K:
      return (size_t)(k / 256) * 210;
    default:
      return 0;
  }
}

static uint16_t ld16(const uint8_t* p) {
  uint16_t v;
  memcpy(&v, p, 2);
  return v;
}

/* kernels.h:18-26 */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* --------------------------------------------------------------- vectors */

float or_reduce16(const float* v) {
  float a[8], b[4], c[2];
  for (int i = 0; i < 8; ++i) a[i] = v[i] + v[i + 8];
  for (int i = 0; i < 4; ++i) b[i] = a[i] + a[i + 4];
  for (int i = 0; i < 2; ++i) c[i] = b[i] + b[i + 2];
  return c[0] + c[1];
}

/* _mm512_cvtps_epi32 under the default MXCSR: round to nearest even, out of range / NaN -> INT32_MIN. */
static int32_t cvt_rne(float x) {
  if (!(x >= -2147483648.0f && x < 2147483648.0f)) return INT32_MIN;
  return (int32_t)rintf(x);
}

static int8_t sat8(int32_t v) { return (int8_t)(v > 127 ? 127 : v < -128 ? -128 : v); }

/* kernels_avx512.cpp:66-80 */
void or_quantize_row_q8(const float* x, or_block_q8* y, int64_t k) {
  for (int64_t i = 0; i < k / 32; ++i, x += 32) {
    float amax = 0.0f;
    for (int l = 0; l < 32; ++l) {
      const float a = fabsf(x[l]);
      amax = a > amax ? a : amax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int32_t s0 = 0, s1 = 0;
    for (int l = 0; l < 32; ++l) {
      const int32_t q = cvt_rne(x[l] * id);
      y[i].qs[l] = sat8(q);
      if (l < 16)
        s0 += q;
      else
        s1 += q;
    }
    y[i].d = d;
    y[i].s[0] = (int16_t)s0;
    y[i].s[1] = (int16_t)s1;
  }
}

/* quant.cpp:134-140 */
float or_quantize_i8(const float* x, int n, int8_t* q) {
  float amax = 0.0f;
  for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(x[i]));
  const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int i = 0; i < n; ++i) q[i] = (int8_t)lrintf(x[i] * id);
  return d;
}

/* quant.cpp:70-128, 142-169 */
int or_dequantize_row(int type, const void* src, float* y, int64_t k) {
  const uint8_t* b = (const uint8_t*)src;
  switch (type) {
    case OR_F32:
      memcpy(y, src, (size_t)k * 4);
      return 0;
    case OR_F16:
      for (int64_t i = 0; i < k; ++i) y[i] = or_fp16_to_fp32(ld16(b + 2 * i));
      return 0;
    case OR_BF16:
      for (int64_t i = 0; i < k; ++i) {
        const uint32_t u = (uint32_t)ld16(b + 2 * i) << 16;
        memcpy(y + i, &u, 4);
      }
      return 0;
    case OR_Q8_0:
      for (int64_t i = 0; i < k / 32; ++i, b += 34) {
        const float d = or_fp16_to_fp32(ld16(b));
        for (int l = 0; l < 32; ++l) y[i * 32 + l] = d * (float)(int8_t)b[2 + l];
      }
      return 0;
    case OR_Q4_K:
    case OR_Q5_K: {
      const int high = type == OR_Q5_K;
      for (int64_t i = 0; i < k / 256; ++i, b += high ? 176 : 144) {
        const float d = or_fp16_to_fp32(ld16(b)), dmin = or_fp16_to_fp32(ld16(b + 2));
        const uint8_t* sc = b + 4;
        const uint8_t* qh = b + 16;
        const uint8_t* q = b + (high ? 48 : 16);
        for (int j = 0; j < 4; ++j, q += 32) {
          int s0, m0, s1, m1;
          scale_min_k4(2 * j, sc, &s0, &m0);
          scale_min_k4(2 * j + 1, sc, &s1, &m1);
          /* d * s * q and dmin * m are exact products; the difference is rounded once either way. */
          for (int l = 0; l < 32; ++l) {
            const int qq = (q[l] & 0xF) + (high ? ((qh[l] >> (2 * j)) & 1) << 4 : 0);
            *y++ = d * (float)s0 * (float)qq - dmin * (float)m0;
          }
          for (int l = 0; l < 32; ++l) {
            const int qq = (q[l] >> 4) + (high ? ((qh[l] >> (2 * j + 1)) & 1) << 4 : 0);
            *y++ = d * (float)s1 * (float)qq - dmin * (float)m1;
          }
        }
      }
      return 0;
    }
    case OR_Q6_K:
      for (int64_t i = 0; i < k / 256; ++i, b += 210) {
        const uint8_t* ql = b;
        const uint8_t* qh = b + 128;
        const int8_t* sc = (const int8_t*)(b + 192);
        const float d = or_fp16_to_fp32(ld16(b + 208));
        for (int n = 0; n < 2; ++n, ql += 64, qh += 32, sc += 8, y += 128) {
          for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
          }
        }
      }
      return 0;
    default:
      return -1;
  }
}

/* kernels_avx512.cpp:82-89 (the scalar tail is contracted by clang: s = fma(w, x, s)) */
float or_dot_f32(int64_t k, const float* w, const float* x) {
  float acc[16] = {0};
  int64_t i = 0;
  for (; i + 16 <= k; i += 16)
    for (int l = 0; l < 16; ++l) acc[l] = fmaf(w[i + l], x[i + l], acc[l]);
  float s = or_reduce16(acc);
  for (; i < k; ++i) s = fmaf(w[i], x[i], s);
  return s;
}

/* ------------------------------------------------------------ row path
 * vec_dot (quant.cpp:171-191): one weight row . one activation row, used by matmul's row path (quant.cpp:330-351)
 * for F32/F16/BF16 weights and, under MALKIN_NO_PACK, for the quantized types. Each restates the register layout of
 * its AVX-512 kernel: lane l of the 16-float accumulator, then the halving tree. Scalar expressions follow clang's
 * default contraction (-ffp-contract=on: a*b + c in one expression becomes one fma, the left product first). */

static float bf16_to_fp32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* kernels_avx512.cpp:91-107: dot_f16 / dot_bf16, the dot_f32 lanes over converted weights. */
static float dot_half(int bf, int64_t k, const uint8_t* w, const float* x) {
  float acc[16] = {0};
  int64_t i = 0;
  for (; i + 16 <= k; i += 16)
    for (int l = 0; l < 16; ++l) {
      const uint16_t h = ld16(w + 2 * (i + l));
      acc[l] = fmaf(bf ? bf16_to_fp32(h) : or_fp16_to_fp32(h), x[i + l], acc[l]);
    }
  float s = or_reduce16(acc);
  for (; i < k; ++i) {
    const uint16_t h = ld16(w + 2 * i);
    s = fmaf(bf ? bf16_to_fp32(h) : or_fp16_to_fp32(h), x[i], s);
  }
  return s;
}

/* Exact int dot of n int8 weights with n int8 activations. */
static int32_t idot8(const int8_t* w, const int8_t* x, int n) {
  int32_t s = 0;
  for (int e = 0; e < n; ++e) s += (int32_t)w[e] * x[e];
  return s;
}

/* kernels_avx512.cpp:110-137: blocks in pairs, lanes 0-7 the first block's 4-byte groups, lanes 8-15 the second's;
   an odd last block is added after the tree, s += float(dot) * dw * dx. */
static float dot_q8_0_rows(int64_t k, const uint8_t* w, const or_block_q8* x) {
  const int64_t nb = k / 32;
  float acc[16] = {0};
  int64_t i = 0;
  for (; i + 2 <= nb; i += 2)
    for (int l = 0; l < 16; ++l) {
      const int64_t b = i + l / 8;
      const uint8_t* blk = w + b * 34;
      const int32_t dp = idot8((const int8_t*)blk + 2 + 4 * (l % 8), x[b].qs + 4 * (l % 8), 4);
      acc[l] = fmaf((float)dp, or_fp16_to_fp32(ld16(blk)) * x[b].d, acc[l]);
    }
  float s = or_reduce16(acc);
  for (; i < nb; ++i) {
    const uint8_t* blk = w + i * 34;
    const int32_t dp = idot8((const int8_t*)blk + 2, x[i].qs, 32);
    s = fmaf((float)dp * or_fp16_to_fp32(ld16(blk)), x[i].d, s);
  }
  return s;
}

/* kernels_avx512.cpp:31-64 (dot_qk_45): per super-block and sub-block pair j, lanes 0-7 the 4-value groups of
   sub-block 2j (low nibbles), lanes 8-15 those of 2j + 1 (high nibbles); Q5_K adds the high bit of each value.
   mins is one scalar chain: mins = fma(dmin, fma(m0 * dx0, S0, (m1 * dx1) * S1), mins). */
static float dot_qk_45_rows(int high, int64_t k, const uint8_t* w, const or_block_q8* x) {
  const size_t bytes = high ? 176 : 144;
  float acc[16] = {0};
  float mins = 0.0f;
  for (int64_t i = 0; i < k / 256; ++i, w += bytes, x += 8) {
    const float d = or_fp16_to_fp32(ld16(w)), dmin = or_fp16_to_fp32(ld16(w + 2));
    const uint8_t* qh = w + 16;
    const uint8_t* q = w + (high ? 48 : 16);
    for (int j = 0; j < 4; ++j, q += 32) {
      int s0, m0, s1, m1;
      scale_min_k4(2 * j, w + 4, &s0, &m0);
      scale_min_k4(2 * j + 1, w + 4, &s1, &m1);
      const or_block_q8* x0 = x + 2 * j;
      const or_block_q8* x1 = x + 2 * j + 1;
      const float sc0 = d * (float)s0 * x0->d, sc1 = d * (float)s1 * x1->d;
      for (int l = 0; l < 16; ++l) {
        const int hi = l >= 8, g = l % 8;
        int32_t dp = 0;
        for (int e = 0; e < 4; ++e) {
          const int idx = 4 * g + e;
          int v = hi ? q[idx] >> 4 : q[idx] & 0xF;
          if (high) v |= ((qh[idx] >> (2 * j + hi)) & 1) << 4;
          dp += v * (hi ? x1 : x0)->qs[idx];
        }
        acc[l] = fmaf((float)dp, hi ? sc1 : sc0, acc[l]);
      }
      const float in = fmaf((float)m0 * x0->d, (float)(x0->s[0] + x0->s[1]), ((float)m1 * x1->d) * (float)(x1->s[0] + x1->s[1]));
      mins = fmaf(dmin, in, mins);
    }
  }
  return or_reduce16(acc) - mins;
}

/* kernels_avx512.cpp:142-171 (dot_q6_k): per 128-value half, lanes 0-7 / 8-15 the 4-value groups of its first /
   second 32 values (unsigned q, 0..63) times the 16-value sub-block scale, then the third / fourth 32 values; the
   q - 32 offset comes back through bias = fma(d * dx * 32, sc0 * s0 + sc1 * s1, bias). */
static float dot_q6_k_rows(int64_t k, const uint8_t* w, const or_block_q8* x) {
  float acc[16] = {0};
  float bias = 0.0f;
  for (int64_t i = 0; i < k / 256; ++i, w += 210) {
    const uint8_t* ql = w;
    const uint8_t* qh = w + 128;
    const int8_t* sc = (const int8_t*)(w + 192);
    const float d = or_fp16_to_fp32(ld16(w + 208));
    for (int n = 0; n < 2; ++n, ql += 64, qh += 32, sc += 8, x += 4) {
      /* q of value v (0..127) of this half: groups of 32 per (low/high nibble, first/second 32 bytes) */
      int q[128];
      for (int l = 0; l < 32; ++l) {
        q[l] = (ql[l] & 0xF) | ((qh[l] & 3) << 4);
        q[32 + l] = (ql[32 + l] & 0xF) | (((qh[l] >> 2) & 3) << 4);
        q[64 + l] = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
        q[96 + l] = (ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4);
      }
      for (int pass = 0; pass < 2; ++pass)
        for (int l = 0; l < 16; ++l) {
          const int grp = 2 * pass + l / 8;  /* 32-value group: x block grp of this half */
          int32_t dp = 0;
          for (int e = 0; e < 4; ++e) dp += q[32 * grp + 4 * (l % 8) + e] * x[grp].qs[4 * (l % 8) + e];
          const int32_t scl = sc[4 * pass + l / 4];
          acc[l] = fmaf((float)(dp * scl), d * x[grp].d, acc[l]);
        }
      for (int g = 0; g < 4; ++g)
        bias = fmaf(d * x[g].d * 32.0f, (float)(sc[2 * g] * x[g].s[0] + sc[2 * g + 1] * x[g].s[1]), bias);
    }
  }
  return or_reduce16(acc) - bias;
}

float or_vec_dot(int type, int64_t k, const uint8_t* w, const float* x, const or_block_q8* xq) {
  switch (type) {
    case OR_F32:
      return or_dot_f32(k, (const float*)w, x);
    case OR_F16:
      return dot_half(0, k, w, x);
    case OR_BF16:
      return dot_half(1, k, w, x);
    case OR_Q8_0:
      return dot_q8_0_rows(k, w, xq);
    case OR_Q4_K:
      return dot_qk_45_rows(0, k, w, xq);
    case OR_Q5_K:
      return dot_qk_45_rows(1, k, w, xq);
    case OR_Q6_K:
      return dot_q6_k_rows(k, w, xq);
    default:
      return NAN;
  }
}

/* quant.cpp:330-351: y[t][r] = vec_dot(row r, token t). */
int or_matmul_rows(int type, const uint8_t* w, size_t row_bytes, int64_t rows, int64_t cols, const float* x,
                   const or_block_q8* xq, int n, float* y, int64_t y_stride) {
  if (or_row_size(type, cols) == 0) return -1;
  for (int t = 0; t < n; ++t)
    for (int64_t r = 0; r < rows; ++r)
      y[(int64_t)t * y_stride + r] = or_vec_dot(type, cols, w + (size_t)r * row_bytes, x + (int64_t)t * cols,
                                                xq ? xq + (int64_t)t * (cols / 32) : NULL);
  return 0;
}

/* kernels_avx512.cpp:186-202: max(x, -87), Cody-Waite reduction, degree-6 Taylor, scalef. */
float or_exp(float x) {
  x = fmaxf(x, -87.0f); /* _mm512_max_ps(x, -87): NaN x gives -87, as fmaxf */
  const float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.0f / 720.0f;
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  /* _mm512_scalef_ps(p, n) = p * 2^floor(n), n integral here */
  if (isnan(n) || isnan(p)) return NAN;
  if (n > 300.0f) return p == 0.0f ? p : copysignf(INFINITY, p);
  if (n < -300.0f) return copysignf(0.0f, p);
  return ldexpf(p, (int)n);
}

/* kernels_avx512.cpp:205-226 */
float or_softmax_inplace(float* s, int n) {
  float mx = -INFINITY;
  for (int i = 0; i < n; ++i) mx = fmaxf(mx, s[i]);
  float sum[16] = {0};
  for (int i = 0; i < n; ++i) {
    const float e = or_exp(s[i] - mx);
    s[i] = e;
    sum[i % 16] = sum[i % 16] + e;
  }
  return 1.0f / or_reduce16(sum);
}

/* kernels_avx512.cpp:271-280 */
void or_silu_mul(int64_t n, float* g, const float* u) {
  int64_t i = 0;
  for (; i + 16 <= n; i += 16) {
    for (int l = 0; l < 16; ++l) {
      const float x = g[i + l];
      const float e = or_exp(0.0f - x);
      g[i + l] = (x / (1.0f + e)) * u[i + l];
    }
  }
  for (; i < n; ++i) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* model.cpp:46-49 */
void or_rmsnorm(float* y, const float* x, const float* w, int n, float eps) {
  const float s = 1.0f / sqrtf(or_dot_f32(n, x, x) / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = x[i] * s * w[i];
}

static float kv_scale(const int8_t* head, ptrdiff_t soff) {
  float s;
  memcpy(&s, head + soff, 4);
  return s;
}

/* kernels_avx512.cpp:228-267 */
static void attend_t(int DC, const float* q, int G, const int8_t* k, const int8_t* v, size_t stride, ptrdiff_t soff,
                     int n0, const int* extra, int ne, float scale, float* out, float* sc) {
  const int D = DC * 16;
  const int n = n0 + ne;
  for (int j = 0; j < n; ++j) {
    const int8_t* kr = k + (size_t)(j < n0 ? j : extra[j - n0]) * stride;
    const float ks = kv_scale(kr, soff) * scale;
    for (int h = 0; h < G; ++h) {
      float s[16];
      for (int l = 0; l < 16; ++l) s[l] = q[h * D + l] * (float)kr[l];
      for (int d = 1; d < DC; ++d)
        for (int l = 0; l < 16; ++l) s[l] = fmaf(q[h * D + 16 * d + l], (float)kr[16 * d + l], s[l]);
      sc[h * n + j] = or_reduce16(s) * ks;
    }
  }
  for (int h = 0; h < G; ++h) {
    const float inv = or_softmax_inplace(sc + h * n, n);
    for (int i = 0; i < D; ++i) {
      float acc = 0.0f;
      for (int j = 0; j < n; ++j) {
        const int8_t* vr = v + (size_t)(j < n0 ? j : extra[j - n0]) * stride;
        acc = fmaf(sc[h * n + j] * kv_scale(vr, soff), (float)vr[i], acc);
      }
      out[h * D + i] = acc * inv;
    }
  }
}

/* kernels_avx512.cpp:173-177 */
static float dot_f32_i8(const float* q, const int8_t* k, int n) {
  float s[16] = {0};
  for (int d = 0; d < n; d += 16)
    for (int l = 0; l < 16; ++l) s[l] = fmaf(q[d + l], (float)k[d + l], s[l]);
  return or_reduce16(s);
}

/* kernels_avx512.cpp:282-306 */
void or_attend_gqa(const float* q, int G, int D, const int8_t* k, const int8_t* v, size_t stride, ptrdiff_t soff,
                   int n, float scale, float* out, float* scratch, const int* extra, int ne) {
  if (G <= 16 && (D == 64 || D == 128 || D == 256)) {
    attend_t(D / 16, q, G, k, v, stride, soff, n, extra, ne, scale, out, scratch);
    return;
  }
  const int nk = n + ne;
  for (int h = 0; h < G; ++h) {
    float* s = scratch + (size_t)h * nk;
    for (int j = 0; j < nk; ++j) {
      const size_t r = (size_t)(j < n ? j : extra[j - n]) * stride;
      s[j] = dot_f32_i8(q + h * D, k + r, D) * kv_scale(k + r, soff) * scale;
    }
    const float iv = or_softmax_inplace(s, nk);
    float* o = out + h * D;
    for (int d = 0; d < D; ++d) o[d] = 0.0f;
    for (int j = 0; j < nk; ++j) {
      const size_t r = (size_t)(j < n ? j : extra[j - n]) * stride;
      const float a = s[j] * iv * kv_scale(v + r, soff);
      for (int d = 0; d < D; ++d) o[d] = fmaf(a, (float)v[r + d], o[d]);
    }
  }
}

/* ------------------------------------------------------------ panel GEMM */

/* gemm_avx512.cpp:422-428 */
static int q6_value(const uint8_t* s, int k) {
  const int n = k / 128, rem = k % 128, c = rem / 32, l = rem % 32;
  const uint8_t lo = s[64 * n + l + (c & 1) * 32];
  const int nib = c >= 2 ? lo >> 4 : lo & 0xF;
  const int hb = (s[128 + 32 * n + l] >> (2 * c)) & 3;
  return nib | (hb << 4);
}

/* gemm_avx512.cpp:67-102: acc = fma(float(sum (w+128) x - 128 (s0+s1)), f16(dw) * dx, acc), blocks in order. */
static float row_q8_0(const uint8_t* w, int64_t cols, const or_block_q8* x) {
  float acc = 0.0f;
  for (int64_t b = 0; b < cols / 32; ++b) {
    const uint8_t* blk = w + b * 34;
    int32_t ai = 0;
    for (int k = 0; k < 32; ++k) ai += (int32_t)(int8_t)blk[2 + k] * x[b].qs[k];
    acc = fmaf((float)ai, or_fp16_to_fp32(ld16(blk)) * x[b].d, acc);
  }
  return acc;
}

/* gemm_avx512.cpp:104-155 (compact) and 217-266 (wide: same arithmetic). */
static float row_q45_k(int high, const uint8_t* w, int64_t cols, const or_block_q8* x) {
  float acc = 0.0f;
  const size_t bytes = high ? 176 : 144;
  for (int64_t sb = 0; sb < cols / 256; ++sb) {
    const uint8_t* s = w + sb * bytes;
    const float d = or_fp16_to_fp32(ld16(s)), dmin = or_fp16_to_fp32(ld16(s + 2));
    const uint8_t* qh = s + 16;
    const uint8_t* qs = s + (high ? 48 : 16);
    for (int j = 0; j < 8; ++j) {
      int sc, m;
      scale_min_k4(j, s + 4, &sc, &m);
      const float fsc = d * (float)sc, fmn = dmin * (float)m;
      const or_block_q8* xq = x + sb * 8 + j;
      int32_t ai = 0;
      for (int k = 0; k < 32; ++k) {
        const uint8_t byte = qs[32 * (j / 2) + k];
        int q = (j & 1) ? byte >> 4 : byte & 0xF;
        if (high) q |= ((qh[k] >> j) & 1) << 4;
        ai += q * xq->qs[k];
      }
      const float dsx = xq->d * (float)(xq->s[0] + xq->s[1]);
      acc = fmaf((float)ai, fsc * xq->d, acc);
      acc = fmaf(-fmn, dsx, acc);
    }
  }
  return acc;
}

/* gemm_avx512.cpp:157-205: per 16-value half h, acc = fma(float(sum q x - 32 s[h&1]), (d*sc_h) * dx, acc). */
static float row_q6_k(const uint8_t* w, int64_t cols, const or_block_q8* x) {
  float acc = 0.0f;
  for (int64_t sb = 0; sb < cols / 256; ++sb) {
    const uint8_t* s = w + sb * 210;
    const float d = or_fp16_to_fp32(ld16(s + 208));
    for (int h = 0; h < 16; ++h) {
      const float dsc = d * (float)(int8_t)s[192 + h];
      const or_block_q8* xq = x + sb * 8 + h / 2;
      const int off = (h & 1) * 16;
      int32_t ai = 0;
      for (int k = 0; k < 16; ++k) ai += q6_value(s, 16 * h + k) * xq->qs[off + k];
      ai -= 32 * xq->s[h & 1];
      acc = fmaf((float)ai, dsc * xq->d, acc);
    }
  }
  return acc;
}

/* gemm_avx512.cpp:268-316: per Q8 block b, s = fma(ai1, d1, ai0 * d0), acc = fma(s, dx, acc). */
static float row_q6_w(const uint8_t* w, int64_t cols, const or_block_q8* x) {
  float acc = 0.0f;
  for (int64_t sb = 0; sb < cols / 256; ++sb) {
    const uint8_t* s = w + sb * 210;
    const float d = or_fp16_to_fp32(ld16(s + 208));
    for (int b = 0; b < 8; ++b) {
      const or_block_q8* xq = x + sb * 8 + b;
      int32_t ai[2] = {0, 0};
      for (int k = 0; k < 32; ++k) ai[k / 16] += (q6_value(s, 32 * b + k) - 32) * xq->qs[k];
      const float d0 = d * (float)(int8_t)s[192 + 2 * b], d1 = d * (float)(int8_t)s[192 + 2 * b + 1];
      const float sum = fmaf((float)ai[1], d1, (float)ai[0] * d0);
      acc = fmaf(sum, xq->d, acc);
    }
  }
  return acc;
}

int or_matmul(int type, const uint8_t* w, size_t row_bytes, int64_t rows, int64_t cols, const or_block_q8* xq, int n,
              float* y, int64_t y_stride, int wide) {
  if (type != OR_Q8_0 && type != OR_Q4_K && type != OR_Q5_K && type != OR_Q6_K) return -1;
  const int64_t nb = cols / 32;
  const int q6w = type == OR_Q6_K && wide && n > 16;
  for (int t = 0; t < n; ++t) {
    const or_block_q8* x = xq + (int64_t)t * nb;
    for (int64_t r = 0; r < rows; ++r) {
      const uint8_t* wr = w + (size_t)r * row_bytes;
      float v;
      switch (type) {
        case OR_Q8_0:
          v = row_q8_0(wr, cols, x);
          break;
        case OR_Q4_K:
          v = row_q45_k(0, wr, cols, x);
          break;
        case OR_Q5_K:
          v = row_q45_k(1, wr, cols, x);
          break;
        default:
          v = q6w ? row_q6_w(wr, cols, x) : row_q6_k(wr, cols, x);
          break;
      }
      y[(int64_t)t * y_stride + r] = v;
    }
  }
  return 0;
}

int32_t or_argmax(const float* l, int n) {
  int32_t best = 0;
  for (int i = 1; i < n; ++i)
    if (l[best] < l[i]) best = i;
  return best;
}

void or_top2(const float* l, int n, int32_t* pa, int32_t* pb) {
  int32_t a = 0, b = 1;
  if (l[b] > l[a]) {
    const int32_t t = a;
    a = b;
    b = t;
  }
  for (int32_t v = 2; v < n; ++v) {
    if (l[v] > l[a])
      b = a, a = v;
    else if (l[v] > l[b])
      b = v;
  }
  *pa = a;
  *pb = b;
}

/* ------------------------------------------------------------------ GGUF */

typedef struct {
  char name[96];
  int type;
  int64_t ne[4];
  int nd;
  const uint8_t* data;
} or_tensor;

typedef struct {
  int fd;
  uint8_t* base;
  size_t size;
  or_tensor* t;
  int nt;
  /* metadata the model reads (model.cpp:78-101) */
  char arch[32];
  int64_t block_count, embd, ff, heads, heads_kv, key_length, alignment;
  double rope_base, rms_eps;
} or_gguf;

typedef struct {
  const uint8_t* p;
  const uint8_t* end;
  int bad;
} rd;

static void need(rd* r, size_t n) {
  if ((size_t)(r->end - r->p) < n) r->bad = 1;
}
static uint64_t rd_u(rd* r, int bytes) {
  need(r, bytes);
  if (r->bad) return 0;
  uint64_t v = 0;
  memcpy(&v, r->p, bytes);
  r->p += bytes;
  return v;
}
static int type_bytes(uint32_t t) { /* gguf.cpp:222: u8 i8 u16 i16 u32 i32 f32 bool str arr u64 i64 f64 */
  static const int b[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  return t < 13 ? b[t] : -1;
}

static void skip_value(rd* r, uint32_t t) {
  if (t == 8) {
    const uint64_t n = rd_u(r, 8);
    need(r, n);
    if (!r->bad) r->p += n;
  } else if (t == 9) {
    const uint32_t et = (uint32_t)rd_u(r, 4);
    const uint64_t n = rd_u(r, 8);
    for (uint64_t i = 0; i < n && !r->bad; ++i) skip_value(r, et);
  } else {
    const int b = type_bytes(t);
    if (b <= 0) {
      r->bad = 1;
      return;
    }
    need(r, b);
    if (!r->bad) r->p += b;
  }
}

static int64_t read_intv(rd* r, uint32_t t) {
  switch (t) {
    case 0:
      return (uint8_t)rd_u(r, 1);
    case 1:
      return (int8_t)rd_u(r, 1);
    case 2:
      return (uint16_t)rd_u(r, 2);
    case 3:
      return (int16_t)rd_u(r, 2);
    case 4:
      return (uint32_t)rd_u(r, 4);
    case 5:
      return (int32_t)rd_u(r, 4);
    case 7:
      return (uint8_t)rd_u(r, 1);
    case 10:
    case 11:
      return (int64_t)rd_u(r, 8);
    default:
      r->bad = 1;
      return 0;
  }
}

static double read_floatv(rd* r, uint32_t t) {
  if (t == 6) {
    const uint32_t u = (uint32_t)rd_u(r, 4);
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  if (t == 12) {
    const uint64_t u = rd_u(r, 8);
    double d;
    memcpy(&d, &u, 8);
    return d;
  }
  return (double)read_intv(r, t);
}

static void gguf_close(or_gguf* g) {
  if (g->base) munmap(g->base, g->size);
  if (g->fd >= 0) close(g->fd);
  free(g->t);
}

/* gguf.cpp:205-249 */
static int gguf_open(or_gguf* g, const char* path, char* err, int errlen) {
  memset(g, 0, sizeof *g);
  g->fd = -1;
  g->rope_base = 10000.0;
  g->rms_eps = 1e-6;
  g->alignment = 32;
  g->heads_kv = -1;
  g->key_length = -1;
  g->fd = open(path, O_RDONLY);
  if (g->fd < 0) {
    snprintf(err, errlen, "cannot open %s", path);
    return -1;
  }
  struct stat st;
  fstat(g->fd, &st);
  g->size = (size_t)st.st_size;
  void* m = mmap(NULL, g->size, PROT_READ, MAP_SHARED, g->fd, 0);
  if (m == MAP_FAILED) {
    snprintf(err, errlen, "mmap failed");
    return -1;
  }
  g->base = (uint8_t*)m;
  rd r = {g->base, g->base + g->size, 0};
  if (rd_u(&r, 4) != 0x46554747 || rd_u(&r, 4) < 3) {
    snprintf(err, errlen, "%s is not a GGUF v3 file", path);
    return -1;
  }
  const uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
  for (uint64_t i = 0; i < nkv && !r.bad; ++i) {
    const uint64_t kl = rd_u(&r, 8);
    need(&r, kl);
    if (r.bad) break;
    char key[256] = {0};
    memcpy(key, r.p, kl < 255 ? kl : 255);
    r.p += kl;
    const uint32_t t = (uint32_t)rd_u(&r, 4);
    const char* a = g->arch[0] ? g->arch : "qwen3";
    char k2[256];
#define KEY(s) (snprintf(k2, sizeof k2, "%s.%s", a, s), strcmp(key, k2) == 0)
    if (strcmp(key, "general.architecture") == 0 && t == 8) {
      const uint64_t n = rd_u(&r, 8);
      need(&r, n);
      if (r.bad) break;
      memcpy(g->arch, r.p, n < 31 ? n : 31);
      r.p += n;
    } else if (strcmp(key, "general.alignment") == 0) {
      g->alignment = read_intv(&r, t);
    } else if (KEY("block_count")) {
      g->block_count = read_intv(&r, t);
    } else if (KEY("embedding_length")) {
      g->embd = read_intv(&r, t);
    } else if (KEY("feed_forward_length")) {
      g->ff = read_intv(&r, t);
    } else if (KEY("attention.head_count")) {
      g->heads = read_intv(&r, t);
    } else if (KEY("attention.head_count_kv")) {
      g->heads_kv = read_intv(&r, t);
    } else if (KEY("attention.key_length")) {
      g->key_length = read_intv(&r, t);
    } else if (KEY("rope.freq_base")) {
      g->rope_base = read_floatv(&r, t);
    } else if (KEY("attention.layer_norm_rms_epsilon")) {
      g->rms_eps = read_floatv(&r, t);
    } else {
      skip_value(&r, t);
    }
#undef KEY
  }
  g->t = (or_tensor*)calloc(nt ? nt : 1, sizeof(or_tensor));
  uint64_t* off = (uint64_t*)calloc(nt ? nt : 1, 8);
  for (uint64_t i = 0; i < nt && !r.bad; ++i) {
    const uint64_t nl = rd_u(&r, 8);
    need(&r, nl);
    if (r.bad) break;
    memcpy(g->t[i].name, r.p, nl < 95 ? nl : 95);
    r.p += nl;
    g->t[i].nd = (int)rd_u(&r, 4);
    for (int d = 0; d < 4; ++d) g->t[i].ne[d] = 1;
    for (int d = 0; d < g->t[i].nd; ++d) {
      const int64_t v = (int64_t)rd_u(&r, 8);
      if (d < 4) g->t[i].ne[d] = v;
    }
    g->t[i].type = (int)rd_u(&r, 4);
    off[i] = rd_u(&r, 8);
  }
  if (r.bad) {
    free(off);
    snprintf(err, errlen, "gguf: truncated header");
    return -1;
  }
  g->nt = (int)nt;
  const size_t hdr = (size_t)(r.p - g->base);
  const size_t start = (hdr + g->alignment - 1) / g->alignment * g->alignment;
  for (int i = 0; i < g->nt; ++i) {
    const int64_t nel = g->t[i].ne[0] * g->t[i].ne[1] * g->t[i].ne[2] * g->t[i].ne[3];
    const size_t nb = or_row_size(g->t[i].type, g->t[i].ne[0]) * (size_t)(nel / g->t[i].ne[0]);
    if (start + off[i] + nb > g->size) {
      free(off);
      snprintf(err, errlen, "gguf: tensor %s out of bounds", g->t[i].name);
      return -1;
    }
    g->t[i].data = g->base + start + off[i];
  }
  free(off);
  return 0;
}

static const or_tensor* gguf_tensor(const or_gguf* g, const char* name) {
  for (int i = 0; i < g->nt; ++i)
    if (strcmp(g->t[i].name, name) == 0) return &g->t[i];
  return NULL;
}

/* ----------------------------------------------------------------- Model */

typedef struct {
  int type;
  const uint8_t* data;
  int64_t rows, cols;
  size_t row_bytes;
} or_weight;

typedef struct {
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
  or_weight wq, wk, wv, wo, w_gate, w_up, w_down;
} or_layer;

enum { kMaxBatch = 256 }; /* model.h:35 */

struct or_model {
  or_gguf g;
  or_config c;
  int n_ctx, n_seq, wide, no_pack;
  or_weight tok_embd, output;
  const float* output_norm;
  or_layer* layers;
  float* inv_freq;
  int8_t *kcache, *vcache;
  size_t kv_row; /* bytes per KV row: KV*D int8 + KV float */
  /* per-token layout (model.h:67,83) */
  int *rpos, *kv_at, *kv_base, *n_keys, *out, n_out;
  int *anc, n_anc, *anc_off, tree, *depth;
  int32_t* ids;
  float *x, *h, *q, *k, *v, *att, *gate, *up, *cs, *sn, *scratch;
  or_block_q8* xq;
};

static int get_weight(const or_gguf* g, const char* name, or_weight* w, int required, char* err, int errlen) {
  const or_tensor* t = gguf_tensor(g, name);
  memset(w, 0, sizeof *w);
  if (!t) {
    if (required) snprintf(err, errlen, "model: tensor %s missing", name);
    return required ? -1 : 0;
  }
  if (!or_row_size(t->type, 256) && t->type != OR_F32) {
    snprintf(err, errlen, "model: tensor %s has unsupported type", name);
    return -1;
  }
  w->type = t->type;
  w->data = t->data;
  w->cols = t->ne[0];
  w->rows = t->ne[1] * t->ne[2] * t->ne[3];
  w->row_bytes = or_row_size(t->type, t->ne[0]);
  return 0;
}

static const float* get_norm(const or_gguf* g, const char* name, int64_t n, char* err, int errlen) {
  const or_tensor* t = gguf_tensor(g, name);
  if (!t || t->type != OR_F32 || t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3] != n) {
    snprintf(err, errlen, "model: norm %s missing or not F32[%lld]", name, (long long)n);
    return NULL;
  }
  return (const float*)t->data;
}

void or_model_free(or_model* m) {
  if (!m) return;
  gguf_close(&m->g);
  free(m->layers);
  free(m->inv_freq);
  free(m->kcache);
  free(m->vcache);
  free(m->rpos);
  free(m->kv_at);
  free(m->kv_base);
  free(m->n_keys);
  free(m->out);
  free(m->anc);
  free(m->anc_off);
  free(m->depth);
  free(m->ids);
  free(m->x);
  free(m->h);
  free(m->q);
  free(m->k);
  free(m->v);
  free(m->att);
  free(m->gate);
  free(m->up);
  free(m->cs);
  free(m->sn);
  free(m->scratch);
  free(m->xq);
  free(m);
}

or_model* or_model_open(const char* path, int n_ctx, int n_seq, int wide, char* err, int errlen) {
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  if (gguf_open(&m->g, path, err, errlen)) goto fail;
  if (strcmp(m->g.arch, "qwen3") != 0) {
    snprintf(err, errlen, "architecture '%s' unsupported (supported: qwen3)", m->g.arch);
    goto fail;
  }
  or_config* c = &m->c;
  c->n_layer = (int)m->g.block_count;
  c->n_embd = (int)m->g.embd;
  c->n_ff = (int)m->g.ff;
  c->n_head = (int)m->g.heads;
  c->n_head_kv = m->g.heads_kv >= 0 ? (int)m->g.heads_kv : c->n_head;
  c->head_dim = m->g.key_length >= 0 ? (int)m->g.key_length : c->n_embd / c->n_head;
  c->rope_base = (float)m->g.rope_base;
  c->rms_eps = (float)m->g.rms_eps;
  if (c->head_dim % 32 || c->n_head % c->n_head_kv) {
    snprintf(err, errlen, "model: unsupported head layout");
    goto fail;
  }
  if (get_weight(&m->g, "token_embd.weight", &m->tok_embd, 1, err, errlen)) goto fail;
  if (get_weight(&m->g, "output.weight", &m->output, 0, err, errlen)) goto fail;
  if (!m->output.data) m->output = m->tok_embd; /* tied embeddings (model.cpp:116-118) */
  c->n_vocab = (int)m->output.rows;
  if (!(m->output_norm = get_norm(&m->g, "output_norm.weight", c->n_embd, err, errlen))) goto fail;
  m->layers = (or_layer*)calloc(c->n_layer, sizeof(or_layer));
  for (int i = 0; i < c->n_layer; ++i) {
    or_layer* L = &m->layers[i];
    char nm[128];
#define NORM(field, s, n)                                               \
  snprintf(nm, sizeof nm, "blk.%d.%s", i, s);                           \
  if (!(L->field = get_norm(&m->g, nm, n, err, errlen))) goto fail;
#define W(field, s)                                                     \
  snprintf(nm, sizeof nm, "blk.%d.%s", i, s);                           \
  if (get_weight(&m->g, nm, &L->field, 1, err, errlen)) goto fail;
    NORM(attn_norm, "attn_norm.weight", c->n_embd)
    NORM(ffn_norm, "ffn_norm.weight", c->n_embd)
    NORM(q_norm, "attn_q_norm.weight", c->head_dim)
    NORM(k_norm, "attn_k_norm.weight", c->head_dim)
    W(wq, "attn_q.weight")
    W(wk, "attn_k.weight")
    W(wv, "attn_v.weight")
    W(wo, "attn_output.weight")
    W(w_gate, "ffn_gate.weight")
    W(w_up, "ffn_up.weight")
    W(w_down, "ffn_down.weight")
#undef NORM
#undef W
  }
  m->wide = wide & 1;
  m->no_pack = (wide & 2) != 0; /* MALKIN_NO_PACK (model.cpp:136): every matmul on the row path */
  m->inv_freq = (float*)malloc(sizeof(float) * c->head_dim / 2);
  for (int i = 0; i < c->head_dim / 2; ++i)
    m->inv_freq[i] = powf(c->rope_base, -2.0f * (float)i / (float)c->head_dim); /* model.cpp:137 */
  m->n_ctx = n_ctx;
  m->n_seq = n_seq;
  m->kv_row = (size_t)c->n_head_kv * (c->head_dim + 4);
  m->kcache = (int8_t*)calloc((size_t)c->n_layer * n_seq * n_ctx, m->kv_row);
  m->vcache = (int8_t*)calloc((size_t)c->n_layer * n_seq * n_ctx, m->kv_row);
  const size_t B = kMaxBatch, E = c->n_embd, HD = (size_t)c->n_head * c->head_dim;
  const size_t KVD = (size_t)c->n_head_kv * c->head_dim;
  m->rpos = (int*)malloc(B * sizeof(int));
  m->kv_at = (int*)malloc(B * sizeof(int));
  m->kv_base = (int*)malloc(B * sizeof(int));
  m->n_keys = (int*)malloc(B * sizeof(int));
  m->out = (int*)malloc(B * sizeof(int));
  m->depth = (int*)malloc(B * sizeof(int));
  m->anc = (int*)malloc(B * B * sizeof(int));
  m->anc_off = (int*)malloc((B + 1) * sizeof(int));
  m->ids = (int32_t*)malloc(B * sizeof(int32_t));
  m->x = (float*)malloc(B * E * 4);
  m->h = (float*)malloc(B * E * 4);
  m->q = (float*)malloc(B * HD * 4);
  m->att = (float*)malloc(B * HD * 4);
  m->k = (float*)malloc(B * KVD * 4);
  m->v = (float*)malloc(B * KVD * 4);
  m->gate = (float*)malloc(B * c->n_ff * 4);
  m->up = (float*)malloc(B * c->n_ff * 4);
  m->cs = (float*)malloc(B * c->head_dim / 2 * 4);
  m->sn = (float*)malloc(B * c->head_dim / 2 * 4);
  m->scratch = (float*)malloc((size_t)c->n_head * ((size_t)n_ctx + B) * 4);
  const size_t maxk = (size_t)(c->n_ff > (int)HD ? c->n_ff : HD) > E ? (size_t)(c->n_ff > (int)HD ? c->n_ff : HD) : E;
  m->xq = (or_block_q8*)malloc(B * (maxk / 32) * sizeof(or_block_q8));
  return m;
fail:
  or_model_free(m);
  return NULL;
}

void or_model_config(const or_model* m, or_config* c) { *c = m->c; }
size_t or_model_kv_row_bytes(const or_model* m) { return m->kv_row; }

const int8_t* or_model_kv_row(const or_model* m, int il, int seq, int pos, int k) {
  const size_t row = ((size_t)il * m->n_seq * m->n_ctx + (size_t)seq * m->n_ctx + pos) * m->kv_row;
  return (k ? m->kcache : m->vcache) + row;
}

static void quantize_acts(const float* x, int n, int64_t k, or_block_q8* out) {
  for (int t = 0; t < n; ++t) or_quantize_row_q8(x + (int64_t)t * k, out + (int64_t)t * (k / 32), k);
}

/* quant.cpp:320-351: panels for the quantized types unless MALKIN_NO_PACK; F32/F16/BF16 have no panels (row path). */
static void matmul(const or_model* m, const or_weight* w, const float* x, const or_block_q8* xq, int n, float* y) {
  const int rows_path = m->no_pack || w->type == OR_F32 || w->type == OR_F16 || w->type == OR_BF16;
  if (rows_path)
    or_matmul_rows(w->type, w->data, w->row_bytes, w->rows, w->cols, x, xq, n, y, w->rows);
  else
    or_matmul(w->type, w->data, w->row_bytes, w->rows, w->cols, xq, n, y, w->rows, m->wide);
}

/* model.cpp:204-247 (AVX-512 attends one token per call, attend_block_tokens = 1) */
static void attention(or_model* m, int il, int n) {
  const or_config* c = &m->c;
  const int D = c->head_dim, H = c->n_head, KV = c->n_head_kv, G = H / KV;
  const size_t layer = (size_t)il * m->n_seq * m->n_ctx * m->kv_row;
  const float scale = 1.0f / sqrtf((float)D);
  for (int t = 0; t < n; ++t) {
    for (int g = 0; g < KV; ++g) {
      const size_t qoff = ((size_t)t * H + (size_t)g * G) * D;
      const size_t kv = layer + (size_t)m->kv_base[t] * m->kv_row + (size_t)g * D;
      const ptrdiff_t soff = (ptrdiff_t)(KV - g) * D + (ptrdiff_t)(g * 4);
      or_attend_gqa(m->q + qoff, G, D, m->kcache + kv, m->vcache + kv, m->kv_row, soff, m->n_keys[t], scale,
                    m->att + qoff, m->scratch, m->tree ? m->anc + m->anc_off[t] : NULL,
                    m->tree ? m->anc_off[t + 1] - m->anc_off[t] : 0);
    }
  }
}

/* model.cpp:325-426 */
static int run(or_model* m, const int32_t* tokens, int n, float* logits, char* err, int errlen) {
  const or_config* c = &m->c;
  const int E = c->n_embd, D = c->head_dim, H = c->n_head, KV = c->n_head_kv, F = c->n_ff;
  const size_t kvd = (size_t)KV * D;
  for (int t = 0; t < n; ++t) {
    if (tokens[t] < 0 || tokens[t] >= m->tok_embd.rows) {
      snprintf(err, errlen, "forward: token id out of range");
      return -1;
    }
    or_dequantize_row(m->tok_embd.type, m->tok_embd.data + (size_t)tokens[t] * m->tok_embd.row_bytes,
                      m->x + (size_t)t * E, E);
  }
  for (int t = 0; t < n; ++t)
    for (int i = 0; i < D / 2; ++i) {
      const float a = (float)m->rpos[t] * m->inv_freq[i];
      m->cs[t * D / 2 + i] = cosf(a);
      m->sn[t * D / 2 + i] = sinf(a);
    }
  for (int il = 0; il < c->n_layer; ++il) {
    const or_layer* L = &m->layers[il];
    for (int t = 0; t < n; ++t) or_rmsnorm(m->h + (size_t)t * E, m->x + (size_t)t * E, L->attn_norm, E, c->rms_eps);
    quantize_acts(m->h, n, E, m->xq);
    matmul(m, &L->wq, m->h, m->xq, n, m->q);
    matmul(m, &L->wk, m->h, m->xq, n, m->k);
    matmul(m, &L->wv, m->h, m->xq, n, m->v);
    const size_t layer = (size_t)il * m->n_seq * m->n_ctx;
    for (int t = 0; t < n; ++t) {
      const float* cs = m->cs + t * D / 2;
      const float* sn = m->sn + t * D / 2;
      for (int hh = 0; hh < H + KV; ++hh) {
        float* v = hh < H ? m->q + ((size_t)t * H + hh) * D : m->k + ((size_t)t * KV + hh - H) * D;
        or_rmsnorm(v, v, hh < H ? L->q_norm : L->k_norm, D, c->rms_eps);
        /* model.cpp:341-350 (RoPE, NeoX pairs): clang contracts x0*c - x1*s to fma(x0, c, -(x1*s)) and
           x0*s + x1*c to fma(x0, s, x1*c). */
        for (int i = 0; i < D / 2; ++i) {
          const float x0 = v[i], x1 = v[i + D / 2];
          v[i] = fmaf(x0, cs[i], -(x1 * sn[i]));
          v[i + D / 2] = fmaf(x0, sn[i], x1 * cs[i]);
        }
      }
      const size_t row = (layer + m->kv_at[t]) * m->kv_row;
      for (int pass = 0; pass < 2; ++pass) {
        const float* src = (pass ? m->v : m->k) + (size_t)t * kvd;
        int8_t* dst = (pass ? m->vcache : m->kcache) + row;
        for (int hh = 0; hh < KV; ++hh) {
          const float s = or_quantize_i8(src + (size_t)hh * D, D, dst + (size_t)hh * D);
          memcpy(dst + kvd + hh * 4, &s, 4);
        }
      }
    }
    attention(m, il, n);
    quantize_acts(m->att, n, (int64_t)H * D, m->xq);
    matmul(m, &L->wo, m->att, m->xq, n, m->h);
    for (size_t i = 0; i < (size_t)n * E; ++i) m->x[i] += m->h[i];
    for (int t = 0; t < n; ++t) or_rmsnorm(m->h + (size_t)t * E, m->x + (size_t)t * E, L->ffn_norm, E, c->rms_eps);
    quantize_acts(m->h, n, E, m->xq);
    matmul(m, &L->w_gate, m->h, m->xq, n, m->gate);
    matmul(m, &L->w_up, m->h, m->xq, n, m->up);
    for (int t = 0; t < n; ++t) or_silu_mul(F, m->gate + (size_t)t * F, m->up + (size_t)t * F);
    quantize_acts(m->gate, n, F, m->xq);
    matmul(m, &L->w_down, m->gate, m->xq, n, m->h);
    for (size_t i = 0; i < (size_t)n * E; ++i) m->x[i] += m->h[i];
  }
  if (m->n_out == 0) return 0;
  for (int i = 0; i < m->n_out; ++i)
    or_rmsnorm(m->h + (size_t)i * E, m->x + (size_t)m->out[i] * E, m->output_norm, E, c->rms_eps);
  quantize_acts(m->h, m->n_out, E, m->xq);
  matmul(m, &m->output, m->h, m->xq, m->n_out, logits);
  return 0;
}

/* model.cpp:249-278 */
int or_model_forward(or_model* m, const int32_t* tokens, int n, int pos, float* logits, int all_logits,
                     const int* parent, int seq, char* err, int errlen) {
  if (n <= 0 || n > kMaxBatch) return snprintf(err, errlen, "forward: batch size out of range"), -1;
  if (pos + n > m->n_ctx) return snprintf(err, errlen, "forward: context full"), -1;
  if (seq < 0 || seq >= m->n_seq) return snprintf(err, errlen, "forward: bad sequence"), -1;
  m->n_anc = 0;
  m->tree = parent != NULL;
  if (parent) {
    for (int t = 0; t < n; ++t) {
      m->depth[t] = parent[t] < 0 ? 0 : m->depth[parent[t]] + 1;
      m->anc_off[t] = m->n_anc;
      for (int a = t; a >= 0; a = parent[a]) m->anc[m->n_anc++] = pos + a;
      for (int i = m->anc_off[t], j = m->n_anc - 1; i < j; ++i, --j) { /* root first */
        const int tmp = m->anc[i];
        m->anc[i] = m->anc[j];
        m->anc[j] = tmp;
      }
    }
    m->anc_off[n] = m->n_anc;
  }
  m->n_out = 0;
  for (int t = 0; t < n; ++t) {
    m->rpos[t] = pos + (parent ? m->depth[t] : t);
    m->kv_base[t] = seq * m->n_ctx;
    m->kv_at[t] = seq * m->n_ctx + pos + t;
    m->n_keys[t] = parent ? pos : pos + t + 1;
    if (all_logits || t == n - 1) m->out[m->n_out++] = t;
  }
  return run(m, tokens, n, logits, err, errlen);
}

/* model.cpp:280-323 */
int or_model_forward_batch(or_model* m, const or_batch_token* batch, int n, float* logits, char* err, int errlen) {
  if (n <= 0 || n > kMaxBatch) return snprintf(err, errlen, "forward: batch size out of range"), -1;
  m->n_anc = 0;
  m->n_out = 0;
  int tree = 0;
  for (int t = 0; t < n; ++t) {
    const or_batch_token* b = &batch[t];
    const int kv = b->parent < 0 ? b->pos : b->kv;
    if (b->seq < 0 || b->seq >= m->n_seq || b->pos < 0 || b->pos >= m->n_ctx || kv < 0 || kv >= m->n_ctx)
      return snprintf(err, errlen, "forward: bad slot"), -1;
    if (b->parent >= t || (b->parent >= 0 && batch[b->parent].seq != b->seq))
      return snprintf(err, errlen, "forward: bad tree parent"), -1;
    m->ids[t] = b->id;
    m->rpos[t] = b->pos;
    m->kv_base[t] = b->seq * m->n_ctx;
    m->kv_at[t] = m->kv_base[t] + kv;
    tree = tree || b->parent >= 0;
    if (b->logits) m->out[m->n_out++] = t;
  }
  m->tree = tree;
  if (tree) m->anc_off[0] = 0;
  for (int t = 0; t < n; ++t) {
    const or_batch_token* b = &batch[t];
    if (b->parent < 0) {
      m->n_keys[t] = b->pos + 1;
    } else {
      m->n_keys[t] = m->n_keys[b->parent];
      for (int i = m->anc_off[b->parent]; i < m->anc_off[b->parent + 1]; ++i) m->anc[m->n_anc++] = m->anc[i];
      m->anc[m->n_anc++] = m->kv_at[t] - m->kv_base[t];
    }
    if (tree) m->anc_off[t + 1] = m->n_anc;
  }
  return run(m, m->ids, n, logits, err, errlen);
}

/* model.cpp:432-440 */
void or_model_move_kv(or_model* m, int from, int to, int seq) {
  if (from == to) return;
  for (int il = 0; il < m->c.n_layer; ++il) {
    const size_t base = (size_t)il * m->n_seq * m->n_ctx + (size_t)seq * m->n_ctx;
    memcpy(m->kcache + (base + to) * m->kv_row, m->kcache + (base + from) * m->kv_row, m->kv_row);
    memcpy(m->vcache + (base + to) * m->kv_row, m->vcache + (base + from) * m->kv_row, m->kv_row);
  }
}

/* ---------------------------------------------------------------- sampling (sampler.cpp:22-141) */

#define MT_N 312
#define MT_M 156

void or_mt64_seed(or_mt64* g, uint64_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < MT_N; ++i) g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
  g->i = MT_N;
}

uint64_t or_mt64_next(or_mt64* g) {
  const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL, a = 0xB5026F5AA96619E9ULL;
  if (g->i >= MT_N) { /* regenerate the whole state */
    for (int k = 0; k < MT_N; ++k) {
      const uint64_t y = (g->mt[k] & upper) | (g->mt[(k + 1) % MT_N] & lower);
      g->mt[k] = g->mt[(k + MT_M) % MT_N] ^ (y >> 1) ^ ((y & 1) ? a : 0);
    }
    g->i = 0;
  }
  uint64_t z = g->mt[g->i++];
  z ^= (z >> 29) & 0x5555555555555555ULL;
  z ^= (z << 17) & 0x71D67FFFEDA60000ULL;
  z ^= (z << 37) & 0xFFF7EEE000000000ULL;
  z ^= z >> 43;
  return z;
}

double or_mt64_uniform(or_mt64* g) {
  const double u = (double)or_mt64_next(g) / 18446744073709551616.0;
  return u >= 1.0 ? nextafter(1.0, 0.0) : u;
}

void or_penalize(float* l, const int32_t* ids, const int* counts, int n, float presence, float frequency) {
  for (int i = 0; i < n; ++i) l[ids[i]] -= fmaf(frequency, (float)counts[i], presence);
}

typedef struct {
  float v;
  int32_t id;
} or_cand;

static int cand_before(const void* pa, const void* pb) {
  const or_cand *a = (const or_cand*)pa, *b = (const or_cand*)pb;
  if (a->v > b->v) return -1;
  if (b->v > a->v) return 1;
  return a->id < b->id ? -1 : a->id > b->id;
}

int or_distribution(const or_sampling* p, const float* l, int n_vocab, float* probs, int32_t* ids) {
  if (n_vocab < 1) return 0;
  if (p->temperature <= 0.0f) { /* the first maximum */
    probs[0] = 1.0f;
    ids[0] = or_argmax(l, n_vocab);
    return 1;
  }
  or_cand* c = (or_cand*)malloc(sizeof(or_cand) * (size_t)n_vocab);
  double* w = (double*)malloc(sizeof(double) * (size_t)n_vocab);
  for (int i = 0; i < n_vocab; ++i) {
    c[i].v = l[i];
    c[i].id = i;
  }
  qsort(c, (size_t)n_vocab, sizeof(or_cand), cand_before);
  const int k = p->top_k > 0 && p->top_k < n_vocab ? p->top_k : n_vocab;
  for (int i = k; i < n_vocab; ++i) w[i] = 0.0;
  double sum = 0.0;
  for (int i = 0; i < k; ++i) {
    const float e = expf((c[i].v - c[0].v) / p->temperature); /* float weight, as the reference stores it */
    w[i] = e;
    sum += e;
  }
  const double floor_w = (double)p->min_p * w[0];
  double kept = 0.0;
  int n = 0;
  for (; n < k; ++n) {
    if (n > 0 && w[n] < floor_w) break;
    kept += w[n];
    if (kept >= (double)p->top_p * sum) {
      ++n;
      break;
    }
  }
  if (n < 1) n = 1;
  double total = 0.0;
  for (int i = 0; i < n; ++i) total += w[i];
  for (int i = 0; i < n; ++i) {
    probs[i] = (float)(w[i] / total);
    ids[i] = c[i].id;
  }
  free(c);
  free(w);
  return n;
}

int32_t or_draw(or_mt64* g, const float* probs, const int32_t* ids, int n) {
  if (n == 1) return ids[0];
  double r = or_mt64_uniform(g);
  for (int i = 0; i < n; ++i) {
    r -= probs[i];
    if (r <= 0.0) return ids[i];
  }
  return ids[n - 1];
}

static float prob_of(const float* probs, const int32_t* ids, int n, int32_t id) {
  for (int i = 0; i < n; ++i)
    if (ids[i] == id) return probs[i];
  return 0.0f;
}

int32_t or_verify(or_mt64* g, const float* pp, const int32_t* pi, int np, const float* qp, const int32_t* qi, int nq,
                  int32_t draft, int* accepted) {
  const float pd = prob_of(pp, pi, np, draft), qd = prob_of(qp, qi, nq, draft);
  const double u = or_mt64_uniform(g);
  *accepted = qd > 0.0f && u * (double)qd < (double)pd;
  if (*accepted) return draft;
  float* rp = (float*)malloc(sizeof(float) * (size_t)np);
  int32_t* ri = (int32_t*)malloc(sizeof(int32_t) * (size_t)np);
  int m = 0;
  double total = 0.0;
  for (int i = 0; i < np; ++i) {
    const float r = pp[i] - prob_of(qp, qi, nq, pi[i]);
    if (r > 0.0f) {
      rp[m] = r;
      ri[m++] = pi[i];
      total += r;
    }
  }
  int32_t t;
  if (m == 0) {
    t = or_draw(g, pp, pi, np);
  } else {
    for (int i = 0; i < m; ++i) rp[i] = (float)(rp[i] / total);
    t = or_draw(g, rp, ri, m);
  }
  free(rp);
  free(ri);
  return t;
}

long or_verify_experiment(const float* pp, const int32_t* pi, int np, const float* qp, const int32_t* qi, int nq,
                          uint64_t target_seed, uint64_t draft_seed, long n_trials, long* hist, int V) {
  or_mt64 target, draft;
  or_mt64_seed(&target, target_seed);
  or_mt64_seed(&draft, draft_seed);
  long acc = 0;
  for (long n = 0; n < n_trials; ++n) {
    const int32_t d = or_draw(&draft, qp, qi, nq);
    int a = 0;
    const int32_t t = or_verify(&target, pp, pi, np, qp, qi, nq, d, &a);
    if (t >= 0 && t < V) ++hist[t];
    acc += a;
  }
  return acc;
}
