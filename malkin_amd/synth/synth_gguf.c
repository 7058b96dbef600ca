/*
 * Deterministic random-init qwen3 GGUF writer (synthetic models for the parity tests and the benchmark).
 *
 * The reference ships no models and no quantizer; its Model only needs general.architecture = qwen3, the qwen3.* keys
 * (model.cpp:78-101) and the token_embd / output_norm / output / blk.N.* tensors (model.cpp:112-135). This writer
 * produces exactly that. It is libm-free and uses only float add/mul/div (compiled with -ffp-contract=off), so the
 * file bytes are identical on any x86-64 host: weights are N(0, std) approximated by an Irwin-Hall sum of four
 * 16-bit uniforms from a counter-based splitmix64 hash of (seed, tensor, element), quantized by the simple
 * quantizers below. Tensor data is generated in parallel straight into an mmap of the output file.
 */
#define _GNU_SOURCE
#include "synth_gguf.h"

#include <fcntl.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

static uint64_t splitmix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Approximately N(0, 1): Irwin-Hall of 4 uniforms, centred and scaled to unit variance. */
static float normal(uint64_t key, uint64_t i) {
  const uint64_t h = splitmix(key ^ (i * 0xD6E8FEB86659FD93ull));
  const uint32_t s = (uint32_t)(h & 0xFFFF) + (uint32_t)((h >> 16) & 0xFFFF) + (uint32_t)((h >> 32) & 0xFFFF) +
                     (uint32_t)(h >> 48);
  return ((float)s / 65536.0f - 2.0f) * 1.7320508f;
}

static float fabs_(float x) { return x < 0.0f ? -x : x; }

/* Round half away from zero, exact (no libm). */
static int round_(float v) {
  const int t = (int)v;
  const float fr = v - (float)t;
  return fr >= 0.5f ? t + 1 : fr <= -0.5f ? t - 1 : t;
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* float -> IEEE half, round to nearest even (normal and subnormal range; values here are small and finite). */
static uint16_t to_half(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t a = u & 0x7FFFFFFF;
  if (a >= 0x477FF000) return sign | 0x7C00;
  if (a < 0x38800000) {
    if (a < 0x33000000) return sign;
    const uint32_t e = a >> 23, mant = (a & 0x7FFFFF) | 0x800000;
    const int shift = 126 - (int)e;
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return sign | (uint16_t)q;
  }
  uint32_t h = (a >> 13) - (112u << 10);
  const uint32_t rem = a & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
  return sign | (uint16_t)h;
}

/* IEEE half -> float, exact for normal and subnormal halves (Q6_K's d of N(0, 0.02) weights is a subnormal half:
   about 1.4e-5 < 2^-14). A subnormal is m * 2^-24, exact in float. */
static float from_half(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  float f;
  if (e == 0) {
    f = (float)m * (1.0f / 16777216.0f);
    return sign ? -f : f;
  }
  const uint32_t u = sign | ((e + 112) << 23) | (m << 13);
  memcpy(&f, &u, 4);
  return f;
}

static void put16(uint8_t* p, uint16_t v) { memcpy(p, &v, 2); }

/* Q8_0: d = amax / 127 stored as half, q = round(x / d). */
static void quant_q8_0(const float* x, uint8_t* out, int64_t k) {
  for (int64_t b = 0; b < k / 32; ++b, x += 32, out += 34) {
    float amax = 0.0f;
    for (int l = 0; l < 32; ++l) amax = fabs_(x[l]) > amax ? fabs_(x[l]) : amax;
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(out, to_half(d));
    for (int l = 0; l < 32; ++l) out[2 + l] = (uint8_t)(int8_t)clampi(round_(x[l] * id), -127, 127);
  }
}

/* Q4_K: per 32-value sub-block an asymmetric 4-bit range, 6-bit sub-scales/mins under half d / dmin. */
static void quant_q4_k(const float* x, uint8_t* out, int64_t k) {
  for (int64_t sb = 0; sb < k / 256; ++sb, x += 256, out += 144) {
    float scale[8], mins[8], maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; ++j) {
      float lo = 0.0f, hi = x[32 * j];
      for (int l = 0; l < 32; ++l) {
        const float v = x[32 * j + l];
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
      }
      scale[j] = (hi - lo) / 15.0f;
      mins[j] = -lo;
      maxs = scale[j] > maxs ? scale[j] : maxs;
      maxm = mins[j] > maxm ? mins[j] : maxm;
    }
    const uint16_t hd = to_half(maxs / 63.0f), hm = to_half(maxm / 63.0f);
    const float d = from_half(hd), dmin = from_half(hm);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
      sc[j] = d > 0.0f ? clampi(round_(scale[j] / d), 0, 63) : 0;
      m[j] = dmin > 0.0f ? clampi(round_(mins[j] / dmin), 0, 63) : 0;
    }
    put16(out, hd);
    put16(out + 2, hm);
    uint8_t* s = out + 4;
    for (int j = 0; j < 4; ++j) {
      s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qs = out + 16;
    memset(qs, 0, 128);
    for (int j = 0; j < 8; ++j) {
      const float step = d * (float)sc[j], off = dmin * (float)m[j];
      for (int l = 0; l < 32; ++l) {
        const int q = step > 0.0f ? clampi(round_((x[32 * j + l] + off) / step), 0, 15) : 0;
        qs[32 * (j / 2) + l] |= (uint8_t)(q << (4 * (j & 1)));
      }
    }
  }
}

/* Q5_K: Q4_K's asymmetric sub-block ranges with 5-bit values: low nibbles in qs (Q4_K layout), the fifth bit of value l
   of sub-block j in bit j of qh[l]. */
static void quant_q5_k(const float* x, uint8_t* out, int64_t k) {
  for (int64_t sb = 0; sb < k / 256; ++sb, x += 256, out += 176) {
    float scale[8], mins[8], maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; ++j) {
      float lo = 0.0f, hi = x[32 * j];
      for (int l = 0; l < 32; ++l) {
        const float v = x[32 * j + l];
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
      }
      scale[j] = (hi - lo) / 31.0f;
      mins[j] = -lo;
      maxs = scale[j] > maxs ? scale[j] : maxs;
      maxm = mins[j] > maxm ? mins[j] : maxm;
    }
    const uint16_t hd = to_half(maxs / 63.0f), hm = to_half(maxm / 63.0f);
    const float d = from_half(hd), dmin = from_half(hm);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
      sc[j] = d > 0.0f ? clampi(round_(scale[j] / d), 0, 63) : 0;
      m[j] = dmin > 0.0f ? clampi(round_(mins[j] / dmin), 0, 63) : 0;
    }
    put16(out, hd);
    put16(out + 2, hm);
    uint8_t* s = out + 4;
    for (int j = 0; j < 4; ++j) {
      s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qh = out + 16;
    uint8_t* qs = out + 48;
    memset(qh, 0, 32);
    memset(qs, 0, 128);
    for (int j = 0; j < 8; ++j) {
      const float step = d * (float)sc[j], off = dmin * (float)m[j];
      for (int l = 0; l < 32; ++l) {
        const int q = step > 0.0f ? clampi(round_((x[32 * j + l] + off) / step), 0, 31) : 0;
        qs[32 * (j / 2) + l] |= (uint8_t)((q & 0xF) << (4 * (j & 1)));
        qh[l] |= (uint8_t)(((q >> 4) & 1) << j);
      }
    }
  }
}

/* Q6_K: per 16-value sub-block an int8 scale under half d, q in [-32, 31] stored + 32. */
static void quant_q6_k(const float* x, uint8_t* out, int64_t k) {
  for (int64_t sb = 0; sb < k / 256; ++sb, x += 256, out += 210) {
    float scale[16], maxs = 0.0f;
    for (int i = 0; i < 16; ++i) {
      float amax = 0.0f;
      for (int l = 0; l < 16; ++l) amax = fabs_(x[16 * i + l]) > amax ? fabs_(x[16 * i + l]) : amax;
      scale[i] = amax / 31.0f;
      maxs = scale[i] > maxs ? scale[i] : maxs;
    }
    const uint16_t hd = to_half(maxs / 127.0f);
    const float d = from_half(hd);
    int q[256];
    int8_t sc[16];
    for (int i = 0; i < 16; ++i) {
      sc[i] = (int8_t)(d > 0.0f ? clampi(round_(scale[i] / d), -128, 127) : 0);
      const float step = d * (float)sc[i];
      for (int l = 0; l < 16; ++l) q[16 * i + l] = (step > 0.0f ? clampi(round_(x[16 * i + l] / step), -32, 31) : 0) + 32;
    }
    uint8_t* ql = out;
    uint8_t* qh = out + 128;
    for (int n = 0; n < 2; ++n)
      for (int l = 0; l < 32; ++l) {
        const int q1 = q[128 * n + l], q2 = q[128 * n + 32 + l], q3 = q[128 * n + 64 + l], q4 = q[128 * n + 96 + l];
        ql[64 * n + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
        ql[64 * n + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
        qh[32 * n + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
      }
    memcpy(out + 192, sc, 16);
    put16(out + 208, hd);
  }
}

/* float -> bfloat16, round to nearest even (finite values). */
static uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static size_t row_bytes(int type, int64_t k) {
  switch (type) {
    case T_F32:
      return (size_t)k * 4;
    case T_F16:
    case T_BF16:
      return (size_t)k * 2;
    case T_Q8_0:
      return (size_t)(k / 32) * 34;
    case T_Q4_K:
      return (size_t)(k / 256) * 144;
    case T_Q5_K:
      return (size_t)(k / 256) * 176;
    case T_Q6_K:
      return (size_t)(k / 256) * 210;
    default:
      return 0;
  }
}

typedef struct {
  char name[64];
  int type, nd;
  int64_t ne0, ne1;
  uint64_t off;
  int norm; /* 1: F32 norm weights around 1 */
} tinfo;

typedef struct {
  tinfo* t;
  int nt;
  uint8_t* data; /* start of the tensor data section in the mapping */
  uint64_t seed;
  float std;
  int64_t next_row; /* work counter over the concatenated rows of all tensors, in chunks */
  int64_t total_rows;
  pthread_mutex_t mu;
} job;

/* q4_k_m-like mix (the draft model of config 5): Q6_K for output and for attn_v / ffn_down in the layers llama.cpp's
   use_more_bits rule picks (i < L/8, i >= 7L/8, or (i - L/8) % 3 == 2), Q4_K elsewhere. */
static int more_bits(int i, int L) { return i < L / 8 || i >= 7 * L / 8 || (i - L / 8) % 3 == 2; }

static int weight_type(const mks_config* c, const char* what, int layer) {
  if (c->mix == MKS_MIX_Q4_K_M) {
    if (!strcmp(what, "output")) return T_Q6_K;
    if ((!strcmp(what, "attn_v") || !strcmp(what, "ffn_down")) && more_bits(layer, c->n_layer)) return T_Q6_K;
    return T_Q4_K;
  }
  return c->type;
}

static int build_table(const mks_config* c, tinfo* t) {
  int n = 0;
  const int64_t E = c->n_embd, HD = (int64_t)c->n_head * c->head_dim, KVD = (int64_t)c->n_head_kv * c->head_dim;
#define ADD(nm, ty, a, b, isnorm)                 \
  do {                                            \
    if (t) {                                      \
      snprintf(t[n].name, 64, "%s", nm);          \
      t[n].type = ty;                             \
      t[n].ne0 = a;                               \
      t[n].ne1 = b;                               \
      t[n].nd = (b) > 1 ? 2 : 1;                  \
      t[n].norm = isnorm;                         \
    }                                             \
    ++n;                                          \
  } while (0)
  ADD("token_embd.weight", weight_type(c, "token_embd", 0), E, c->n_vocab, 0);
  ADD("output_norm.weight", T_F32, E, 1, 1);
  if (!c->tied) ADD("output.weight", weight_type(c, "output", 0), E, c->n_vocab, 0);
  for (int i = 0; i < c->n_layer; ++i) {
    char nm[64];
#define L(s, ty, a, b, isnorm)                    \
  snprintf(nm, sizeof nm, "blk.%d.%s", i, s);     \
  ADD(nm, ty, a, b, isnorm);
    L("attn_norm.weight", T_F32, E, 1, 1)
    L("attn_q.weight", weight_type(c, "attn_q", i), E, HD, 0)
    L("attn_k.weight", weight_type(c, "attn_k", i), E, KVD, 0)
    L("attn_v.weight", weight_type(c, "attn_v", i), E, KVD, 0)
    L("attn_output.weight", weight_type(c, "attn_output", i), HD, E, 0)
    L("attn_q_norm.weight", T_F32, c->head_dim, 1, 1)
    L("attn_k_norm.weight", T_F32, c->head_dim, 1, 1)
    L("ffn_norm.weight", T_F32, E, 1, 1)
    L("ffn_gate.weight", weight_type(c, "ffn_gate", i), E, c->n_ff, 0)
    L("ffn_up.weight", weight_type(c, "ffn_up", i), E, c->n_ff, 0)
    L("ffn_down.weight", weight_type(c, "ffn_down", i), c->n_ff, E, 0)
#undef L
  }
#undef ADD
  return n;
}

static void gen_row(const job* j, const tinfo* t, int ti, int64_t r, float* buf) {
  const uint64_t key = splitmix(j->seed * 0x100000001B3ull + (uint64_t)ti);
  for (int64_t i = 0; i < t->ne0; ++i) {
    const float z = normal(key, (uint64_t)r * (uint64_t)t->ne0 + (uint64_t)i);
    buf[i] = t->norm ? 1.0f + 0.1f * z : j->std * z;
  }
  uint8_t* dst = j->data + t->off + row_bytes(t->type, t->ne0) * (size_t)r;
  switch (t->type) {
    case T_F32:
      memcpy(dst, buf, (size_t)t->ne0 * 4);
      break;
    case T_F16:
      for (int64_t i = 0; i < t->ne0; ++i) put16(dst + 2 * i, to_half(buf[i]));
      break;
    case T_BF16:
      for (int64_t i = 0; i < t->ne0; ++i) put16(dst + 2 * i, to_bf16(buf[i]));
      break;
    case T_Q8_0:
      quant_q8_0(buf, dst, t->ne0);
      break;
    case T_Q4_K:
      quant_q4_k(buf, dst, t->ne0);
      break;
    case T_Q5_K:
      quant_q5_k(buf, dst, t->ne0);
      break;
    case T_Q6_K:
      quant_q6_k(buf, dst, t->ne0);
      break;
  }
}

static void* worker(void* arg) {
  job* j = (job*)arg;
  int64_t maxk = 0;
  for (int i = 0; i < j->nt; ++i) maxk = j->t[i].ne0 > maxk ? j->t[i].ne0 : maxk;
  float* buf = (float*)malloc((size_t)maxk * 4);
  const int64_t chunk = 64;
  for (;;) {
    pthread_mutex_lock(&j->mu);
    const int64_t start = j->next_row;
    j->next_row += chunk;
    pthread_mutex_unlock(&j->mu);
    if (start >= j->total_rows) break;
    int64_t base = 0;
    for (int ti = 0; ti < j->nt; ++ti) {
      const int64_t rows = j->t[ti].ne1;
      const int64_t lo = start > base ? start : base, hi = start + chunk < base + rows ? start + chunk : base + rows;
      for (int64_t r = lo; r < hi; ++r) gen_row(j, &j->t[ti], ti, r - base, buf);
      base += rows;
      if (base >= start + chunk) break;
    }
  }
  free(buf);
  return NULL;
}

/* ---- GGUF serialisation (v3; key/value types: u32 = 4, f32 = 6, string = 8) ---- */

typedef struct {
  uint8_t* p;
  size_t n;
} wbuf;

static void w_bytes(wbuf* w, const void* s, size_t n) {
  if (w->p) memcpy(w->p + w->n, s, n);
  w->n += n;
}
static void w_u32(wbuf* w, uint32_t v) { w_bytes(w, &v, 4); }
static void w_u64(wbuf* w, uint64_t v) { w_bytes(w, &v, 8); }
static void w_str(wbuf* w, const char* s) {
  w_u64(w, strlen(s));
  w_bytes(w, s, strlen(s));
}
static void kv_str(wbuf* w, const char* k, const char* v) {
  w_str(w, k);
  w_u32(w, 8);
  w_str(w, v);
}
static void kv_u32(wbuf* w, const char* k, uint32_t v) {
  w_str(w, k);
  w_u32(w, 4);
  w_u32(w, v);
}
static void kv_f32(wbuf* w, const char* k, float v) {
  w_str(w, k);
  w_u32(w, 6);
  w_bytes(w, &v, 4);
}

static size_t header(wbuf* w, const mks_config* c, const tinfo* t, int nt) {
  w_u32(w, 0x46554747);
  w_u32(w, 3);
  w_u64(w, (uint64_t)nt);
  w_u64(w, c->eos_id >= 0 ? 13 : 12);
  kv_str(w, "general.architecture", "qwen3");
  kv_str(w, "general.name", c->name[0] ? c->name : "synthetic");
  kv_u32(w, "general.alignment", 32);
  kv_u32(w, "qwen3.block_count", (uint32_t)c->n_layer);
  kv_u32(w, "qwen3.embedding_length", (uint32_t)c->n_embd);
  kv_u32(w, "qwen3.feed_forward_length", (uint32_t)c->n_ff);
  kv_u32(w, "qwen3.attention.head_count", (uint32_t)c->n_head);
  kv_u32(w, "qwen3.attention.head_count_kv", (uint32_t)c->n_head_kv);
  kv_u32(w, "qwen3.attention.key_length", (uint32_t)c->head_dim);
  kv_u32(w, "qwen3.context_length", (uint32_t)c->n_ctx_train);
  kv_f32(w, "qwen3.rope.freq_base", c->rope_base);
  kv_f32(w, "qwen3.attention.layer_norm_rms_epsilon", c->rms_eps);
  if (c->eos_id >= 0) kv_u32(w, "tokenizer.ggml.eos_token_id", (uint32_t)c->eos_id);
  for (int i = 0; i < nt; ++i) {
    w_str(w, t[i].name);
    w_u32(w, (uint32_t)t[i].nd);
    w_u64(w, (uint64_t)t[i].ne0);
    if (t[i].nd > 1) w_u64(w, (uint64_t)t[i].ne1);
    w_u32(w, (uint32_t)t[i].type);
    w_u64(w, t[i].off);
  }
  return (w->n + 31) / 32 * 32;
}

int mks_quantize_rows(int type, const float* x, int64_t rows, int64_t k, uint8_t* out) {
  const size_t rb = row_bytes(type, k);
  if (!rb || (type != T_Q8_0 && type != T_Q4_K && type != T_Q5_K && type != T_Q6_K) || k % (type == T_Q8_0 ? 32 : 256))
    return -2;
  for (int64_t r = 0; r < rows; ++r, x += k, out += rb) {
    if (type == T_Q8_0)
      quant_q8_0(x, out, k);
    else if (type == T_Q4_K)
      quant_q4_k(x, out, k);
    else if (type == T_Q5_K)
      quant_q5_k(x, out, k);
    else
      quant_q6_k(x, out, k);
  }
  return 0;
}

int64_t mks_file_bytes(const mks_config* c) {
  const int nt = build_table(c, NULL);
  tinfo* t = (tinfo*)calloc((size_t)nt, sizeof(tinfo));
  build_table(c, t);
  uint64_t off = 0;
  for (int i = 0; i < nt; ++i) {
    t[i].off = off;
    off += (row_bytes(t[i].type, t[i].ne0) * (uint64_t)t[i].ne1 + 31) / 32 * 32;
  }
  wbuf w = {NULL, 0};
  const size_t hdr = header(&w, c, t, nt);
  free(t);
  return (int64_t)(hdr + off);
}

int mks_write_gguf(const char* path, const mks_config* c, int threads) {
  if (c->n_embd % 256 || c->n_ff % 256 || ((int64_t)c->n_head * c->head_dim) % 256 || c->head_dim % 32 ||
      c->n_head % c->n_head_kv)
    return -2;
  const int nt = build_table(c, NULL);
  tinfo* t = (tinfo*)calloc((size_t)nt, sizeof(tinfo));
  build_table(c, t);
  uint64_t off = 0;
  int64_t rows = 0;
  for (int i = 0; i < nt; ++i) {
    if (!row_bytes(t[i].type, t[i].ne0)) {
      free(t);
      return -2;
    }
    t[i].off = off;
    off += (row_bytes(t[i].type, t[i].ne0) * (uint64_t)t[i].ne1 + 31) / 32 * 32;
    rows += t[i].ne1;
  }
  wbuf w = {NULL, 0};
  const size_t hdr = header(&w, c, t, nt);
  const size_t total = hdr + off;
  const int fd = open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) {
    free(t);
    return -1;
  }
  if (ftruncate(fd, (off_t)total) != 0) {
    close(fd);
    free(t);
    return -1;
  }
  uint8_t* map = (uint8_t*)mmap(NULL, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  if (map == MAP_FAILED) {
    close(fd);
    free(t);
    return -1;
  }
  memset(map, 0, hdr);
  w.p = map;
  w.n = 0;
  header(&w, c, t, nt);
  job j;
  j.t = t;
  j.nt = nt;
  j.data = map + hdr;
  j.seed = c->seed;
  j.std = c->std;
  j.next_row = 0;
  j.total_rows = rows;
  pthread_mutex_init(&j.mu, NULL);
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t th[256];
  for (int i = 0; i < threads; ++i) pthread_create(&th[i], NULL, worker, &j);
  for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
  pthread_mutex_destroy(&j.mu);
  munmap(map, total);
  close(fd);
  free(t);
  return 0;
}
