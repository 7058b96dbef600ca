// QK-norm + RoPE + int8 KV write, GQA attention over the int8 KV cache, KV row moves, greedy selection.
// Bit-identical to the reference:
//   qk_norm_rope_kv  model.cpp:370-392 (rmsnorm per head, NeoX RoPE as clang contracts it, quantize_i8 rows)
//   attention        kernels_avx512.cpp:228-267 (attend_t<D/16>) and 282-306 (other head sizes), model.cpp:204-247
//   move_kv_rows     model.cpp:432-440
//   argmax_top2      sampler.cpp:27-30 (first maximum), engine.cpp:309-318 (runner-up scan)
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

// One wavefront per (token, head): heads [0, H) are query heads, [H, H+KV) key heads, [H+KV, H+2KV) value heads.
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
  for (int i = lane; i < D; i += 64) sh[i] = src[i];
  __syncthreads();
  if (!is_v) {
    // rmsnorm (model.cpp:46-49) over D: 16 fma chains + halving tree.
    if (lane < 16) {
      float acc = 0.0f;
      for (int i = lane; i < D; i += 16) acc = fma_(sh[i], sh[i], acc);
      acc = reduce16_lanes(acc);
      if (lane == 0) scale_s = 1.0f / sqrtf(acc / (float)D + eps);
    }
    __syncthreads();
    const float s = scale_s;
    const float* w = is_q ? q_norm : k_norm;
    for (int i = lane; i < D; i += 64) sh[i] = sh[i] * s * w[i];
    __syncthreads();
    // RoPE on pairs (i, i + D/2): clang contracts x0*c - x1*s to fma(x0, c, -(x1*s)), x0*s + x1*c to fma(x0, s, x1*c).
    const float* cs = cos_t + (int64_t)rpos[t] * (D / 2);
    const float* sn = sin_t + (int64_t)rpos[t] * (D / 2);
    for (int i = lane; i < D / 2; i += 64) {
      const float x0 = sh[i], x1 = sh[i + D / 2];
      const float c = cs[i], si = sn[i];
      sh[i] = fma_(x0, c, -(x1 * si));
      sh[i + D / 2] = fma_(x0, si, x1 * c);
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
  amax_s[lane] = amax;
  __syncthreads();
  if (lane == 0) {
    float m = 0.0f;
    for (int i = 0; i < 64; ++i) m = fmaxf(m, amax_s[i]);
    amax_s[0] = m;
  }
  __syncthreads();
  const float d = amax_s[0] / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  const int64_t row = ((int64_t)seq[t] * KV + head) * n_ctx + kv_row[t];
  int8_t* dst = (is_v ? kv.v : kv.k) + row * D;
  for (int i = lane; i < D; i += 64) dst[i] = (int8_t)(int)__builtin_rintf(sh[i] * id);
  if (lane == 0) (is_v ? kv.vs : kv.ks)[row] = d;
}

// Attention of one query head per workgroup. kRef: attend_t semantics (D in {64,128,256}, G <= 16); else the
// per-head path of attend_gqa (kernels_avx512.cpp:296-305).
template <bool kRef>
__global__ __launch_bounds__(256) void k_attention(const float* __restrict__ q, int64_t q_stride,
                                                   float* __restrict__ out, int64_t out_stride, int H, int G, int D,
                                                   float scale,
                                                   AttnAddr a, const int32_t* __restrict__ seqs,
                                                   const int32_t* __restrict__ n_keys,
                                                   const int32_t* __restrict__ anc_off,
                                                   const int32_t* __restrict__ anc) {
  const int t = blockIdx.x, h = blockIdx.y, g = h / G, tid = threadIdx.x;
  extern __shared__ float sm[];
  float* qs = sm;       // D
  float* sc = qs + D;   // keys: scores, then e^(s - max)
  __shared__ float red[256];
  __shared__ float inv_s;
  const int n0 = n_keys[t];
  const int e0 = anc_off ? anc_off[t] : 0, ne = anc_off ? anc_off[t + 1] - e0 : 0;
  const int nk = n0 + ne;
  float* pv = sc + nk;  // per key: p * v-scale (kRef) or p * inv * v-scale
  const int64_t sq = seqs[t];
  const int8_t* kb = a.k + sq * a.k_seq + g * a.k_head;
  const int8_t* vb = a.v + sq * a.k_seq + g * a.k_head;
  const char* ksb = a.ks + sq * a.s_seq + g * a.s_head;
  const char* vsb = a.vs + sq * a.s_seq + g * a.s_head;
  const float* qh = q + t * q_stride + (int64_t)h * D;
  for (int i = tid; i < D; i += 256) qs[i] = qh[i];
  __syncthreads();

  // Scores.
  for (int j = tid; j < nk; j += 256) {
    const int64_t row = j < n0 ? j : anc[e0 + j - n0];
    const int8_t* kr = kb + row * a.k_row;
    const float kscale = *reinterpret_cast<const float*>(ksb + row * a.s_row);
    float lanes[16];
    for (int l = 0; l < 16; ++l) lanes[l] = kRef ? qs[l] * (float)kr[l] : fma_(qs[l], (float)kr[l], 0.0f);
    for (int c = 16; c < D; c += 16)
      for (int l = 0; l < 16; ++l) lanes[l] = fma_(qs[c + l], (float)kr[c + l], lanes[l]);
    const float dot = reduce16(lanes);
    sc[j] = kRef ? dot * (kscale * scale) : dot * kscale * scale;
  }
  __syncthreads();

  // softmax_inplace (kernels_avx512.cpp:205-226): exact max, e = exp512(s - max), 16 sequential lane sums, tree.
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
    const float vscale = *reinterpret_cast<const float*>(vsb + row * a.s_row);
    pv[j] = kRef ? sc[j] * vscale : sc[j] * inv * vscale;
  }
  __syncthreads();

  // P.V: one sequential fma chain per output element, keys in order.
  for (int d = tid; d < D; d += 256) {
    float acc = 0.0f;
    int j = 0;
    for (; j + 4 <= nk; j += 4) {
      int64_t r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = (j + u) < n0 ? (j + u) : anc[e0 + j + u - n0];
      float vv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) vv[u] = (float)vb[r[u] * a.k_row + d];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = fma_(pv[j + u], vv[u], acc);
    }
    for (; j < nk; ++j) {
      const int64_t r = j < n0 ? j : anc[e0 + j - n0];
      acc = fma_(pv[j], (float)vb[r * a.k_row + d], acc);
    }
    out[t * out_stride + (int64_t)h * D + d] = kRef ? acc * inv : acc;
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

constexpr int kSelT = 1024;

// Top-1 under (value desc, index asc) is std::max_element's first maximum; top-2 is the best of the rest under the
// same order, which is what the reference's strict-'>' runner-up scan returns.
__global__ __launch_bounds__(kSelT) void k_argmax_top2(const float* __restrict__ logits, int n, int32_t* top1,
                                                       int32_t* top2) {
  const float* l = logits + (int64_t)blockIdx.x * n;
  Top2 t{-INFINITY, -INFINITY, 0x7fffffff, 0x7fffffff};
  for (int i = threadIdx.x; i < n; i += kSelT) push(t, l[i], i);
  __shared__ Top2 red[kSelT];
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
  if (threadIdx.x == 0) {
    top1[blockIdx.x] = red[0].i1;
    if (top2) top2[blockIdx.x] = red[0].i2;
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

}  // namespace

void greedy_advance(hipStream_t s, const int32_t* top1, int32_t* ids, int32_t* rpos, int32_t* kv_row, int32_t* n_keys,
                    int32_t* out_tokens, int32_t* counter) {
  hipLaunchKernelGGL(k_greedy_advance, dim3(1), dim3(1), 0, s, top1, ids, rpos, kv_row, n_keys, out_tokens, counter);
  check_launch("greedy_advance");
}

void qk_norm_rope_kv(hipStream_t s, float* q, float* k, const float* v, int64_t stride, int n, int H, int KV, int D,
                     const float* q_norm, const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                     const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const KvLayer& kv, int n_ctx) {
  if (n <= 0) return;
  require(D % 16 == 0, "qk_norm_rope_kv: head_dim must be a multiple of 16");
  hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3(n, H + 2 * KV), dim3(64), D * sizeof(float), s, q, k, v, stride, H, KV,
                     D, q_norm, k_norm, eps, cos_t, sin_t, rpos, seq, kv_row, kv, n_ctx);
  check_launch("qk_norm_rope_kv");
}

void attention(hipStream_t s, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int H, int KV,
               int D, float scale,
               const AttnAddr& a, const int32_t* seq, const int32_t* n_keys, const int32_t* anc_off,
               const int32_t* anc, int max_keys) {
  if (n <= 0) return;
  require(D % 16 == 0 && D <= 256 && H % KV == 0, "attention: unsupported head layout");
  const int G = H / KV;
  const size_t lds = (size_t)(D + 2 * (size_t)max_keys) * sizeof(float);
  require(lds <= 150 * 1024, "attention: too many keys for one workgroup");
  const bool ref = G <= 16 && (D == 64 || D == 128 || D == 256);
  if (ref)
    hipLaunchKernelGGL(k_attention<true>, dim3(n, H), dim3(256), lds, s, q, q_stride, out, out_stride, H, G, D, scale, a, seq,
                       n_keys, anc_off, anc);
  else
    hipLaunchKernelGGL(k_attention<false>, dim3(n, H), dim3(256), lds, s, q, q_stride, out, out_stride, H, G, D, scale, a, seq,
                       n_keys, anc_off, anc);
  check_launch("attention");
}

void move_kv_rows(hipStream_t s, int8_t* k8, int8_t* v8, float* ks, float* vs, int n_layer, int n_seq, int KV, int D,
                  int n_ctx, int seq, int from, int to) {
  if (from == to) return;
  hipLaunchKernelGGL(k_move_kv, dim3(n_layer, KV), dim3(128), 0, s, k8, v8, ks, vs, n_seq, KV, D, n_ctx, seq, from,
                     to);
  check_launch("move_kv");
}

void argmax_top2(hipStream_t s, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2) {
  if (rows <= 0) return;
  require(n_vocab >= 2, "argmax_top2: need at least two logits");
  hipLaunchKernelGGL(k_argmax_top2, dim3(rows), dim3(kSelT), 0, s, logits, n_vocab, top1, top2);
  check_launch("argmax_top2");
}

}  // namespace mk
