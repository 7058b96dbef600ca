// Library-internal launchers (throw mk::Error). The extern "C" layer and the host Model call these.
#pragma once

#include "../../../include/malkin_hip.h"
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "layout.h"

namespace mk {

// Per-token batch layout of one forward pass, resident in device memory (the reference's rpos_, kv_at_, kv_base_,
// n_keys_, anc_, anc_off_, out_ of model.h:67-83). seq replaces kv_base (= seq * n_ctx).
struct DevLayout {
  int32_t* ids;      // [n] token ids
  int32_t* rpos;     // [n] RoPE position
  int32_t* seq;      // [n] sequence
  int32_t* kv_row;   // [n] KV row written (within the sequence)
  int32_t* n_keys;   // [n] contiguous keys from row 0
  int32_t* anc_off;  // [n + 1] offsets into anc (tree mode), or null
  int32_t* anc;      // ancestor rows (within the sequence)
  int32_t* out;      // [n_out] tokens whose logits are produced
};

// Device KV cache of one layer: int8 rows [seq][kv_head][n_ctx][D] and float scales [seq][kv_head][n_ctx].
struct KvLayer {
  int8_t* k;
  int8_t* v;
  float* ks;
  float* vs;
};

size_t packed_bytes(int type, int64_t rows, int64_t cols);
// Rows r0 .. r0 + nrows of a rows x cols weight (src holds just those rows, srb bytes apart) into its packed buffer;
// r0 on an 8-row group, nrows too unless the range ends the weight.
void pack_weight_rows(hipStream_t s, int type, const void* src, size_t srb, int64_t r0, int64_t nrows, int64_t rows,
                      int64_t cols, void* dst);
void pack_weight(hipStream_t s, int type, const void* src, size_t src_row_bytes, int64_t rows, int64_t cols, void* dst);
void unpack_weight(hipStream_t s, int type, const void* packed, int64_t rows, int64_t cols, void* dst);

void quantize_q8(hipStream_t s, const float* x, int n, int64_t k, BlockQ8* xq);
void quantize_i8_rows(hipStream_t s, const float* x, int rows, int n, int8_t* q, float* d);
void dequantize_rows(hipStream_t s, int type, const void* src, size_t row_bytes, const int32_t* ids, int n, int64_t k,
                     float* dst);
void rmsnorm(hipStream_t s, const float* x, const float* w, int rows, int n, float eps, float* y,
             const int32_t* rows_idx = nullptr);
void rmsnorm_q8(hipStream_t s, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                BlockQ8* xq);
void silu_mul(hipStream_t s, int64_t n, float* g, const float* u);
// Per row of gu ([gate | up], 2n floats at stride 2n): gate = silu(gate) * up in place.
void silu_mul_rows(hipStream_t s, float* gu, int rows, int64_t n);
// matmul's row path (quant.cpp:171-191, 330-351) over GGUF rows: fp32 x for F32/F16/BF16, BlockQ8 xq otherwise.
bool rows_supported(int type, int64_t cols);
// The Q4_K / Q5_K panel arithmetic (gemm_avx512.cpp:104-155, 217-266) over GGUF rows: Q5_K's device path.
void matmul_gguf(hipStream_t s, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols,
                 const BlockQ8* xq, int n, float* y, int64_t ys, bool accumulate);
void matmul_rows(hipStream_t s, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols, const float* x,
                 int64_t xs, const BlockQ8* xq, int n, float* y, int64_t ys, bool accumulate);
// gu rows of 2n floats: [gate | up], or (interleave4) gate/up interleaved by 4 as matmul_f32's silu_pairs rows.
void silu_mul_q8(hipStream_t s, const float* gu, int rows, int64_t n, BlockQ8* xq, bool interleave4 = false);
void add(hipStream_t s, int64_t n, float* x, const float* h);
void fill(hipStream_t s, void* p, int value, size_t bytes);
// p[0..3] = a, b, c, d (p 16-byte aligned), in stream order.
void put4(hipStream_t s, int32_t* p, int a, int b, int c, int d);

// y[t * ys + r] (+)= W[r] . xq[t]; wide: Q6_K wide-panel arithmetic for n > 16.
void matmul(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* xq, int n,
            float* y, int64_t ys, bool accumulate);

// Activations of a decode GEMV given as fp32 rows xf[t * xfs + i]: quantized to BlockQ8 inside the matmul, after
// rmsnorm with weights nw (eps) when nw is not null (model.cpp:46-49, 362-364, 403-405). Same results as
// rmsnorm_q8 / quantize_q8 followed by matmul.
struct GemvIn {
  const BlockQ8* xq;
  const float* xf;
  int64_t xfs;
  const float* nw;
  float eps;
};
// Whether matmul_f32 has a fused kernel for this shape (decode: n <= 2, cols % 32 == 0; with rmsnorm cols <= 8192).
bool matmul_f32_supported(int type, bool wide, int64_t rows, int64_t cols, int n, bool norm);
// silu_pairs: the rows are gate/up pairs interleaved by 4 (each 8-row group: 4 gate rows, then the 4 up rows of the
// same outputs); y[t * ys + i] = silu(gate_i) * up_i for i < rows / 2 (kernels_avx512.cpp:271-280).
void matmul_f32(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const float* xf,
                int64_t xfs, const float* nw, float eps, int n, float* y, int64_t ys, bool accumulate,
                bool silu_pairs);

// Prefill GEMM for Q8_0 on int8 MFMA (same results as matmul's GEMV); supported for rows % 32 == 0 and n > 8.
bool gemm_q8_0_supported(int64_t rows, int64_t cols, int n);
void gemm_q8_0(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
               bool accumulate);
// The same for Q4_K and Q6_K (Q6_K: wide-panel arithmetic when wide and n > 16); rows % 32 == 0, cols % 256 == 0, n > 8.
bool gemm_kq_supported(int type, int64_t rows, int64_t cols, int n);
void gemm_kq(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n,
             float* y, int64_t ys, bool accumulate);

// Short batches (1..32 tokens) of any quantized type on int8 MFMA, 16-row x 16-token tiles streamed through a deep LDS
// ring (same results as matmul's other kernels); rows % 32 == 0, cols % 256 == 0. ksplit: four waves per 16-row tile
// (matrices with few rows), else one.
bool mmv_supported(int type, int64_t rows, int64_t cols, int n);
void mmv(hipStream_t s, int type, bool wide, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n,
         float* y, int64_t ys, bool accumulate, bool ksplit);

// Generic attention addressing: key row (t, g, row) at k + seq*k_seq + g*k_head + row*k_row (bytes), its scale at
// ks + seq*s_seq + g*s_head + row*s_row (bytes); values likewise with v / vs.
// k_perm: K rows are stored permuted (kv_perm below), as the device KV cache keeps them; else in element order.
struct AttnAddr {
  const int8_t* k;
  const int8_t* v;
  const char* ks;
  const char* vs;
  int64_t k_seq, k_head, k_row;
  int64_t s_seq, s_head, s_row;
  int k_perm;
};

// Byte position of element e in a permuted K row of D = 16 * DC values: the DC values a reference lane l
// (kernels_avx512.cpp:234-244) multiplies, e = 16 c + l for c < DC, are contiguous at DC * l.
__host__ __device__ constexpr int kv_perm(int e, int DC) { return DC * (e & 15) + (e >> 4); }
// With xq (D % 32 == 0) both also write the BlockQ8 rows of out (token t's H*D/32 blocks at xq + t * xq_stride), as
// quantize_q8 of out would, so the attn_output matmul needs no separate quantization launch.
// q [n][H*D] (token stride q_stride floats), out [n][H*D] (stride out_stride). Per token t: keys rows
// 0..n_keys[t]-1 of sequence seq[t], then anc[anc_off[t] .. anc_off[t+1]) when anc_off is non-null. Rows with more
// keys than one workgroup's LDS holds keep their scores in `scratch` (attention_scratch_bytes of it for full speed;
// a smaller scratch runs fewer workgroups at a time; one without room for a single row fails).
void attention(hipStream_t s, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int H, int KV,
               int D, float scale,
               const AttnAddr& a, const int32_t* seq, const int32_t* n_keys, const int32_t* anc_off,
               const int32_t* anc, int max_keys, void* scratch, size_t scratch_bytes, BlockQ8* xq = nullptr,
               int64_t xq_stride = 0);
// Scratch the attention of `pairs` (token, head) pairs over max_keys keys uses (0: none).
size_t attention_scratch_bytes(int D, int max_keys, int pairs);

// qk_norm_rope_kv followed by attention in one launch, for batches whose tokens are plain (no tree) and belong to
// distinct sequences, so that no token reads another's new KV row. qkv rows: H query heads, KV key heads, KV value
// heads (raw), token stride `stride`. Returns false (nothing launched) where the fused kernel does not apply.
bool attention_decode_fused(hipStream_t s, const float* qkv, int64_t stride, float* out, int64_t out_stride, int n,
                            int H, int KV, int D, float scale, const AttnAddr& a, const float* q_norm,
                            const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                            const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys,
                            const KvLayer& kv, int n_ctx, int max_keys, BlockQ8* xq = nullptr,
                            int64_t xq_stride = 0);

// The weights of one decoder layer for the persistent decode kernel: Q8_0 packed q|k|v rows (H + 2 KV heads of D), the
// attn_output rows, gate|up rows interleaved by 4 (matmul_f32's silu_pairs layout) and the down rows; the layer's
// norm weights.
struct DecodeLayer {
  const void* qkv;
  const void* wo;
  const void* gate_up;
  const void* down;
  const float* attn_norm;
  const float* ffn_norm;
  const float* q_norm;
  const float* k_norm;
};
// Layers [l0, l1) of a one-token decode step (model.cpp:355-417 at n = 1) in one persistent launch, one workgroup
// per CU: x += every layer's attention and FFN, with the same results as the per-step launches (matmul_f32 with the
// rmsnorm / silu / residual forms, attention_decode_fused with BlockQ8 output). The kernel's argument block lives in
// device memory (decode_args_bytes), written once by decode_set_args:
//   layers   device array of the model's layers;
//   kv0      layer 0 of the cache (KV heads, n_ctx rows per head, n_seq sequences);
//   qkv [(H + 2 KV) D], att (BlockQ8 [H D / 32]), h [F]: the step's scratch rows;
//   rpos, seq, kv_row, n_keys: the token's layout on the device (one entry each);
//   sync     decode_sync_bytes(layers per launch) bytes, zero before the first launch (each launch leaves them zero).
// A wait longer than spin_max polls sets the error word (word decode_error_word(layers per launch) of sync): the
// launch's results are then invalid.
struct DecodeDims {
  int E, H, KV, D, F, n_ctx, n_seq;
  float eps;
};
struct DecodeBufs {
  const DecodeLayer* layers;
  KvLayer kv0;
  float* x;
  float* qkv;
  void* att;
  float* h;
  const float* cos_t;
  const float* sin_t;
  const int32_t* rpos;
  const int32_t* seq;
  const int32_t* kv_row;
  const int32_t* n_keys;
  unsigned* sync;
  unsigned spin_max;
};
bool decode_layers_supported(const DecodeDims& d, int max_keys);
int decode_ring(const DecodeDims& d, int max_keys);
size_t decode_sync_bytes(int n_layer);
size_t decode_error_word(int n_layer);
size_t decode_args_bytes();
void decode_set_args(void* dev_args, const DecodeDims& d, const DecodeBufs& b);
void decode_layers(hipStream_t s, const void* dev_args, const DecodeDims& d, int l0, int l1, int max_keys);
// Layer `layer`'s attention and attn_output GEMV in one launch (the q|k|v output in place; sync sized for n_layer).
void decode_attn_wo(hipStream_t s, const void* dev_args, const DecodeDims& d, int layer, int n_layer, int max_keys);

// QK-norm + RoPE on q [n][H*D] and k [n][KV*D] (in place), then k, v quantized into the KV cache (model.cpp:370-392).
// cos/sin tables [n_pos][D/2].
void qk_norm_rope_kv(hipStream_t s, float* q, float* k, const float* v, int64_t stride, int n, int H, int KV, int D,
                     const float* q_norm, const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                     const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const KvLayer& kv, int n_ctx);

// Scratch: argmax_scratch_bytes(rows) of device memory (per-row partial results).
size_t argmax_scratch_bytes(int rows);
// argmax_top2 with its partial results in a file-scope device array (one per GPU, kNoAllocSelectRows rows): no
// allocation, no context. Calls that overlap on one GPU race on that array.
constexpr int kNoAllocSelectRows = 256;
void argmax_top2_noalloc(hipStream_t s, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2);
void argmax_top2(hipStream_t s, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2,
                 void* scratch, size_t scratch_bytes);

// Stochastic sampling's candidate selection (sampler.cpp:24-36). Row r of a launch is logits row rows[r] (rows null:
// row r) of `stride` floats. penalize: l[pen_id[i]] -= pen_amt[i] for i in pen_off[r] .. pen_off[r + 1] (ids outside
// the vocabulary skipped). topk: the k (1..1024) largest logits of each row, highest first, ties by lower id, into
// values / ids [n_rows][k].
void penalize(hipStream_t s, float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
              const int32_t* pen_off, const int32_t* pen_id, const float* pen_amt);
void topk(hipStream_t s, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab, int k,
          float* values, int32_t* ids);
size_t sample_cut_workspace(int n_rows, int n_vocab);
void sample_cut(hipStream_t s, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
                const mk_cut_params* params, int cap, float* values, int32_t* ids, int32_t* keep, double* sums,
                void* workspace, size_t workspace_bytes);
void sample_cut_tail(hipStream_t s, void* workspace, int n_rows, int n_vocab, int row, int from, int count,
                     float* values, int32_t* ids);
// One draw per top-k row from its std::mt19937_64 state (MK_MT64_WORDS words each, advanced in place).
void sample_draw(hipStream_t s, const float* values, const int32_t* ids, int stride, int n_rows,
                 const mk_draw_params* params, uint64_t* states, int n_states, int32_t* out, int n_out);

// dst[dst_idx[i]] = src[src_idx[i]], i < n; null index arrays are the identity, negative indices skip.
void move_ids(hipStream_t s, int32_t* dst, const int32_t* dst_idx, const int32_t* src, const int32_t* src_idx,
              int n);
void greedy_advance(hipStream_t s, const int32_t* top1, int32_t* ids, int32_t* rpos, int32_t* kv_row, int32_t* n_keys,
                    int32_t* out_tokens, int32_t* counter);

// Copies KV rows (all layers' K and V of one sequence): row from -> row to (model.cpp:432-440). The cache is one
// allocation per K / V / K-scale / V-scale: [layer][seq][kv_head][n_ctx] rows.
void move_kv_rows(hipStream_t s, int8_t* k8, int8_t* v8, float* ks, float* vs, int n_layer, int n_seq, int KV, int D,
                  int n_ctx, int seq, int from, int to);

}  // namespace mk
