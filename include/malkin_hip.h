/*
 * malkin-mi355x: C ABI of the gfx950 kernels (libmalkin_hip.so).
 *
 * This is the device-side replacement of the reference's per-ISA operator surface, malkin::kern (src/kernels.h) and
 * the quantization / matmul API of src/quant.h. Each entry point cites the reference interface it replaces. Unlike
 * the reference's per-panel functions, every call here works on a whole batch in device memory.
 *
 * Conventions:
 *   - every function returns MK_OK (0) or an MK_ERR_* status; mk_last_error() holds the message (thread-local),
 *     worded like the reference's std::runtime_error texts where one exists;
 *   - pointers named *_dev, and every tensor argument, are device pointers (mk_malloc); sizes are element counts;
 *   - all work is queued on the context's one HIP stream, in call order; mk_synchronize waits for it;
 *   - BlockQ8 activation blocks keep the reference's 40-byte layout (quant.h:11-16): float d; int16 s[2]; int8 qs[32].
 */
#ifndef MALKIN_HIP_H
#define MALKIN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MK_OK = 0,
  MK_ERR_INVALID = 1,     /* bad argument; the reference throws std::runtime_error / std::invalid_argument */
  MK_ERR_HIP = 2,         /* HIP runtime error */
  MK_ERR_UNSUPPORTED = 3, /* type / shape without a kernel (the reference's panel_bytes == 0 row-path case) */
  MK_ERR_NO_DEVICE = 4
};

/* ggml tensor types (gguf.h:12-29) accepted by the kernels. F16 / BF16 / Q5_K: row path (mk_matmul_rows) and
   embedding lookup. */
enum { MK_F32 = 0, MK_F16 = 1, MK_Q8_0 = 8, MK_Q4_K = 12, MK_Q5_K = 13, MK_Q6_K = 14, MK_BF16 = 30 };

typedef struct mk_ctx mk_ctx;

/* ---- context (no reference counterpart: the CPU build has no device) ---- */
int mk_init(int device, mk_ctx** ctx);
int mk_destroy(mk_ctx* ctx);
/* Name of the device architecture this library runs on (replaces kern::isa_name, kernels.h:84). */
const char* mk_device_name(const mk_ctx* ctx);
const char* mk_last_error(void);
int mk_synchronize(mk_ctx* ctx);
/* Grows the context's device scratch buffer to at least `bytes` (never shrinks; waits for the stream first). Calls
   that use the scratch (mk_attention on rows longer than one workgroup's LDS, mk_argmax_top2) then run without
   allocating, also under graph capture. No reference counterpart (the CPU engine's scratch is host memory). */
int mk_reserve_scratch(mk_ctx* ctx, size_t bytes);
/* Scratch mk_attention needs for `pairs` (token, query head) pairs over up to max_keys keys: 0 while a row fits in
   one workgroup's LDS (about 7600 keys at head_dim 128); beyond that, global slots of 2 floats per key per pair
   (up to 1024 pairs at once). */
size_t mk_attention_scratch_bytes(int head_dim, int max_keys, int pairs);
/* Host waits on the device made by this library so far (stream and event synchronizations, including those inside
   mk_upload / mk_download / mk_free), for tests that bound the waits of a token loop. */
uint64_t mk_host_waits(void);
/* Bytes this library has copied from device memory into host memory so far (mk_download, and mk_copy_async into
   pinned memory), for tests that bound what a token loop downloads. */
uint64_t mk_host_bytes(void);
/* The context's hipStream_t. */
void* mk_stream(mk_ctx* ctx);

/* ---- device memory (replaces PackedBuffer / LazyBytes ownership, quant.h:34-42, gguf.h:82-95) ---- */
int mk_malloc(mk_ctx* ctx, size_t bytes, void** dev);
int mk_free(mk_ctx* ctx, void* dev);
int mk_upload(mk_ctx* ctx, void* dev_dst, const void* host_src, size_t bytes);
int mk_download(mk_ctx* ctx, void* host_dst, const void* dev_src, size_t bytes);
/* Fills with a kernel (safe inside captured graphs). */
int mk_fill(mk_ctx* ctx, void* dev, int byte_value, size_t bytes);
/* Pinned host memory (hipHostMalloc) for asynchronous copies; mk_host_free waits for the stream first. */
int mk_host_alloc(mk_ctx* ctx, size_t bytes, void** host);
int mk_host_free(mk_ctx* ctx, void* host);
/* Copy of `bytes` in stream order without waiting (any direction; host memory must be pinned and stay untouched until
   the copy has run: record an event after it and wait for that event before reusing the memory). */
int mk_copy_async(mk_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Records *event (created on first use) at the current end of the stream / waits on the host until it has passed. */
int mk_event_record(mk_ctx* ctx, void** event);
int mk_event_wait(mk_ctx* ctx, void* event);
/* 1 when the event has passed (or is NULL), 0 while work before it is pending; never waits. */
int mk_event_done(void* event);
int mk_event_free(void* event);

/* ---- timing on the context stream (bench) ---- */
int mk_timer_start(mk_ctx* ctx);
int mk_timer_stop(mk_ctx* ctx, float* ms);

/* ---- load-time repack (replaces kern::panel_rows / panel_bytes / pack_panel, kernels.h:67-73, and
 *      quant.h:129-134 packed_bytes / pack_weight_into) ---- */
/* Bytes of the CDNA-packed form of a rows x cols weight; 0 = no kernel for this type/shape (rows % 8 or block). */
size_t mk_packed_bytes(int type, int64_t rows, int64_t cols);
/* src_dev: rows of GGUF blocks, src_row_bytes apart. dst_dev: mk_packed_bytes bytes. */
int mk_pack_weight(mk_ctx* ctx, int type, const void* src_dev, size_t src_row_bytes, int64_t rows, int64_t cols,
                   void* dst_dev);
/* mk_pack_weight for rows row0 .. row0 + n_rows of a rows x cols weight, src_dev holding only those rows (a chunk of a
   weight streamed from the file): row0 a multiple of 8, n_rows too unless the chunk ends the weight. Chunks packed in
   any order fill the same buffer mk_pack_weight fills. */
int mk_pack_weight_rows(mk_ctx* ctx, int type, const void* src_dev, size_t src_row_bytes, int64_t row0, int64_t n_rows,
                        int64_t rows, int64_t cols, void* dst_dev);
/* Inverse of mk_pack_weight: GGUF rows, ggml_row_size(type, cols) bytes apart (pack round-trip tests). */
int mk_unpack_weight(mk_ctx* ctx, int type, const void* packed_dev, int64_t rows, int64_t cols, void* dst_dev);

/* ---- activations ---- */
/* x [n][k] f32 -> xq [n][k/32] BlockQ8 (replaces kern::quantize_row_q8, kernels.h:28; quantize_acts, quant.h:151). */
int mk_quantize_q8(mk_ctx* ctx, const float* x, int n, int64_t k, void* xq);
/* Per row of n floats: q = round(x / d), d = max|x| / 127 (replaces quantize_i8, quant.h:144). */
int mk_quantize_i8(mk_ctx* ctx, const float* x, int rows, int n, int8_t* q, float* d);
/* Rows ids[i] of a GGUF matrix (row_bytes apart) dequantized to f32 [n][k] (dequantize_row, quant.h:145; the token
   embedding lookup of model.cpp:331-334). */
int mk_dequantize_rows(mk_ctx* ctx, int type, const void* src, size_t row_bytes, const int32_t* ids, int n, int64_t k,
                       float* dst);

/* ---- matmul (replaces matmul / matmul_group, quant.h:154-161, and kern::gemm_panels, kernels.h:80) ---- */
typedef struct {
  int32_t type;  /* MK_Q8_0, MK_Q4_K, MK_Q6_K */
  int32_t wide;  /* Q6_K only: the weight also has the reference's wide panels, used for n > 16 (quant.h:50) */
  int64_t rows, cols;
  const void* data; /* mk_pack_weight output */
} mk_weight;

/* y[t * y_stride + r] (+)= row r . xq[t] for t < n, r < rows. accumulate != 0 adds to y (the residual add x += h of
   model.cpp:352-356 fused into the epilogue). Results are bit-identical to the reference's panel kernels. */
int mk_matmul(mk_ctx* ctx, const mk_weight* w, const void* xq, int n, float* y, int64_t y_stride, int accumulate);
/* The same matmul from fp32 activations x[t * x_stride + i]: rmsnorm with norm_w (when not NULL, eps) and
   quantize_row_q8 run inside the matmul, bit-identical to mk_rmsnorm_q8 / mk_quantize_q8 followed by mk_matmul
   (replaces the rmsnorm -> quantize_acts -> matmul sequences of model.cpp:362-365, 403-406 and the quantize_acts ->
   matmul of 397-399). For 1 or 2 tokens and a multiple of 32 columns (<= 8192 with rmsnorm); MK_ERR_UNSUPPORTED
   otherwise.
   silu_pairs != 0: the weight's rows are gate/up pairs interleaved by 4 (each 8-row group: 4 ffn_gate rows, then
   the 4 ffn_up rows of the same outputs) and y[t * y_stride + i] = silu(gate_i) * up_i for i < rows / 2, the
   kern::silu_mul of model.cpp:409 fused into the gate/up matmul (no accumulate). */
int mk_matmul_f32(mk_ctx* ctx, const mk_weight* w, const float* x, int64_t x_stride, const float* norm_w, float eps,
                  int n, float* y, int64_t y_stride, int accumulate, int silu_pairs);

/* matmul's row path (quant.cpp:171-191 vec_dot, 330-351 matmul; kernels_avx512.cpp:82-171): y[t * y_stride + r]
   (+)= vec_dot(row r, token t) over a weight kept as GGUF rows (row_bytes apart, not repacked). The reference takes
   this path for F32 / F16 / BF16 weights and, under MALKIN_NO_PACK, for Q8_0 / Q4_K / Q5_K / Q6_K; its arithmetic
   differs from the panel kernels', and the results here are bit-identical to it. x: fp32 activations (x_stride
   apart), read by F32 / F16 / BF16; xq: their BlockQ8 rows, read by the quantized types. */
int mk_matmul_rows(mk_ctx* ctx, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols, const float* x,
                   int64_t x_stride, const void* xq, int n, float* y, int64_t y_stride, int accumulate);

/* The reference's Q4_K / Q5_K panel arithmetic (gemm_avx512.cpp:104-155 compact, 217-266 wide: one sequence per output
   over its 32-value sub-blocks, acc = fma(float(int dot), (d*sc)*dx, acc), acc = fma(-(dmin*m), dx*(s0+s1), acc)) read
   straight from GGUF rows: the device path of Q5_K weights, which have no CDNA layout. Same results as mk_matmul's
   packed Q4_K kernels for Q4_K. */
int mk_matmul_gguf(mk_ctx* ctx, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols, const void* xq,
                   int n, float* y, int64_t y_stride, int accumulate);

/* ---- elementwise (model.cpp:46-49, kernels.h:39) ---- */
/* y = rmsnorm(x) * w per row of n floats (model.cpp:46-49). */
int mk_rmsnorm(mk_ctx* ctx, const float* x, const float* w, int rows, int n, float eps, float* y);
/* rmsnorm of rows x[rows_idx[i]] (all rows when rows_idx is NULL) quantized straight to BlockQ8 [rows][n/32]. */
int mk_rmsnorm_q8(mk_ctx* ctx, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                  void* xq);
/* y[i] = rmsnorm(x[rows_idx[i]]) * w (all rows in order when rows_idx is NULL), fp32 (model.cpp:46-49, 419-421). */
int mk_rmsnorm_rows(mk_ctx* ctx, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                    float* y);
/* Rows [gate | up] (2n floats apart): gate = silu(gate) * up in place (kern::silu_mul per token, model.cpp:409). */
int mk_silu_mul_rows(mk_ctx* ctx, float* gu, int rows, int64_t n);
/* g = g / (1 + e^-g) * u (kern::silu_mul, kernels.h:39). */
int mk_silu_mul(mk_ctx* ctx, int64_t n, float* g, const float* u);
/* silu_mul of rows of gu (2n floats per row) quantized to BlockQ8 [rows][n/32] (model.cpp:409-411). gu rows are
   [gate | up], or, with interleave4, gate/up rows interleaved by 4 as in mk_matmul_f32's silu_pairs weights. */
int mk_silu_mul_q8(mk_ctx* ctx, const float* gu, int rows, int64_t n, int interleave4, void* xq);
/* x += h (model.cpp:352-356). */
int mk_add(mk_ctx* ctx, int64_t n, float* x, const float* h);

/* ---- attention (replaces kern::attend_gqa, kernels.h:55-56) ----
 * One query token, G heads sharing one KV head; keys/values 0..n-1 at k + j * stride (bytes), then rows extra[i];
 * value = scale(row) * q, the float scale soff bytes after the row's first value. D % 16 == 0. */
int mk_attend_gqa(mk_ctx* ctx, const float* q, int G, int D, const int8_t* k, const int8_t* v, size_t stride,
                  ptrdiff_t soff, int n, float scale, float* out, const int32_t* extra, int ne);

/* ---- device KV cache (replaces the reference's int8 LazyBytes kcache_ / vcache_, model.h:91, model.cpp:105-110) ----
 * Rows of head_dim int8 values with one float scale per row, indexed [layer][seq][kv_head][position]. V rows hold
 * the values in order; K rows are permuted so that the head_dim / 16 values one lane of the reference's scoring loop
 * multiplies are contiguous: element e sits at byte (head_dim / 16) * (e % 16) + e / 16. */
typedef struct {
  int8_t* k;
  int8_t* v;
  float* k_scale;
  float* v_scale;
  int32_t n_layer, n_seq, n_head_kv, head_dim, n_ctx;
} mk_kv_cache;

/* model.cpp:370-392, per token t: QK-norm (rmsnorm with q_norm / k_norm) and NeoX RoPE at position rpos[t] on the
   n_head query heads of q and the key heads of k (in place), then k and v quantized (quantize_i8) into KV row
   kv_row[t] of sequence seq[t] of `layer`. q, k, v share the token stride; cos_t / sin_t are [n_ctx][head_dim/2]. */
int mk_qk_norm_rope_kv(mk_ctx* ctx, float* q, float* k, const float* v, int64_t stride, int n, int n_head,
                       const float* q_norm, const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                       const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const mk_kv_cache* kv,
                       int layer);
/* mk_qk_norm_rope_kv followed by mk_attention in one launch (model.cpp:370-392 then 204-247), for batches whose
   tokens are all plain (no tree: keys 0..n_keys[t]-1, the last being the token's own row kv_row[t]) and belong to
   distinct sequences, so that no token attends to another token's new KV row. qkv[t * stride ...]: the n_head query
   heads, then the n_head_kv key heads, then the n_head_kv value heads, raw (before QK-norm and RoPE; not modified).
   The KV rows kv_row[t] are written as mk_qk_norm_rope_kv writes them; out as mk_attention. MK_ERR_UNSUPPORTED
   (nothing launched) where the fused kernel does not apply (head_dim other than 64 / 128, more than 16 query heads per
   KV head, or max_keys beyond its LDS capacity); the caller then uses the two calls. */
int mk_attention_decode(mk_ctx* ctx, const float* qkv, int64_t stride, int n, int n_head, const float* q_norm,
                        const float* k_norm, float eps, const float* cos_t, const float* sin_t, const int32_t* rpos,
                        const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys, const mk_kv_cache* kv,
                        int layer, float* out, int64_t out_stride, int max_keys);
/* Model::attention (model.cpp:204-247) over the device cache: token t attends with its n_head query heads to rows
   0..n_keys[t]-1 of sequence seq[t], then (tree verification) rows anc[anc_off[t] .. anc_off[t+1]) when anc_off is
   not NULL: the KV rows of its ancestors in the batch (model.h:83), so at most n of them. max_keys bounds
   n_keys[t] + ancestors for every t. Rows longer than one workgroup's LDS holds use the
   context's scratch (mk_reserve_scratch, mk_attention_scratch_bytes); with none reserved they fail. */
int mk_attention(mk_ctx* ctx, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int n_head,
                 const mk_kv_cache* kv, int layer, const int32_t* seq, const int32_t* n_keys, const int32_t* anc_off,
                 const int32_t* anc, int max_keys);
/* mk_attention and mk_attention_decode that also write the BlockQ8 rows of `out` into xq: token t's
   n_head * head_dim / 32 blocks at xq + t * n_head * head_dim / 32 blocks, byte-identical to mk_quantize_q8(out) (the
   reference quantizes the attention output right after attention, model.cpp:398-401; this fuses that launch away).
   head_dim % 32 == 0. Same outputs, errors and MK_ERR_UNSUPPORTED cases as the calls they extend. */
int mk_attention_q8(mk_ctx* ctx, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int n_head,
                    const mk_kv_cache* kv, int layer, const int32_t* seq, const int32_t* n_keys,
                    const int32_t* anc_off, const int32_t* anc, int max_keys, void* xq);
int mk_attention_decode_q8(mk_ctx* ctx, const float* qkv, int64_t stride, int n, int n_head, const float* q_norm,
                           const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                           const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys,
                           const mk_kv_cache* kv, int layer, float* out, int64_t out_stride, int max_keys, void* xq);
/* Model::move_kv (model.cpp:432-440): row `from` -> row `to` of sequence seq, K and V of every layer. */
int mk_move_kv(mk_ctx* ctx, const mk_kv_cache* kv, int seq, int from, int to);

/* ---- persistent decode step: the layer loop of Model::run for one token (model.cpp:355-417 at n = 1) ----
 * Per layer: rmsnorm + q|k|v, QK-norm + RoPE + KV write + attention, attn_output + residual, rmsnorm + gate|up,
 * silu * up, down + residual; all layers of a step in one launch, one workgroup per CU handing off between the steps
 * through device counters. Results are bit-identical to the per-step calls (mk_matmul_f32 with norm_w, silu_pairs
 * and accumulate; mk_attention_decode_q8). */
typedef struct {
  mk_weight qkv;     /* MK_Q8_0: q|k|v rows, (n_head + 2 n_head_kv) head_dim x n_embd */
  mk_weight wo;      /* MK_Q8_0: n_embd x n_head head_dim */
  mk_weight gate_up; /* MK_Q8_0: 2 n_ff x n_embd, gate/up rows interleaved by 4 (mk_matmul_f32's silu_pairs rows) */
  mk_weight down;    /* MK_Q8_0: n_embd x n_ff */
  const float* attn_norm;
  const float* ffn_norm;
  const float* q_norm;
  const float* k_norm;
} mk_decode_layer;
typedef struct mk_decode_plan mk_decode_plan;
/* A plan for one model: device copies of the layer table and of the kernel's argument block, and its hand-off
   counters (allocated here, once). Device buffers: x [n_embd] (the residual stream, updated in place), qkv
   [(n_head + 2 n_head_kv) head_dim], att (BlockQ8 rows of n_head head_dim / 32 blocks), h [n_ff]; the token's layout
   rpos, seq, kv_row, n_keys (one entry each); cos_t / sin_t as for mk_qk_norm_rope_kv. MK_ERR_UNSUPPORTED (no plan)
   where the kernel does not apply: other weight types, head_dim other than 128, rows of 48 blocks or fewer, more
   than 16 query heads per KV head, no more CUs than query heads. */
int mk_decode_plan_create(mk_ctx* ctx, const mk_decode_layer* layers, int n_layer, int n_head, float eps,
                          const mk_kv_cache* kv, float* x, float* qkv, void* att, float* h, const float* cos_t,
                          const float* sin_t, const int32_t* rpos, const int32_t* seq, const int32_t* kv_row,
                          const int32_t* n_keys, mk_decode_plan** plan);
int mk_decode_plan_destroy(mk_decode_plan* plan);
/* 1 if mk_decode_layers runs for a token with up to max_keys keys (its LDS holds them), else 0. */
int mk_decode_supported(const mk_decode_plan* plan, int max_keys);
/* Queues layers [l0, l1) of one decode step on the context's stream; allocates nothing (graph-capturable). Every
   cross-workgroup wait inside is bounded; a wait that runs out marks the plan's error word (mk_decode_check). */
int mk_decode_layers(mk_ctx* ctx, mk_decode_plan* plan, int l0, int l1, int max_keys);
/* Model::run's attention and attn_output steps of layer `layer` for one token (model.cpp:370-401 at n = 1) in one
   launch: after the layer's q|k|v matmul has written qkv, the attention (QK-norm, RoPE, KV write, BlockQ8 output)
   runs on n_head workgroups while the others load their attn_output weights, then x += W_o . att. Same results as
   mk_attention_decode_q8 followed by mk_matmul (accumulate); same support rule and error word as
   mk_decode_layers. */
int mk_decode_attn_wo(mk_ctx* ctx, mk_decode_plan* plan, int layer, int max_keys);
/* After the stream has been synchronized: MK_OK, or MK_ERR_HIP if a launch since the last check timed out in a
   hand-off wait (its results are invalid); the error word and the counters are then cleared. */
int mk_decode_check(mk_ctx* ctx, mk_decode_plan* plan);

/* ---- greedy selection (sampler.cpp:27-30 argmax; engine.cpp:309-318 draft top-2) ---- */
/* Per row of n_vocab logits: top1 = first maximum, top2 = the reference's runner-up scan. top2 may be NULL. */
int mk_argmax_top2(mk_ctx* ctx, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2);
/* mk_argmax_top2 that allocates nothing and needs no context. No counterpart in the reference: it is for callers
   that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
   hipMalloc). The per-row partial results live in a file-scope device array of the library sized for 256 rows
   (256 KiB on each GPU it runs on, held until the process ends); more rows fail with MK_ERR_INVALID. stream: a
   hipStream_t (NULL: the current device's null stream); the work is queued on it and the call does not wait. Every
   call on one GPU shares that array, so calls that overlap on one GPU (two streams) race; calls in one stream's
   order do not. Results are identical to mk_argmax_top2's. */
int mk_argmax_top2_noalloc(void* stream, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2);
/* ---- stochastic sampling: candidate selection (sampler.cpp:22-36) ---- */
/* Row r of a call is logits row rows[r] (rows NULL: row r), `stride` floats apart; rows, pen_* are device arrays.
   mk_penalize: the repetition penalties in place (sampler.cpp:24-26), l[pen_id[i]] -= pen_amt[i] for i in
   pen_off[r] .. pen_off[r + 1] (pen_off has n_rows + 1 entries; ids outside 0..n_vocab-1 are skipped). */
int mk_penalize(mk_ctx* ctx, float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
                const int32_t* pen_off, const int32_t* pen_id, const float* pen_amt);
/* The top-k cut of Sampler::distribution (sampler.cpp:32-36, std::partial_sort by value): per row the k largest
   logits, highest first, into values / ids [n_rows][k]. k = 1..1024 and at most n_vocab. Equal logits are ordered
   by lower id (the reference leaves their order unspecified). One workgroup per row: radix select of the k-th
   largest value, then a sort of the k candidates in LDS. */
int mk_topk(mk_ctx* ctx, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab, int k,
            float* values, int32_t* ids);
/* Per-row parameters of mk_sample_cut: candidates k (<= 0: the whole vocabulary) and the request's temperature
   (> 0), min_p and top_p. */
typedef struct {
  int32_t k;
  float temperature, min_p, top_p;
} mk_cut_params;
/* The rest of Sampler::distribution for candidate counts above mk_topk's 1024 (top_k <= 0 or > 1024), sampler.cpp:
   27-56, so that such a row is not downloaded whole: per row the k largest logits sorted (highest first, equal
   logits by lower id), their weights exp((l - l_max) / T) (float), the total in double in that order, and the kept
   count (the first candidate, then candidates while the weight is at least min_p times the first, up to the one
   whose running sum reaches top_p of the total). Writes keep[r], sums[r] and the first min(keep[r] + 1, k, cap)
   candidates to values / ids [n_rows][cap] (device arrays; params too). The weights are computed as the correctly
   rounded float of exp (the reference's C library expf agrees except within ~2^-60 of a rounding boundary): the
   caller recomputes the kept weights itself. workspace: at least mk_sample_cut_workspace(n_rows, n_vocab) device
   bytes, which also keep the sorted rows for mk_sample_cut_tail until the next call. */
size_t mk_sample_cut_workspace(int n_rows, int n_vocab);
int mk_sample_cut(mk_ctx* ctx, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
                  const mk_cut_params* params, int cap, float* values, int32_t* ids, int32_t* keep, double* sums,
                  void* workspace, size_t workspace_bytes);
/* Candidates [from, from + count) of row `row` of the last mk_sample_cut on this workspace (a kept head longer than
   its cap), into values / ids (device arrays). */
int mk_sample_cut_tail(mk_ctx* ctx, void* workspace, int n_rows, int n_vocab, int row, int from, int count,
                       float* values, int32_t* ids);

/* A std::mt19937_64 generator on the device: its 312 state words, then the index of the next word to temper
   (312 right after seeding: the next output regenerates the state first). */
#define MK_MT64_WORDS 313
/* Per-row parameters of mk_sample_draw. */
typedef struct {
  int32_t k;                        /* candidates of the row (1 .. stride), highest first */
  float temperature, min_p, top_p;  /* temperature > 0 */
  int32_t state;                    /* the row's generator: states + MK_MT64_WORDS * state, 0 .. n_states - 1 */
  int32_t dst;                      /* out[dst] receives the drawn id, 0 .. n_out - 1 */
} mk_draw_params;
/* Sampler::sample over rows already cut to their top k (mk_topk's values / ids [n_rows][stride], stride 1..1024),
   sampler.cpp:27-56 and 108-116, as the draft's proposals draw it (engine.cpp:319-323): per row the weights
   exp((l - l_max) / T) as floats, the total in double in order, the kept head (min_p floor, top_p nucleus), the
   probabilities weight / (kept total) rounded to float, and, when more than one candidate is kept, one
   u = uniform(generator) and the first candidate where the running u - p_i reaches zero (the last if none does).
   The row's generator is advanced in place; a one-candidate head draws nothing. Rows run in parallel: two rows of
   one call must not share a generator. The weights are the correctly rounded float of exp, which the C library's
   expf can differ from in the last bit (within ~2^-60 of a rounding boundary): the caller replays the draw on the
   host to know the distribution and can compare. All arrays are device arrays; a row whose state or dst is out of
   range is skipped. No reference counterpart as one call: the reference draws on the host after each draft
   forward. */
int mk_sample_draw(mk_ctx* ctx, const float* values, const int32_t* ids, int stride, int n_rows,
                   const mk_draw_params* params, uint64_t* states, int n_states, int32_t* out, int n_out);

/* dst[dst_index[i]] = src[src_index[i]] for i < n, in stream order (a NULL index array is the identity; a negative
   index skips i). Moves token ids between device arrays without a host round trip: draft picks into a proposal tree,
   tree ids into a forward's token slots (no reference counterpart: the CPU engine keeps ids in host vectors). */
int mk_move_ids(mk_ctx* ctx, int32_t* dst, const int32_t* dst_index, const int32_t* src, const int32_t* src_index,
                int n);
/* Device-resident greedy decode bookkeeping for one sequence (no reference counterpart: the CPU engine does this on
   the host, engine.cpp:397-421): out_tokens[*counter] = ids[0] = *top1; ++*counter; ++rpos[0], ++kv_row[0],
   ++n_keys[0]. Lets a captured decode step be replayed without host round trips. */
int mk_greedy_advance(mk_ctx* ctx, const int32_t* top1, int32_t* ids, int32_t* rpos, int32_t* kv_row, int32_t* n_keys,
                      int32_t* out_tokens, int32_t* counter);

#ifdef __cplusplus
}
#endif

#endif
