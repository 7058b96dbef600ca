/*
 * CPU oracle for the malkin token loop — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the arithmetic of the reference's AVX-512 hot path (kekzl/malkin, src/). Every function
 * cites the reference file:line it follows. 16-wide AVX-512 registers are modelled as float[16] arrays; every
 * rounding step of the reference (mul, fma, add, the halving-tree horizontal sum) is restated one for one, so that
 * outputs are bit-identical to the reference on the same inputs.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the checker.
 * The product path (malkin_amd) never links or calls it.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off; explicit fmaf() wherever the reference fuses).
 */
#ifndef MALKIN_ORACLE_H
#define MALKIN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids as stored in GGUF (gguf.h:12-29). */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_BF16 = 30 };

/* Activation block (quant.h:11-16): 32 int8 values, scale d, int sums of each 16-value half. */
typedef struct {
  float d;
  int16_t s[2];
  int8_t qs[32];
} or_block_q8;

float or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);
size_t or_row_size(int type, int64_t k);

/* kernels_avx512.cpp:66-80 */
void or_quantize_row_q8(const float* x, or_block_q8* y, int64_t k);
/* quant.cpp:134-140 */
float or_quantize_i8(const float* x, int n, int8_t* q);
/* quant.cpp:70-169; returns 0, or -1 for an unsupported type */
int or_dequantize_row(int type, const void* src, float* dst, int64_t k);
/* kernels_avx512.cpp:82-89 */
float or_dot_f32(int64_t k, const float* w, const float* x);
/* vec_dot (quant.cpp:171-191; kernels_avx512.cpp:82-171): the row path's dot of one weight row (GGUF bytes of
   `type`) with one activation row (x: fp32, used by F32/F16/BF16; xq: BlockQ8, used by the quantized types). */
float or_vec_dot(int type, int64_t k, const uint8_t* w, const float* x, const or_block_q8* xq);
/* matmul's row path (quant.cpp:330-351): y[t * y_stride + r] = vec_dot(row r, x[t], xq[t]). -1 for unknown types. */
int or_matmul_rows(int type, const uint8_t* w, size_t row_bytes, int64_t rows, int64_t cols, const float* x,
                   const or_block_q8* xq, int n, float* y, int64_t y_stride);
/* _mm512_reduce_add_ps: halving tree (i, i+8), (i, i+4), (i, i+2), (0, 1) */
float or_reduce16(const float* v);
/* kernels_avx512.cpp:186-202, one lane */
float or_exp(float x);
/* kernels_avx512.cpp:205-226 */
float or_softmax_inplace(float* s, int n);
/* kernels_avx512.cpp:271-280 */
void or_silu_mul(int64_t n, float* g, const float* u);
/* model.cpp:46-49 */
void or_rmsnorm(float* y, const float* x, const float* w, int n, float eps);
/* kernels_avx512.cpp:282-306 (attend_t<DC> for D in {64,128,256} and G <= 16, else the per-head path) */
void or_attend_gqa(const float* q, int G, int D, const int8_t* k, const int8_t* v, size_t stride, ptrdiff_t soff,
                   int n, float scale, float* out, float* scratch, const int* extra, int ne);

/*
 * Panel GEMM semantics (gemm_avx512.cpp:67-205, 268-316; selection quant.cpp:251-268): y[t*y_stride + r] =
 * row r . xq[t] for r < rows, t < n. w holds rows of GGUF blocks, row_bytes apart. wide != 0: the weight also has
 * wide panels, which Q6_K uses for n > 16 (kWideMinTokens, quant.h:50). Returns 0, or -1 for a type without
 * panels (the row path is not on the configs' path and is not restated).
 */
int or_matmul(int type, const uint8_t* w, size_t row_bytes, int64_t rows, int64_t cols, const or_block_q8* xq, int n,
              float* y, int64_t y_stride, int wide);

/* Greedy selection: first maximum (sampler.cpp:27-30, std::max_element). */
int32_t or_argmax(const float* l, int n);
/* Draft top-1 / top-2 scan (engine.cpp:309-318). */
void or_top2(const float* l, int n, int32_t* a, int32_t* b);

/* ---- Model (model.h:22-97, model.cpp) ---- */

typedef struct {
  int32_t id, seq, pos, logits, kv, parent; /* BatchToken, model.h:25-30 (kv/parent -1 = plain) */
} or_batch_token;

typedef struct {
  int n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_vocab;
  float rope_base, rms_eps;
} or_config;

typedef struct or_model or_model;

/* Opens a qwen3 GGUF (model.cpp:78-152). wide != 0: the Q6_K prefill path of Model::pack_wide (model.cpp:187). */
or_model* or_model_open(const char* path, int n_ctx, int n_seq, int wide, char* err, int errlen);
void or_model_free(or_model* m);
void or_model_config(const or_model* m, or_config* c);
/* model.cpp:280-323 + 325-426; 0 on success, -1 with err filled (the reference's runtime_error text). */
int or_model_forward_batch(or_model* m, const or_batch_token* batch, int n, float* logits, char* err, int errlen);
/* model.cpp:249-278 */
int or_model_forward(or_model* m, const int32_t* tokens, int n, int pos, float* logits, int all_logits,
                     const int* parent, int seq, char* err, int errlen);
/* model.cpp:432-440 */
void or_model_move_kv(or_model* m, int from, int to, int seq);
/* KV row (reference layout: KV*D int8 then KV float scales) of layer il, sequence seq, position pos; k != 0: K. */
const int8_t* or_model_kv_row(const or_model* m, int il, int seq, int pos, int k);
size_t or_model_kv_row_bytes(const or_model* m);

/* ---- Sampling (sampler.h:10-43, sampler.cpp:22-141) ---- */

/* std::mt19937_64: the 64-bit Mersenne Twister of Matsumoto & Nishimura (2004) with the parameters the C++ standard
   fixes for it ([rand.predef]: n 312, m 156, r 31, a 0xB5026F5AA96619E9, tempering u 29 / d 0x5555555555555555,
   s 17 / b 0x71D67FFFEDA60000, t 37 / c 0xFFF7EEE000000000, l 43, initialisation multiplier 6364136223846793005). */
typedef struct {
  uint64_t mt[312];
  int i;
} or_mt64;
void or_mt64_seed(or_mt64* g, uint64_t seed);
uint64_t or_mt64_next(or_mt64* g);
/* std::uniform_real_distribution<double>(0, 1) on it as libstdc++'s generate_canonical computes it for a 64-bit
   generator: one output x, (double)x / 2^64, a result that rounds to 1 replaced by the largest double below 1. */
double or_mt64_uniform(or_mt64* g);

typedef struct {
  float temperature, top_p;
  int top_k;
  float min_p;
} or_sampling;
/* The penalty step of Sampler::distribution (sampler.cpp:68-70): l[ids[i]] -= presence + frequency * counts[i], the
   amount one fused multiply-add (the reference is built with contraction on). */
void or_penalize(float* l, const int32_t* ids, const int* counts, int n, float presence, float frequency);
/* The rest of Sampler::distribution (sampler.cpp:71-105) over penalized logits l[n_vocab]: greedy -> the first
   maximum; else the top_k candidates (value descending, equal values by lower id), temperature weights, min-p and
   top-p cut, normalisation. Writes the distribution (at most n_vocab entries) and returns its size. */
int or_distribution(const or_sampling* p, const float* l, int n_vocab, float* probs, int32_t* ids);
/* Sampler::draw (sampler.cpp:108-116). */
int32_t or_draw(or_mt64* g, const float* probs, const int32_t* ids, int n);
/* Sampler::verify (sampler.cpp:124-141). */
int32_t or_verify(or_mt64* g, const float* pp, const int32_t* pi, int np, const float* qp, const int32_t* qi, int nq,
                  int32_t draft, int* accepted);
/* The experiment of the reference's test_sampler.cpp:20-51: n_trials drafts d ~ q drawn by a generator seeded
   draft_seed, each verified against p by one seeded target_seed; hist[id] counts the verified tokens (ids < V).
   Returns the number of accepted drafts. */
long or_verify_experiment(const float* pp, const int32_t* pi, int np, const float* qp, const int32_t* qi, int nq,
                          uint64_t target_seed, uint64_t draft_seed, long n_trials, long* hist, int V);

#ifdef __cplusplus
}
#endif

#endif
