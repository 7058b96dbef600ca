/* Deterministic random-init qwen3 GGUF writer (synthetic models for tests and benchmarks). */
#ifndef MALKIN_SYNTH_GGUF_H
#define MALKIN_SYNTH_GGUF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MKS_MIX_UNIFORM = 0, MKS_MIX_Q4_K_M = 1 };

typedef struct {
  int n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_vocab, n_ctx_train;
  float rope_base, rms_eps;
  int tied;     /* 1: no output.weight (LM head = token_embd, model.cpp:116-118) */
  int type;     /* ggml type of every matmul weight and token_embd under MKS_MIX_UNIFORM: 8 Q8_0, 12 Q4_K, 13 Q5_K,
                   14 Q6_K, 1 F16, 30 BF16 */
  int mix;      /* MKS_MIX_* */
  float std;    /* weight standard deviation (0.02) */
  uint64_t seed;
  char name[32];
  int eos_id;   /* >= 0: written as tokenizer.ggml.eos_token_id (the model's end-of-generation id); < 0: no such key */
} mks_config;

/* Size of the file mks_write_gguf writes for c. */
int64_t mks_file_bytes(const mks_config* c);
/* 0 on success; -1 I/O error; -2 unsupported shape or type. */
int mks_write_gguf(const char* path, const mks_config* c, int threads);
/* The writer's quantizer on caller data: rows x k floats -> rows of GGUF blocks of `type` (Q8_0, Q4_K, Q6_K; k a
   multiple of the block size), out holding rows * row bytes. 0 on success, -2 unsupported type or k. */
int mks_quantize_rows(int type, const float* x, int64_t rows, int64_t k, uint8_t* out);

#ifdef __cplusplus
}
#endif

#endif
