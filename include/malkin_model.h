/*
 * malkin-mi355x: C ABI of the device Model (libmalkin_hip.so).
 *
 * Replaces the reference's malkin::Model (src/model.h:33-97) behind a C boundary: the same constructor inputs (a
 * qwen3 GGUF, n_ctx, n_seq), the same forward entry points with the same batch semantics and error texts, and
 * move_kv. Logits are returned in host memory exactly like Model::forward; mk_model_forward_top2 keeps them on the
 * device and returns the greedy picks instead (what Engine needs, engine.cpp:309-318, 441-479).
 * Status codes and mk_last_error() as in malkin_hip.h.
 */
#ifndef MALKIN_MODEL_H
#define MALKIN_MODEL_H

#include <stdint.h>

#include "malkin_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mk_model mk_model;

/* What mk_gguf_inspect reports about a GGUF file. */
typedef struct {
  int64_t n_tensors;
  int64_t tensor_bytes; /* sum of the tensors' data bytes */
  int32_t n_layer;      /* <arch>.block_count, 0 when absent */
  char arch[32];        /* general.architecture ("" when absent) */
  int32_t n_eog;        /* end-of-generation ids the metadata names (as mk_model_eog, before the vocabulary bound) */
  int32_t eog[8];       /* the first min(n_eog, 8) of them, ascending */
} mk_gguf_info;

/* Opens and validates a GGUF v3 file without a device: header, metadata and tensor directory, every tensor inside
   the file (the checks GgufFile's constructor makes, gguf.h:44-69). MK_ERR_INVALID with the reason otherwise. */
int mk_gguf_inspect(const char* gguf_path, mk_gguf_info* out);

/* BatchToken (model.h:25-30). logits != 0: produce n_vocab logits for this token. kv / parent = -1 for plain
   tokens; a tree token (parent = batch index of an earlier token of the same sequence) writes KV row kv. */
typedef struct {
  int32_t id, seq, pos, logits, kv, parent;
} mk_batch_token;

typedef struct {
  int32_t n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_vocab, n_ctx, n_seq;
  float rope_base, rms_eps;
} mk_model_config;

enum {
  MK_MODEL_NO_WIDE = 1, /* no wide Q6_K prefill panels (the reference's MALKIN_NO_WIDE, model.cpp:181) */
  MK_MODEL_NO_PACK = 2, /* no packed weights: every matmul on the row path over GGUF rows (MALKIN_NO_PACK,
                           model.cpp:136; quant.cpp:330-351). F32 / F16 / BF16 weights take that path anyway. */
  MK_MODEL_PERSISTENT = 4, /* one-token forwards run every layer in the persistent decode kernel (mk_decode_layers)
                              instead of launching each step of each layer on its own; the results are the same */
  MK_MODEL_FUSED_ATTN = 8  /* one-token forwards run each layer's attention and attn_output in one launch
                              (mk_decode_attn_wo); the results are the same. Ignored with MK_MODEL_PERSISTENT. */
};

/* Model::Model(GgufFile, n_ctx, n_seq) (model.h:38) + Model::pack_wide (model.h:43) unless MK_MODEL_NO_WIDE. Weights
   stream from the file to HBM in chunks through pinned staging, each chunk packed on the device while the next is
   copied (the reference packs its panels on the host, quant.cpp:212-235, model.cpp:163-178). */
int mk_model_open(mk_ctx* ctx, const char* gguf_path, int n_ctx, int n_seq, int flags, mk_model** out);
int mk_model_free(mk_model* m);
int mk_model_get_config(const mk_model* m, mk_model_config* out);
/* The model's end-of-generation ids (Tokenizer::is_eog's set, tokenizer.cpp:93-102: the eos / eot / eom ids of the
   GGUF metadata and the control tokens among the reference's end-of-turn names), ascending. Writes at most cap ids to
   out (out may be null when cap is 0) and returns the count of the whole set, or a negative error code. */
int mk_model_eog(const mk_model* m, int32_t* out, int cap);
/* Model::forward(const BatchToken*, int, float*) (model.h:52): logits (host) gets n_vocab floats per token with
   logits set, in batch order. */
int mk_model_forward_batch(mk_model* m, const mk_batch_token* batch, int n, float* logits);
/* Model::forward(tokens, n, pos, logits, all_logits, parent, seq) (model.h:58-59). parent may be NULL. */
int mk_model_forward(mk_model* m, const int32_t* tokens, int n, int pos, float* logits, int all_logits,
                     const int32_t* parent, int seq);
/* As mk_model_forward_batch, logits left on the device; per logits row: top1 = first maximum (sampler.cpp:27-30),
   top2 = the draft runner-up (engine.cpp:309-318). top2 may be NULL. */
int mk_model_forward_top2(mk_model* m, const mk_batch_token* batch, int n, int32_t* top1, int32_t* top2);
/* Model::move_kv (model.h:61). */
int mk_model_move_kv(mk_model* m, int from, int to, int seq);
/* KV row of (layer, seq, pos) in the reference's byte layout (n_head_kv*head_dim int8, then n_head_kv float scales;
   model.cpp:105-110). k != 0: the K cache, else V. */
int mk_model_kv_row(mk_model* m, int layer, int seq, int pos, int k, void* out);

/* Greedy generation of one sequence, the protocol of `malkin bench` (main.cpp:126-143): the prompt in 256-token
   forwards, then n_gen tokens, each the argmax of the previous forward (the first from the prompt's last logits).
   Decode steps run as a replayed HIP graph with token and position kept on the device (use_graph != 0). */
typedef struct {
  double prefill_ms, decode_ms;
  int32_t decode_forwards;
} mk_gen_stats;
int mk_model_generate(mk_model* m, const int32_t* prompt, int n_prompt, int n_gen, int seq, int use_graph,
                      int32_t* out_tokens, mk_gen_stats* stats);

/* 1 if the model's one-token forwards run the persistent decode kernel (mk_decode_layers: MK_MODEL_PERSISTENT set,
   and every layer with fused Q8_0 q|k|v and gate|up weights of a supported shape), 2 if they run the fused attention
   and attn_output launch (mk_decode_attn_wo: MK_MODEL_FUSED_ATTN, same conditions), else 0. */
int mk_model_persistent(const mk_model* m);
/* Bytes of packed weights the model holds in HBM. */
int64_t mk_model_weight_bytes(const mk_model* m);
/* Descriptor of a packed matmul weight of the model (benchmarks, tests): which = 0 q|k|v (rows concatenated),
   1 attn_output, 2 ffn_gate|ffn_up (rows interleaved by 4 when both have one type, see mk_matmul_f32 silu_pairs),
   3 ffn_down of layer `layer`; which = 4 (layer ignored): the LM head. */
int mk_model_weight(const mk_model* m, int layer, int which, mk_weight* out);

#ifdef __cplusplus
}
#endif

#endif
