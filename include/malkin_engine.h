/*
 * malkin-mi355x: C ABI of the device token loop (libmalkin_hip.so): continuous batching and speculative decoding
 * over mk_model, the reference's malkin::Engine (engine.h:51-141, engine.cpp:242-501) without tokenizer or text:
 * requests are token ids in, token ids out, greedy (mk_engine_submit) or with SamplingParams
 * (mk_engine_submit_sampled).
 *
 * A request is admitted into the idle slot (model sequence) whose cached tokens share the longest prefix with its
 * prompt (that prefix's KV is reused); each step is one target forward over all busy slots: decoding slots put their
 * next token, with a draft model also the draft's greedy tree [next, chain0, alt0, chain1, alt1, ...], then prompt
 * chunks fill the batch up to 256 tokens. Accepted tree nodes move their KV rows (Model::move_kv). Greedy picks run
 * on the device (first maximum, strict-> runner-up for the draft alternative). Sampled requests draft a chain with
 * the draft's sampler and verify it with Sampler::verify (engine.cpp:481-501). Status codes and mk_last_error() as
 * in malkin_hip.h.
 */
#ifndef MALKIN_ENGINE_H
#define MALKIN_ENGINE_H

#include <stdint.h>

#include "malkin_model.h"
#include "malkin_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mk_engine mk_engine;

/* GenResult (engine.h:36-42) without text. finish: 0 = "length" (budget or context end), 1 = "stop" (an
   end-of-generation id, which is not part of the tokens), 2 = "cancelled" (an HTTP client went away or the server
   stopped). */
typedef struct {
  int32_t prompt_tokens, cached_tokens, completion_tokens, drafted, accepted, finish, done;
  double prefill_ms, decode_ms;
} mk_request_info;

/* Engine::Engine (engine.cpp:94-191) over loaded models: target has one slot per sequence (mk_model_open n_seq);
   draft (NULL: no speculation) must have the same vocabulary and at least as many sequences and context; n_draft:
   maximum draft tokens per step (0: 8). The engine does not own the models. */
int mk_engine_create(mk_model* target, mk_model* draft, int n_draft, mk_engine** out);
int mk_engine_free(mk_engine* e);
/* Engine::generate's request (engine.cpp:226-240) queued: prompt ids, max_tokens (0: until the context ends), eog
   ids (may be NULL). Errors as the reference: empty prompt, prompt not shorter than the context. */
int mk_engine_submit(mk_engine* e, const int32_t* prompt, int n_prompt, int max_tokens, const int32_t* eog, int n_eog,
                     int32_t* request_id);
/* The same request with the reference's SamplingParams (GenRequest::sampling, engine.h:29-34): temperature > 0 samples
   (speculative chains verified exactly), penalties count the request's generated tokens, seed 0 is random. */
int mk_engine_submit_sampled(mk_engine* e, const int32_t* prompt, int n_prompt, int max_tokens, const int32_t* eog,
                             int n_eog, const mk_sampling_params* sampling, int32_t* request_id);
/* The worker loop's iteration (engine.cpp:193-224): pending requests into idle slots, then one step. busy (may be
   NULL): slots still in flight. */
int mk_engine_step(mk_engine* e, int32_t* busy);
/* Steps until no request is pending or in flight. */
int mk_engine_run(mk_engine* e);
/* Steps (target forwards) run so far; with mk_host_waits() it bounds the host waits per step (one). */
int mk_engine_steps(mk_engine* e, uint64_t* steps);
/* Sampled requests' drafts drawn on the device so far (mk_sample_draw, no host wait per draft forward), and how many
   of them the host's replay of the same draw (the draft sampler's distribution over the same candidates, its own
   generator) picked differently: 0 unless a device weight differed from the C library's expf in its last bit. No
   reference counterpart (the reference draws every draft on the host, engine.cpp:319-323). */
int mk_engine_draws(mk_engine* e, uint64_t* device_draws, uint64_t* mismatches);
/* Generated ids of a request (up to cap) and its counters. */
int mk_engine_result(mk_engine* e, int32_t request_id, int32_t* tokens, int32_t cap, mk_request_info* info);
/* Frees a finished request's result (the reference hands each result to its caller and keeps none, engine.cpp:
   226-240); the id is unknown afterwards. MK_ERR_INVALID for a request still pending or in flight. held (may be
   NULL): results still held after the call. */
int mk_engine_release(mk_engine* e, int32_t request_id, int64_t* held);

#ifdef __cplusplus
}
#endif

#endif
