/*
 * malkin-mi355x: C ABI of stochastic sampling over device logits (libmalkin_hip.so): the reference's
 * malkin::Sampler (src/sampler.h:10-43, src/sampler.cpp:22-97) with the same parameters, penalty counts, random
 * stream (std::mt19937_64 through std::uniform_real_distribution<double>) and results for a given seed.
 *
 * The expensive half of Sampler::distribution runs on the device: repetition penalties applied to the logits row in
 * place and the top-k cut (mk_penalize, mk_topk of malkin_hip.h); the host finishes the distribution over the k
 * candidates (temperature, min-p, top-p, normalisation). Equal logits at the top-k boundary are taken by lower
 * token id (the reference's std::partial_sort leaves their order unspecified). top_k <= 0 or above 1024 copies the
 * penalized row to the host and sorts it there.
 * Status codes and mk_last_error() as in malkin_hip.h.
 */
#ifndef MALKIN_SAMPLER_H
#define MALKIN_SAMPLER_H

#include <stdint.h>

#include "malkin_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* SamplingParams (sampler.h:10-18): the reference's defaults are temperature 0.8, top_p 0.95, top_k 40, min_p 0.05,
   no penalties, seed 0 (random). temperature <= 0: greedy (the first maximum of the penalized logits). */
typedef struct {
  float temperature, top_p;
  int32_t top_k;
  float min_p, presence_penalty, frequency_penalty;
  uint64_t seed;
} mk_sampling_params;

typedef struct mk_sampler mk_sampler;

/* Sampler::Sampler(params, penalties) (sampler.cpp:63-64). penalties = 0: accept() counts are ignored (the draft
   sampler of speculative decoding). */
int mk_sampler_create(const mk_sampling_params* params, int penalties, mk_sampler** out);
int mk_sampler_free(mk_sampler* s);
/* Sampler::accept (sampler.h:31): one more occurrence of id for the presence / frequency penalties. */
int mk_sampler_accept(mk_sampler* s, int32_t id);
/* Sampler::distribution (sampler.cpp:66-106) of one device logits row of n_vocab floats, penalized in place like
   the reference's: up to cap (probability, id) pairs, highest first, into probs / ids (host); *n_out = the
   distribution's size (may exceed cap). Waits for the device once. */
int mk_sampler_distribution(mk_ctx* ctx, mk_sampler* s, float* dev_logits, int n_vocab, float* probs, int32_t* ids,
                            int cap, int* n_out);
/* Sampler::sample (sampler.cpp:118-122): distribution of the device row, then one draw. */
int mk_sampler_sample(mk_ctx* ctx, mk_sampler* s, float* dev_logits, int n_vocab, int32_t* id_out);
/* Sampler::draw (sampler.cpp:108-116) from a host distribution of n entries (no device use). */
int mk_sampler_draw(mk_sampler* s, const float* probs, const int32_t* ids, int n, int32_t* id_out);
/* Sampler::verify (sampler.cpp:124-141), speculative sampling (Leviathan et al. 2023): draft d was drawn from q;
   returns d with probability min(1, p(d) / q(d)), else a draw from the normalised max(0, p - q). Host only. */
int mk_sampler_verify(mk_sampler* s, const float* p_probs, const int32_t* p_ids, int n_p, const float* q_probs,
                      const int32_t* q_ids, int n_q, int32_t draft, int* accepted, int32_t* id_out);

#ifdef __cplusplus
}
#endif

#endif
