// extern "C" layer of include/malkin_model.h over malkin_hip::Model.
#include <cstdio>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../../include/malkin_engine.h"
#include "../../../include/malkin_model.h"
#include "../../../include/malkin_sampler.h"
#include "../kernels/ctx.h"
#include "engine.h"
#include "model.h"

#include "capi_internal.h"

struct mk_sampler {
  std::unique_ptr<malkin_hip::Sampler> sampler;
  // Candidate selection for device rows, made for the first (context, vocabulary) it is used with.
  std::unique_ptr<malkin_hip::Selector> select;
  mk_ctx* ctx = nullptr;
  int n_vocab = 0;
  std::vector<int32_t> pen_ids;
  std::vector<float> pen_amts;
};

namespace {

template <typename F>
int run(F&& f) {
  try {
    f();
    return MK_OK;
  } catch (const std::invalid_argument& e) {
    mk::set_error("%s", e.what());
    return MK_ERR_INVALID;
  } catch (const std::exception& e) {
    mk::set_error("%s", e.what());
    return MK_ERR_INVALID;
  }
}

// The engine's loop belongs to an HTTP server between mk_server_start and mk_server_stop.
void not_serving(const mk_engine* e) {
  if (e->serving) throw std::invalid_argument("engine is serving HTTP (mk_server_stop first)");
}

malkin_hip::SamplingParams to_params(const mk_sampling_params& p) {
  malkin_hip::SamplingParams s;
  s.temperature = p.temperature;
  s.top_p = p.top_p;
  s.top_k = p.top_k;
  s.min_p = p.min_p;
  s.presence_penalty = p.presence_penalty;
  s.frequency_penalty = p.frequency_penalty;
  s.seed = p.seed;
  return s;
}

malkin_hip::Distribution to_dist(const float* probs, const int32_t* ids, int n) {
  if (n <= 0 || !probs || !ids) throw std::invalid_argument("sampler: empty distribution");
  malkin_hip::Distribution d(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) d[static_cast<size_t>(i)] = malkin_hip::Candidate{probs[i], ids[i]};
  return d;
}

// Sampler::distribution of one device row: penalties and top-k on the device, one wait, the rest on the host.
void device_distribution(mk_ctx* ctx, mk_sampler* s, float* dev_logits, int n_vocab, malkin_hip::Distribution& out) {
  if (!ctx || !s || !dev_logits || n_vocab <= 0) throw std::invalid_argument("sampler: bad arguments");
  if (!s->select || s->ctx != ctx || s->n_vocab != n_vocab) {
    s->select = std::make_unique<malkin_hip::Selector>(ctx, n_vocab);
    s->ctx = ctx;
    s->n_vocab = n_vocab;
  }
  s->pen_ids.clear();
  s->pen_amts.clear();
  s->sampler->penalties(nullptr, 0, s->pen_ids, s->pen_amts);
  s->select->clear();
  s->select->add(0, *s->sampler, s->pen_ids, s->pen_amts);
  s->select->enqueue(dev_logits);
  if (mk_synchronize(ctx) != MK_OK) throw std::runtime_error(mk_last_error());
  s->select->collect();
  s->sampler->finish(*s->select, 0, out);
}

std::vector<malkin_hip::BatchToken> to_batch(const mk_batch_token* b, int n) {
  std::vector<malkin_hip::BatchToken> v(static_cast<size_t>(n > 0 ? n : 0));
  for (int i = 0; i < n; ++i) v[i] = {b[i].id, b[i].seq, b[i].pos, b[i].logits != 0, b[i].kv, b[i].parent};
  return v;
}

}  // namespace

extern "C" {

int mk_gguf_inspect(const char* path, mk_gguf_info* out) {
  return run([&] {
    if (!path || !out) throw std::invalid_argument("mk_gguf_inspect: null argument");
    const malkin_hip::GgufFile f(path);
    mk_gguf_info info{};
    info.n_tensors = static_cast<int64_t>(f.tensors().size());
    for (const auto& kv : f.tensors()) info.tensor_bytes += static_cast<int64_t>(kv.second.nbytes);
    const std::string arch = f.get_str("general.architecture").value_or("");
    std::snprintf(info.arch, sizeof info.arch, "%s", arch.c_str());
    info.n_layer = static_cast<int32_t>(f.get_int(arch + ".block_count").value_or(0));
    const std::vector<int32_t> eog = malkin_hip::read_eog(f);
    info.n_eog = static_cast<int32_t>(eog.size());
    for (size_t i = 0; i < eog.size() && i < 8; ++i) info.eog[i] = eog[i];
    *out = info;
  });
}

int mk_model_open(mk_ctx* ctx, const char* path, int n_ctx, int n_seq, int flags, mk_model** out) {
  return run([&] {
    if (!ctx || !path || !out) throw std::invalid_argument("mk_model_open: null argument");
    auto m = std::make_unique<mk_model>();
    m->file = std::make_unique<malkin_hip::GgufFile>(path);
    m->model = std::make_unique<malkin_hip::Model>(ctx, *m->file, n_ctx, n_seq, (flags & MK_MODEL_NO_WIDE) == 0,
                                                    (flags & MK_MODEL_NO_PACK) != 0,
                                                    (flags & MK_MODEL_PERSISTENT)  ? malkin_hip::Model::kDecodePersistent
                                                    : (flags & MK_MODEL_FUSED_ATTN) ? malkin_hip::Model::kDecodeFusedAttn
                                                                                    : malkin_hip::Model::kDecodeSteps);
    *out = m.release();
  });
}

int mk_model_persistent(const mk_model* m) {
  if (!m || !m->model) return 0;
  return m->model->persistent() ? 1 : m->model->fused_attn() ? 2 : 0;
}

int mk_model_eog(const mk_model* m, int32_t* out, int cap) {
  int n = 0;
  const int rc = run([&] {
    if (!m || cap < 0 || (cap > 0 && !out)) throw std::invalid_argument("mk_model_eog: bad argument");
    const auto& eog = m->model->cfg().eog;
    for (size_t i = 0; i < eog.size() && static_cast<int>(i) < cap; ++i) out[i] = eog[i];
    n = static_cast<int>(eog.size());
  });
  return rc != 0 ? rc : n;
}

int mk_model_free(mk_model* m) {
  return run([&] { delete m; });
}

int mk_model_get_config(const mk_model* m, mk_model_config* o) {
  return run([&] {
    const auto& c = m->model->cfg();
    *o = mk_model_config{c.n_layer, c.n_embd, c.n_ff, c.n_head, c.n_head_kv, c.head_dim, c.n_vocab,
                         m->model->n_ctx(), m->model->n_seq(), c.rope_base, c.rms_eps};
  });
}

int mk_model_forward_batch(mk_model* m, const mk_batch_token* batch, int n, float* logits) {
  return run([&] {
    if (n > 0 && !batch) throw std::invalid_argument("forward: null batch");
    auto b = to_batch(batch, n);
    m->model->forward(b.data(), n, logits);
  });
}

int mk_model_forward(mk_model* m, const int32_t* tokens, int n, int pos, float* logits, int all_logits,
                     const int32_t* parent, int seq) {
  return run([&] { m->model->forward(tokens, n, pos, logits, all_logits != 0, parent, seq); });
}

int mk_model_forward_top2(mk_model* m, const mk_batch_token* batch, int n, int32_t* top1, int32_t* top2) {
  return run([&] {
    if (n > 0 && !batch) throw std::invalid_argument("forward: null batch");
    auto b = to_batch(batch, n);
    m->model->forward_top2(b.data(), n, top1, top2);
  });
}

int mk_model_move_kv(mk_model* m, int from, int to, int seq) {
  return run([&] {
    if (seq < 0 || seq >= m->model->n_seq() || from < 0 || to < 0 || from >= m->model->n_ctx() ||
        to >= m->model->n_ctx())
      throw std::invalid_argument("move_kv: bad row");
    m->model->move_kv(from, to, seq);
  });
}

int mk_model_kv_row(mk_model* m, int layer, int seq, int pos, int k, void* out) {
  return run([&] {
    const auto& c = m->model->cfg();
    if (layer < 0 || layer >= c.n_layer || seq < 0 || seq >= m->model->n_seq() || pos < 0 || pos >= m->model->n_ctx())
      throw std::invalid_argument("kv_row: bad index");
    m->model->kv_row(layer, seq, pos, k != 0, static_cast<uint8_t*>(out));
  });
}

int mk_model_generate(mk_model* m, const int32_t* prompt, int n_prompt, int n_gen, int seq, int use_graph,
                      int32_t* out_tokens, mk_gen_stats* stats) {
  return run([&] {
    malkin_hip::Model::GenStats st;
    m->model->generate_greedy(prompt, n_prompt, n_gen, seq, out_tokens, &st, use_graph != 0);
    if (stats) *stats = mk_gen_stats{st.prefill_ms, st.decode_ms, st.decode_forwards};
  });
}

int64_t mk_model_weight_bytes(const mk_model* m) { return m ? static_cast<int64_t>(m->model->weight_bytes()) : 0; }

int mk_model_weight(const mk_model* m, int layer, int which, mk_weight* out) {
  return run([&] { *out = m->model->weight(layer, which); });
}

int mk_engine_create(mk_model* target, mk_model* draft, int n_draft, mk_engine** out) {
  return run([&] {
    if (!target || !out) throw std::invalid_argument("mk_engine_create: null argument");
    auto e = std::make_unique<mk_engine>();
    e->engine = std::make_unique<malkin_hip::Engine>(target->model.get(), draft ? draft->model.get() : nullptr,
                                                      n_draft);
    *out = e.release();
  });
}

int mk_engine_free(mk_engine* e) {
  return run([&] {
    if (e) not_serving(e);
    delete e;
  });
}

int mk_engine_submit(mk_engine* e, const int32_t* prompt, int n_prompt, int max_tokens, const int32_t* eog, int n_eog,
                     int32_t* request_id) {
  return run([&] {
    if (!e || (n_prompt > 0 && !prompt) || (n_eog > 0 && !eog)) throw std::invalid_argument("mk_engine_submit: null argument");
    not_serving(e);
    malkin_hip::EngineRequest r;
    if (n_prompt > 0) r.prompt.assign(prompt, prompt + n_prompt);
    if (n_eog > 0) r.eog.assign(eog, eog + n_eog);
    r.max_tokens = max_tokens;
    const int id = e->engine->submit(r);
    if (request_id) *request_id = id;
  });
}

int mk_engine_submit_sampled(mk_engine* e, const int32_t* prompt, int n_prompt, int max_tokens, const int32_t* eog,
                             int n_eog, const mk_sampling_params* sampling, int32_t* request_id) {
  return run([&] {
    if (!e || (n_prompt > 0 && !prompt) || (n_eog > 0 && !eog) || !sampling)
      throw std::invalid_argument("mk_engine_submit_sampled: null argument");
    not_serving(e);
    malkin_hip::EngineRequest r;
    if (n_prompt > 0) r.prompt.assign(prompt, prompt + n_prompt);
    if (n_eog > 0) r.eog.assign(eog, eog + n_eog);
    r.max_tokens = max_tokens;
    r.sampling = to_params(*sampling);
    const int id = e->engine->submit(r);
    if (request_id) *request_id = id;
  });
}

int mk_engine_step(mk_engine* e, int32_t* busy) {
  return run([&] {
    if (!e) throw std::invalid_argument("mk_engine_step: null engine");
    not_serving(e);
    const int b = e->engine->step_once();
    if (busy) *busy = b;
  });
}

int mk_engine_run(mk_engine* e) {
  return run([&] {
    if (!e) throw std::invalid_argument("mk_engine_run: null engine");
    not_serving(e);
    e->engine->run();
  });
}

int mk_engine_steps(mk_engine* e, uint64_t* steps) {
  return run([&] {
    if (!e || !steps) throw std::invalid_argument("mk_engine_steps: null argument");
    *steps = e->engine->steps();
  });
}

int mk_engine_draws(mk_engine* e, uint64_t* device_draws, uint64_t* mismatches) {
  return run([&] {
    if (!e || !device_draws || !mismatches) throw std::invalid_argument("mk_engine_draws: null argument");
    *device_draws = e->engine->device_draws();
    *mismatches = e->engine->draw_mismatches();
  });
}

int mk_engine_result(mk_engine* e, int32_t request_id, int32_t* tokens, int32_t cap, mk_request_info* info) {
  return run([&] {
    if (!e) throw std::invalid_argument("mk_engine_result: null engine");
    not_serving(e);
    const malkin_hip::EngineResult& r = e->engine->result(request_id);
    if (tokens)
      for (size_t i = 0; i < r.tokens.size() && static_cast<int32_t>(i) < cap; ++i) tokens[i] = r.tokens[i];
    if (info)
      *info = mk_request_info{r.prompt_tokens, r.cached_tokens, r.completion_tokens, r.drafted, r.accepted,
                               r.finish_reason == "stop" ? 1 : r.finish_reason == "cancelled" ? 2 : 0, r.done ? 1 : 0,
                               r.prefill_ms, r.decode_ms};
  });
}

int mk_engine_release(mk_engine* e, int32_t request_id, int64_t* held) {
  return run([&] {
    if (!e) throw std::invalid_argument("mk_engine_release: null engine");
    not_serving(e);
    e->engine->release(request_id);
    if (held) *held = static_cast<int64_t>(e->engine->results_held());
  });
}

int mk_sampler_create(const mk_sampling_params* params, int penalties, mk_sampler** out) {
  return run([&] {
    if (!params || !out) throw std::invalid_argument("mk_sampler_create: null argument");
    auto s = std::make_unique<mk_sampler>();
    s->sampler = std::make_unique<malkin_hip::Sampler>(to_params(*params), penalties != 0);
    *out = s.release();
  });
}

int mk_sampler_free(mk_sampler* s) {
  return run([&] { delete s; });
}

int mk_sampler_accept(mk_sampler* s, int32_t id) {
  return run([&] {
    if (!s) throw std::invalid_argument("mk_sampler_accept: null sampler");
    s->sampler->accept(id);
  });
}

int mk_sampler_distribution(mk_ctx* ctx, mk_sampler* s, float* dev_logits, int n_vocab, float* probs, int32_t* ids,
                            int cap, int* n_out) {
  return run([&] {
    if (cap > 0 && (!probs || !ids)) throw std::invalid_argument("mk_sampler_distribution: null output");
    malkin_hip::Distribution d;
    device_distribution(ctx, s, dev_logits, n_vocab, d);
    for (int i = 0; i < cap && i < static_cast<int>(d.size()); ++i) {
      probs[i] = d[static_cast<size_t>(i)].p;
      ids[i] = d[static_cast<size_t>(i)].id;
    }
    if (n_out) *n_out = static_cast<int>(d.size());
  });
}

int mk_sampler_sample(mk_ctx* ctx, mk_sampler* s, float* dev_logits, int n_vocab, int32_t* id_out) {
  return run([&] {
    if (!id_out) throw std::invalid_argument("mk_sampler_sample: null output");
    malkin_hip::Distribution d;
    device_distribution(ctx, s, dev_logits, n_vocab, d);
    *id_out = s->sampler->draw(d);
  });
}

int mk_sampler_draw(mk_sampler* s, const float* probs, const int32_t* ids, int n, int32_t* id_out) {
  return run([&] {
    if (!s || !id_out) throw std::invalid_argument("mk_sampler_draw: null argument");
    *id_out = s->sampler->draw(to_dist(probs, ids, n));
  });
}

int mk_sampler_verify(mk_sampler* s, const float* p_probs, const int32_t* p_ids, int n_p, const float* q_probs,
                      const int32_t* q_ids, int n_q, int32_t draft, int* accepted, int32_t* id_out) {
  return run([&] {
    if (!s || !accepted || !id_out) throw std::invalid_argument("mk_sampler_verify: null argument");
    const malkin_hip::Distribution p = to_dist(p_probs, p_ids, n_p);
    const malkin_hip::Distribution q = n_q > 0 ? to_dist(q_probs, q_ids, n_q) : malkin_hip::Distribution{};
    bool ok = false;
    *id_out = s->sampler->verify(p, q, draft, ok);
    *accepted = ok ? 1 : 0;
  });
}

}  // extern "C"
