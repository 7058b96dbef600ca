// C entry points over the reference's own C++ API, so tests can drive the compiled reference (oracle/_ref) through
// ctypes. This file is ours; it contains no reference code. It is compiled together with the reference's sources
// where they lie under /root/reference/src (see oracle/Makefile) into oracle/_ref/libmalkin_ref.so.
// TEST INFRASTRUCTURE ONLY: used to pin the C restatement (oracle.c) and as the CPU baseline of bench.py.
#include <omp.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

#include "cpu.h"
#include "gguf.h"
#include "kernels.h"
#include "model.h"
#include "quant.h"
#include "sampler.h"

using namespace malkin;

namespace {

struct RefWeight {
  std::vector<uint8_t> rows;
  Weight w;
  std::unique_ptr<PackedBuffer> compact, wide;
};

struct RefModel {
  std::unique_ptr<GgufFile> file;
  std::unique_ptr<Model> model;
};

struct RefBatchToken {
  int32_t id, seq, pos, logits, kv, parent;
};

void set_err(char* err, int errlen, const char* what) {
  if (err && errlen > 0) std::snprintf(err, static_cast<size_t>(errlen), "%s", what);
}

}  // namespace

extern "C" {

int ref_cpu_ok() { return cpu_missing_features().empty() ? 1 : 0; }
int ref_physical_cores() { return cpu_physical_cores(); }
int ref_cpu_model(char* out, int len) {
  std::snprintf(out, static_cast<size_t>(len), "%s", cpu_model_name().c_str());
  return 0;
}
void ref_set_threads(int n) { omp_set_num_threads(n); }
const char* ref_isa() { return kern::isa_name(); }

void ref_quantize_row_q8(const float* x, void* y, int64_t k) { kern::quantize_row_q8(x, static_cast<BlockQ8*>(y), k); }
float ref_quantize_i8(const float* x, int n, int8_t* q) { return quantize_i8(x, n, q); }
int ref_dequantize_row(int type, const void* src, float* dst, int64_t k) {
  try {
    dequantize_row(static_cast<GgmlType>(type), src, dst, k);
    return 0;
  } catch (...) {
    return -1;
  }
}
float ref_vec_dot(int type, int64_t k, const void* w, const float* x, const void* xq) {
  return vec_dot(static_cast<GgmlType>(type), k, w, x, static_cast<const BlockQ8*>(xq));
}
float ref_dot_f32(int64_t k, const float* w, const float* x) { return kern::dot_f32(k, w, x); }
void ref_silu_mul(int64_t n, float* g, const float* u) { kern::silu_mul(n, g, u); }
void ref_attend_gqa(const float* q, int G, int D, const int8_t* k, const int8_t* v, size_t stride, ptrdiff_t soff,
                    int n, float scale, float* out, float* scratch, const int* extra, int ne) {
  kern::attend_gqa(q, G, D, k, v, stride, soff, n, scale, out, scratch, extra, ne);
}
void ref_attend_block(const float* q, size_t q_stride, int B, int G, int D, const int8_t* k, const int8_t* v,
                      size_t stride, ptrdiff_t soff, const int* n, float scale, float* out, float* scratch) {
  kern::attend_block(q, q_stride, B, G, D, k, v, stride, soff, n, scale, out, scratch);
}
size_t ref_row_size(int type, int64_t k) { return ggml_row_size(static_cast<GgmlType>(type), k); }

// mode 0: row path (no panels); 1: compact panels; 2: compact + wide panels.
void* ref_weight_new(int type, const uint8_t* data, int64_t rows, int64_t cols, int mode) {
  auto* rw = new RefWeight;
  const size_t rb = ggml_row_size(static_cast<GgmlType>(type), cols);
  rw->rows.assign(data, data + rb * static_cast<size_t>(rows));
  rw->w.type = static_cast<GgmlType>(type);
  rw->w.data = rw->rows.data();
  rw->w.rows = rows;
  rw->w.cols = cols;
  rw->w.row_bytes = rb;
  if (mode >= 1) rw->compact = std::make_unique<PackedBuffer>(pack_weight(rw->w, false));
  if (mode >= 2) rw->wide = std::make_unique<PackedBuffer>(pack_weight(rw->w, true));
  return rw;
}
void ref_weight_matmul(void* h, const float* x, const void* xq, int n, float* y) {
  auto* rw = static_cast<RefWeight*>(h);
  matmul(rw->w, x, static_cast<const BlockQ8*>(xq), n, y);
}
void ref_weight_free(void* h) { delete static_cast<RefWeight*>(h); }

// flags: 1 = pack the wide prefill panels (as the engine does when RAM allows); 2 = MALKIN_NO_PACK (model.cpp:136),
// set in the environment only while the Model is constructed.
void* ref_model_open(const char* path, int n_ctx, int n_seq, int flags, char* err, int errlen) {
  try {
    auto m = std::make_unique<RefModel>();
    m->file = std::make_unique<GgufFile>(path);
    if (flags & 2) setenv("MALKIN_NO_PACK", "1", 1);
    try {
      m->model = std::make_unique<Model>(*m->file, n_ctx, n_seq);
    } catch (...) {
      if (flags & 2) unsetenv("MALKIN_NO_PACK");
      throw;
    }
    if (flags & 2) unsetenv("MALKIN_NO_PACK");
    // Model::wide_bytes is 0 under MALKIN_NO_PACK (model.cpp:181): no wide panels then either.
    if ((flags & 1) && !(flags & 2) && m->model->wide_bytes() > 0) m->model->pack_wide();
    return m.release();
  } catch (const std::exception& e) {
    set_err(err, errlen, e.what());
    return nullptr;
  }
}
void ref_model_free(void* h) { delete static_cast<RefModel*>(h); }
int ref_model_config(void* h, int* out) {
  const auto& c = static_cast<RefModel*>(h)->model->cfg();
  out[0] = c.n_layer;
  out[1] = c.n_embd;
  out[2] = c.n_ff;
  out[3] = c.n_head;
  out[4] = c.n_head_kv;
  out[5] = c.head_dim;
  out[6] = c.n_vocab;
  return 0;
}
int ref_model_forward_batch(void* h, const RefBatchToken* b, int n, float* logits, char* err, int errlen) {
  try {
    std::vector<BatchToken> bt(static_cast<size_t>(n > 0 ? n : 0));
    for (int i = 0; i < n; ++i) {
      bt[i].id = b[i].id;
      bt[i].seq = b[i].seq;
      bt[i].pos = b[i].pos;
      bt[i].logits = b[i].logits != 0;
      bt[i].kv = b[i].kv;
      bt[i].parent = b[i].parent;
    }
    static_cast<RefModel*>(h)->model->forward(bt.data(), n, logits);
    return 0;
  } catch (const std::exception& e) {
    set_err(err, errlen, e.what());
    return -1;
  }
}
int ref_model_forward(void* h, const int32_t* tokens, int n, int pos, float* logits, int all_logits,
                      const int* parent, int seq, char* err, int errlen) {
  try {
    static_cast<RefModel*>(h)->model->forward(tokens, n, pos, logits, all_logits != 0, parent, seq);
    return 0;
  } catch (const std::exception& e) {
    set_err(err, errlen, e.what());
    return -1;
  }
}
void ref_model_move_kv(void* h, int from, int to, int seq) { static_cast<RefModel*>(h)->model->move_kv(from, to, seq); }

// The reference's Sampler (sampler.h:24-43) on caller logits: params as {temperature, top_p, min_p, presence,
// frequency} floats plus top_k and seed. A handle keeps the sampler (its RNG and penalty counts) across calls.
void* ref_sampler_new(const float* pf, int top_k, uint64_t seed, int penalties) {
  SamplingParams p;
  p.temperature = pf[0];
  p.top_p = pf[1];
  p.min_p = pf[2];
  p.presence_penalty = pf[3];
  p.frequency_penalty = pf[4];
  p.top_k = top_k;
  p.seed = seed;
  return new Sampler(p, penalties != 0);
}
void ref_sampler_free(void* h) { delete static_cast<Sampler*>(h); }
void ref_sampler_accept(void* h, int32_t id) { static_cast<Sampler*>(h)->accept(id); }
// distribution() over logits (modified in place, as the reference does); up to cap entries out; returns the size.
int ref_sampler_distribution(void* h, float* logits, int n_vocab, float* probs, int32_t* ids, int cap) {
  Dist d;
  static_cast<Sampler*>(h)->distribution(logits, n_vocab, d);
  for (int i = 0; i < static_cast<int>(d.size()) && i < cap; ++i) {
    probs[i] = d[i].first;
    ids[i] = d[i].second;
  }
  return static_cast<int>(d.size());
}
int32_t ref_sampler_sample(void* h, float* logits, int n_vocab) { return static_cast<Sampler*>(h)->sample(logits, n_vocab); }
int32_t ref_sampler_draw(void* h, const float* probs, const int32_t* ids, int n) {
  Dist d;
  for (int i = 0; i < n; ++i) d.emplace_back(probs[i], ids[i]);
  return static_cast<Sampler*>(h)->draw(d);
}
int32_t ref_sampler_verify(void* h, const float* pp, const int32_t* pi, int np, const float* qp, const int32_t* qi,
                           int nq, int32_t draft, int* accepted) {
  Dist p, q;
  for (int i = 0; i < np; ++i) p.emplace_back(pp[i], pi[i]);
  for (int i = 0; i < nq; ++i) q.emplace_back(qp[i], qi[i]);
  bool a = false;
  const int32_t t = static_cast<Sampler*>(h)->verify(p, q, draft, a);
  *accepted = a ? 1 : 0;
  return t;
}

}  // extern "C"
