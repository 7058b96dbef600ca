#include "model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <utility>

namespace malkin_hip {

namespace {

// C-ABI status -> the reference's exception convention.
void ck(int rc) {
  if (rc != MK_OK) throw std::runtime_error(mk_last_error());
}

void hck(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Types with packed (CDNA layout) kernels; types the row path takes; types only the row path takes.
bool device_type(uint32_t t) { return t == MK_Q8_0 || t == MK_Q4_K || t == MK_Q6_K; }
bool row_type(uint32_t t) {
  return t == MK_F32 || t == MK_F16 || t == MK_BF16 || t == MK_Q8_0 || t == MK_Q4_K || t == MK_Q5_K || t == MK_Q6_K;
}
bool raw_only_type(uint32_t t) { return t == MK_F32 || t == MK_F16 || t == MK_BF16; }

constexpr size_t kLoadChunkBytes = 32u << 20;  // rows per streamed chunk: about 32 MiB

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t) { return std::chrono::duration<double, std::milli>(Clock::now() - t).count(); }

constexpr size_t kStagingBlocks = 16;  // layout copies in flight before the host waits for the oldest

}  // namespace

DevBuf::DevBuf(mk_ctx* c, size_t n) : ctx(c), bytes(n) { ck(mk_malloc(c, n, &p)); }

DevBuf& DevBuf::operator=(DevBuf&& o) noexcept {
  if (this != &o) {
    if (p) mk_free(ctx, p);
    ctx = o.ctx;
    p = o.p;
    bytes = o.bytes;
    o.p = nullptr;
  }
  return *this;
}

DevBuf::~DevBuf() {
  if (p) mk_free(ctx, p);
}

mk_weight Model::Weight::w() const { return mk_weight{type, 0, rows, cols, packed.p}; }

// The hyperparameters the qwen3 forward needs, keyed "<arch>.<name>" (the reference reads the same keys with the
// same defaults, model.cpp:78-101; its error texts are kept because callers report them).
ModelConfig read_config(const GgufFile& f) {
  ModelConfig c;
  c.arch = f.get_str("general.architecture").value_or("");
  c.name = f.get_str("general.name").value_or("model");
  if (c.arch != "qwen3") throw std::runtime_error("architecture '" + c.arch + "' unsupported (supported: qwen3)");
  const std::string ns = c.arch + ".";
  const std::pair<const char*, int*> required[] = {{"block_count", &c.n_layer},
                                                   {"embedding_length", &c.n_embd},
                                                   {"feed_forward_length", &c.n_ff},
                                                   {"attention.head_count", &c.n_head}};
  for (const auto& [name, field] : required) {
    const auto v = f.get_int(ns + name);
    if (!v) throw std::runtime_error("model: metadata " + ns + name + " missing");
    *field = static_cast<int>(*v);
  }
  const auto int_or = [&](const char* name, int fallback) {
    return static_cast<int>(f.get_int(ns + name).value_or(fallback));
  };
  const auto float_or = [&](const char* name, double fallback) {
    return static_cast<float>(f.get_float(ns + name).value_or(fallback));
  };
  c.n_head_kv = int_or("attention.head_count_kv", c.n_head);
  c.head_dim = int_or("attention.key_length", c.n_head > 0 ? c.n_embd / c.n_head : 0);
  c.n_ctx_train = int_or("context_length", 4096);
  c.rope_base = float_or("rope.freq_base", 10000.0);
  c.rms_eps = float_or("attention.layer_norm_rms_epsilon", 1e-6);
  c.n_vocab = static_cast<int>(f.str_array_size("tokenizer.ggml.tokens"));
  c.eog = read_eog(f);  // bounded by the vocabulary once its size is known (Model's constructor)
  return c;
}

// tokenizer.cpp:93-102: the eos / eot / eom ids the metadata names, and, where the file carries its token list and
// token types, the control tokens (type 3) among the reference's end-of-turn names.
std::vector<int32_t> read_eog(const GgufFile& f) {
  std::vector<int32_t> eog;
  for (const char* key : {"tokenizer.ggml.eos_token_id", "tokenizer.ggml.eot_token_id", "tokenizer.ggml.eom_token_id"}) {
    const auto id = f.get_int(key);
    if (id && *id >= 0 && *id <= INT32_MAX) eog.push_back(static_cast<int32_t>(*id));
  }
  const std::vector<std::string> toks = f.str_array("tokenizer.ggml.tokens");
  const std::vector<int64_t> types = f.int_array("tokenizer.ggml.token_type");
  if (!toks.empty() && types.size() == toks.size()) {
    constexpr int64_t kControl = 3;
    for (const char* name : {"<|im_end|>", "<|endoftext|>", "<|eot_id|>", "<|eom_id|>", "<end_of_turn>", "<|return|>",
                             "<|call|>", "<|end|>"}) {
      const auto it = std::find(toks.begin(), toks.end(), name);
      if (it != toks.end() && types[static_cast<size_t>(it - toks.begin())] == kControl)
        eog.push_back(static_cast<int32_t>(it - toks.begin()));
    }
  }
  std::sort(eog.begin(), eog.end());
  eog.erase(std::unique(eog.begin(), eog.end()), eog.end());
  return eog;
}

// Loads the named GGUF matrices (same type and column count) as one row-concatenated weight: CDNA-packed for the
// panel types, or kept as GGUF rows for the row path (F32 / F16 / BF16, and every type when the model was opened
// with no_pack: the reference's MALKIN_NO_PACK, model.cpp:136). interleave4 (two matrices of equal shape, packed):
// rows 4k..4k+3 of the first, then rows 4k..4k+3 of the second.
void Model::load_weight(const GgufFile& f, const std::vector<std::string>& names, Weight& w, bool interleave4) {
  std::vector<const GgufTensor*> ts;
  for (const auto& nm : names) {
    const GgufTensor* t = f.tensor(nm);
    if (!t) throw std::runtime_error("model: tensor " + nm + " missing");
    if (!row_type(t->type))
      throw std::runtime_error("model: tensor " + nm + " has type " + ggml_type_name(t->type) +
                               ", supported on the device: Q8_0 Q4_K Q5_K Q6_K F32 F16 BF16");
    ts.push_back(t);
  }
  w.type = static_cast<int>(ts[0]->type);
  w.cols = ts[0]->ne[0];
  w.rows = 0;
  for (const GgufTensor* t : ts) {
    if (t->type != ts[0]->type || t->ne[0] != w.cols) throw std::runtime_error("model: fused weights differ in type");
    w.rows += t->rows();
  }
  w.raw = no_pack_ || !device_type(w.type);
  w.rowdot = no_pack_ || raw_only_type(w.type);
  w.row_bytes = ggml_row_size(w.type, w.cols);
  if (interleave4 && (w.raw || ts.size() != 2 || ts[0]->rows() != ts[1]->rows() || ts[0]->rows() % 4))
    throw std::runtime_error("model: interleaved weights need two packed matrices of equal rows, a multiple of 4");
  size_t bytes = w.row_bytes * static_cast<size_t>(w.rows);
  if (!w.raw) {
    bytes = mk_packed_bytes(w.type, w.rows, w.cols);
    if (!bytes) throw std::runtime_error("model: weight " + names[0] + " has no device layout (rows % 8)");
  }
  w.packed = DevBuf(ctx_, bytes);
  // Logical row r of the weight -> its bytes in the mapped file, and how many rows follow it there contiguously.
  auto src_row = [&](int64_t r) -> std::pair<const uint8_t*, int64_t> {
    if (interleave4) {
      const int64_t k = r / 8, j = r % 8;
      const GgufTensor* t = ts[j < 4 ? 0 : 1];
      return {t->data + static_cast<size_t>(4 * k + j % 4) * w.row_bytes, 4 - j % 4};
    }
    for (const GgufTensor* t : ts) {
      if (r < t->rows()) return {t->data + static_cast<size_t>(r) * w.row_bytes, t->rows() - r};
      r -= t->rows();
    }
    throw std::logic_error("stream_rows: row past the weight");
  };
  stream_rows(w.rows, w.row_bytes, src_row, [&](const void* dev_rows, int64_t r0, int64_t n) {
    if (!w.raw) ck(mk_pack_weight_rows(ctx_, w.type, dev_rows, w.row_bytes, r0, n, w.rows, w.cols, w.packed.p));
  }, w.raw ? w.packed.p : nullptr);
  weight_bytes_ += bytes;
}

// Moves rows 0..rows-1 (row_bytes each; src(r): row r's bytes in the mapped file and the count of rows that follow
// it contiguously there) to the device in chunks through the pinned staging ring: the host copies chunk i + 1 from the mapped file
// while the device receives and consumes chunk i. With dest, chunk rows land at dest + r0 * row_bytes; without, in a
// device staging block, and consume(dev_rows, r0, n) is queued after each chunk's copy (the pack).
void Model::stream_rows(int64_t rows, size_t row_bytes,
                        const std::function<std::pair<const uint8_t*, int64_t>(int64_t)>& src,
                        const std::function<void(const void*, int64_t, int64_t)>& consume, void* dest) {
  if (rows <= 0) return;
  int64_t chunk = std::max<int64_t>(8, static_cast<int64_t>(kLoadChunkBytes / row_bytes) / 8 * 8);
  chunk = std::min(chunk, rows);
  const size_t need = static_cast<size_t>(chunk) * row_bytes;
  if (need > load_block_bytes_) {
    if (load_block_bytes_) ck(mk_synchronize(ctx_));
    for (LoadBlock& b : load_) {
      b.release();
      void* h = nullptr;
      ck(mk_host_alloc(ctx_, need, &h));
      b.ctx = ctx_;
      b.host = static_cast<uint8_t*>(h);
      b.dev = DevBuf(ctx_, need);
    }
    load_block_bytes_ = need;
  }
  for (int64_t r0 = 0, i = 0; r0 < rows; r0 += chunk, ++i) {
    const int64_t n = std::min(chunk, rows - r0);
    LoadBlock& b = load_[static_cast<size_t>(i) % 2];
    if (!mk_event_done(b.done)) ck(mk_event_wait(ctx_, b.done));
    for (int64_t r = r0; r < r0 + n;) {  // contiguous runs of the file
      const auto [p, avail] = src(r);
      const int64_t take = std::min(r0 + n - r, avail);
      std::memcpy(b.host + static_cast<size_t>(r - r0) * row_bytes, p, static_cast<size_t>(take) * row_bytes);
      r += take;
    }
    void* to = dest ? static_cast<uint8_t*>(dest) + static_cast<size_t>(r0) * row_bytes : b.dev.p;
    ck(mk_copy_async(ctx_, to, b.host, static_cast<size_t>(n) * row_bytes));
    ck(mk_event_record(ctx_, &b.done));
    if (!dest) consume(b.dev.p, r0, n);
  }
}

// ffn_gate | ffn_up: interleaved (silu fused into the decode matmul) when both have one type and the row count
// allows; otherwise the plain group.
void Model::load_gateup(const GgufFile& f, const std::string& gate, const std::string& up, Group& g, bool interleave) {
  const GgufTensor* a = f.tensor(gate);
  const GgufTensor* b = f.tensor(up);
  if (interleave && a && b && a->type == b->type && device_type(a->type) && a->ne[0] == b->ne[0] &&
      a->rows() == b->rows() && a->rows() % 4 == 0) {
    Weight w;
    load_weight(f, {gate, up}, w, true);
    g.rows = w.rows;
    g.parts.push_back(std::move(w));
    g.silu_pairs = true;
    return;
  }
  load_group(f, {gate, up}, g);
}

void Model::load_group(const GgufFile& f, const std::vector<std::string>& names, Group& g) {
  size_t i = 0;
  while (i < names.size()) {
    const GgufTensor* t = f.tensor(names[i]);
    if (!t) throw std::runtime_error("model: tensor " + names[i] + " missing");
    std::vector<std::string> run{names[i]};
    size_t j = i + 1;
    for (; j < names.size(); ++j) {
      const GgufTensor* u = f.tensor(names[j]);
      if (!u) throw std::runtime_error("model: tensor " + names[j] + " missing");
      if (u->type != t->type) break;
      run.push_back(names[j]);
    }
    Weight w;
    load_weight(f, run, w);
    w.out_off = g.rows;
    g.rows += w.rows;
    g.parts.push_back(std::move(w));
    i = j;
  }
}

// Whether mk_matmul_f32 has a fused kernel for this weight at n tokens (the library's own rule, mirrored to pick the
// path without a failing call).
static bool matmul_f32_ok(const mk_weight& w, int n, bool norm) {
  return n >= 1 && n <= 2 && w.cols % 32 == 0 && (!norm || w.cols <= 8192) &&
         static_cast<int64_t>(n) * (w.cols / 32) * 40 <= 64 * 1024 &&
         (w.type == MK_Q8_0 || w.type == MK_Q4_K || w.type == MK_Q6_K);
}

// quant.cpp:287-328 (matmul_group): every part writes its rows of the shared output row [t][g.rows].
void Model::matmul_group(const Group& g, const void* xq, int n, float* y) {
  for (const Weight& p : g.parts) {
    mk_weight w = p.w();
    w.wide = wide_ ? 1 : 0;
    ck(mk_matmul(ctx_, &w, xq, n, y + p.out_off, g.rows, 0));
  }
}

bool Model::matmul_group_f32(const Group& g, const float* x, int64_t xs, const float* norm_w, int n, float* y) {
  for (const Weight& p : g.parts) {
    const mk_weight w = p.w();
    if (!matmul_f32_ok(w, n, norm_w != nullptr)) return false;
  }
  for (const Weight& p : g.parts) {
    mk_weight w = p.w();
    w.wide = wide_ ? 1 : 0;
    ck(mk_matmul_f32(ctx_, &w, x, xs, norm_w, cfg_.rms_eps, n, y + p.out_off, g.rows, 0, 0));
  }
  return true;
}

Model::Model(mk_ctx* ctx, const GgufFile& f, int n_ctx, int n_seq, bool wide, bool no_pack, int decode)
    : ctx_(ctx), cfg_(read_config(f)), n_ctx_(n_ctx), n_seq_(n_seq), wide_(wide), no_pack_(no_pack), decode_(decode) {
  auto& c = cfg_;
  if (c.n_head <= 0 || c.n_head_kv <= 0 || c.head_dim <= 0 || c.head_dim % 32 || c.n_head % c.n_head_kv)
    throw std::runtime_error("model: unsupported head layout");
  if (n_ctx <= 0 || n_seq <= 0) throw std::runtime_error("model: n_ctx and n_seq must be positive");
  const int E = c.n_embd, D = c.head_dim, H = c.n_head, KV = c.n_head_kv, F = c.n_ff;

  const GgufTensor* te = f.tensor("token_embd.weight");
  if (!te) throw std::runtime_error("model: tensor token_embd.weight missing");
  embd_type_ = static_cast<int>(te->type);
  if (!row_type(te->type)) throw std::runtime_error("model: tensor token_embd.weight has unsupported type");
  embd_row_bytes_ = ggml_row_size(te->type, te->ne[0]);
  if (te->ne[0] != c.n_embd) throw std::runtime_error("model: token_embd.weight has the wrong row length");
  embd_count_ = te->rows();
  embd_rows_ = DevBuf(ctx_, te->nbytes);
  stream_rows(embd_count_, embd_row_bytes_,
              [&](int64_t r) { return std::make_pair(te->data + static_cast<size_t>(r) * embd_row_bytes_, embd_count_ - r); },
              {}, embd_rows_.p);
  if (f.tensor("output.weight"))
    load_weight(f, {"output.weight"}, output_);
  else
    load_weight(f, {"token_embd.weight"}, output_);  // tied embeddings (model.cpp:116-118)
  c.n_vocab = static_cast<int>(output_.rows);
  c.eog.erase(std::remove_if(c.eog.begin(), c.eog.end(), [&](int32_t id) { return id >= c.n_vocab; }), c.eog.end());

  auto upload_norm = [&](const std::string& nm, int64_t n, float* dst) {
    const GgufTensor* t = f.tensor(nm);
    if (!t) throw std::runtime_error("model: tensor " + nm + " missing");
    if (t->type != 0 || t->nelements() != n)
      throw std::runtime_error("model: norm " + nm + " not F32[" + std::to_string(n) + "]");
    ck(mk_upload(ctx_, dst, t->data, n * sizeof(float)));
  };
  output_norm_ = DevBuf(ctx_, E * sizeof(float));
  upload_norm("output_norm.weight", E, output_norm_.as<float>());
  layers_.resize(c.n_layer);
  for (int i = 0; i < c.n_layer; ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    Layer& L = layers_[i];
    L.norms = DevBuf(ctx_, (2 * E + 2 * D) * sizeof(float));
    upload_norm(p + "attn_norm.weight", E, L.norms.as<float>());
    upload_norm(p + "ffn_norm.weight", E, L.norms.as<float>() + E);
    upload_norm(p + "attn_q_norm.weight", D, L.norms.as<float>() + 2 * E);
    upload_norm(p + "attn_k_norm.weight", D, L.norms.as<float>() + 2 * E + D);
    // A layer with any weight kept as GGUF rows runs the reference's unfused sequence (fp32 activations kept for
    // the row dots); its gate|up stays [gate | up].
    L.row_flow = no_pack_;
    for (const char* nm : {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"}) {
      const GgufTensor* t = f.tensor(p + nm + ".weight");
      if (t && !device_type(t->type)) L.row_flow = true;
    }
    load_group(f, {p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"}, L.qkv);
    load_weight(f, {p + "attn_output.weight"}, L.wo);
    load_gateup(f, p + "ffn_gate.weight", p + "ffn_up.weight", L.gateup, !L.row_flow);
    load_weight(f, {p + "ffn_down.weight"}, L.down);
    if (L.qkv.rows != (int64_t)(H + 2 * KV) * D || L.wo.rows != E || L.gateup.rows != 2 * F || L.down.rows != E)
      throw std::runtime_error("model: layer " + std::to_string(i) + " has unexpected shapes");
  }

  // RoPE tables (model.cpp:137, 335-339), computed on the host with the same float pow / cos / sin calls.
  std::vector<float> inv(D / 2), cs(static_cast<size_t>(n_ctx) * D / 2), sn(cs.size());
  for (int i = 0; i < D / 2; ++i) inv[i] = std::pow(c.rope_base, -2.0f * i / c.head_dim);
  for (int pos = 0; pos < n_ctx; ++pos)
    for (int i = 0; i < D / 2; ++i) {
      const float a = static_cast<float>(pos) * inv[i];
      cs[static_cast<size_t>(pos) * D / 2 + i] = std::cos(a);
      sn[static_cast<size_t>(pos) * D / 2 + i] = std::sin(a);
    }
  rope_cos_ = DevBuf(ctx_, cs.size() * sizeof(float));
  rope_sin_ = DevBuf(ctx_, sn.size() * sizeof(float));
  ck(mk_upload(ctx_, rope_cos_.p, cs.data(), cs.size() * sizeof(float)));
  ck(mk_upload(ctx_, rope_sin_.p, sn.data(), sn.size() * sizeof(float)));

  const size_t rows = static_cast<size_t>(c.n_layer) * n_seq * KV * n_ctx;
  kc_ = DevBuf(ctx_, rows * D);
  vc_ = DevBuf(ctx_, rows * D);
  ks_ = DevBuf(ctx_, rows * sizeof(float));
  vs_ = DevBuf(ctx_, rows * sizeof(float));
  ck(mk_fill(ctx_, kc_.p, 0, kc_.bytes));
  ck(mk_fill(ctx_, vc_.p, 0, vc_.bytes));
  ck(mk_fill(ctx_, ks_.p, 0, ks_.bytes));
  ck(mk_fill(ctx_, vs_.p, 0, vs_.bytes));

  const size_t B = kMaxBatch, T = kDevBatch;
  const size_t qkv_rows = static_cast<size_t>(H + 2 * KV) * D;
  const size_t kmax = std::max({static_cast<size_t>(E), static_cast<size_t>(H) * D, static_cast<size_t>(F)});
  x_ = DevBuf(ctx_, T * E * sizeof(float));
  qkv_ = DevBuf(ctx_, T * qkv_rows * sizeof(float));
  att_ = DevBuf(ctx_, T * H * D * sizeof(float));
  gu_ = DevBuf(ctx_, T * 2 * F * sizeof(float));
  xq_ = DevBuf(ctx_, T * (kmax / 32) * 40);
  h_ = DevBuf(ctx_, T * E * sizeof(float));
  logits_ = DevBuf(ctx_, B * static_cast<size_t>(c.n_vocab) * sizeof(float));
  top_ = DevBuf(ctx_, 2 * B * sizeof(int32_t) + 2 * sizeof(int32_t));

  kv_ = mk_kv_cache{kc_.as<int8_t>(), vc_.as<int8_t>(), ks_.as<float>(), vs_.as<float>(), c.n_layer, n_seq_, KV, D,
                    n_ctx_};
  // Rows longer than one workgroup's LDS keep their attention scores in the context's scratch (global slots, one
  // per workgroup in flight): reserved now, so that no forward allocates (graphs capture them).
  ck(mk_reserve_scratch(ctx_, mk_attention_scratch_bytes(D, n_ctx_, std::min(static_cast<int>(T) * H, 256))));

  // Layout block (see model.h) and its pinned staging ring.
  layout_words_ = 7 * T + (B + 1) + B * (B + 1) / 2;
  layout_ = DevBuf(ctx_, layout_words_ * sizeof(int32_t));
  int32_t* d = layout_.as<int32_t>();
  d_ids_ = d;
  d_rpos_ = d + T;
  d_seq_ = d + 2 * T;
  d_kv_row_ = d + 3 * T;
  d_n_keys_ = d + 4 * T;
  d_out_ = d + 5 * T;
  d_id_from_ = d + 6 * T;
  d_extra_at_ = d + 7 * T;
  d_extra_ = d + 7 * T + B + 1;
  staging_.resize(kStagingBlocks);
  for (Staging& st : staging_) {
    void* h = nullptr;
    ck(mk_host_alloc(ctx_, layout_words_ * sizeof(int32_t), &h));
    st.host = static_cast<int32_t*>(h);
  }
  if (decode_ != kDecodeSteps) make_decode_plan();
  ck(mk_synchronize(ctx_));
  for (LoadBlock& b : load_) b.release();  // loading is done: the staging ring goes
  load_block_bytes_ = 0;
}

// The persistent decode kernel takes the layer loop of one-token forwards where every layer has fused Q8_0 groups
// (q|k|v one buffer, gate|up one interleaved buffer) and the library has a kernel for the shape.
void Model::make_decode_plan() {
  const auto& c = cfg_;
  std::vector<mk_decode_layer> dl(c.n_layer);
  for (int i = 0; i < c.n_layer; ++i) {
    const Layer& L = layers_[i];
    if (L.row_flow || L.qkv.parts.size() != 1 || L.gateup.parts.size() != 1 || !L.gateup.silu_pairs) return;
    const float* nw = L.norms.as<float>();
    dl[i] = mk_decode_layer{L.qkv.parts[0].w(), L.wo.w(), L.gateup.parts[0].w(), L.down.w(),
                            nw,                 nw + c.n_embd, nw + 2 * c.n_embd, nw + 2 * c.n_embd + c.head_dim};
  }
  mk_decode_plan* p = nullptr;
  const int rc = mk_decode_plan_create(ctx_, dl.data(), c.n_layer, c.n_head, c.rms_eps, &kv_, x_.as<float>(),
                                       qkv_.as<float>(), xq_.p, gu_.as<float>(), rope_cos_.as<float>(),
                                       rope_sin_.as<float>(), d_rpos_, d_seq_, d_kv_row_, d_n_keys_, &p);
  if (rc == MK_ERR_UNSUPPORTED) return;
  ck(rc);
  dplan_ = p;
}

void Model::check_device() {
  if (!dplan_pending_) return;
  dplan_pending_ = false;
  ck(mk_decode_check(ctx_, dplan_));
}

void Model::LoadBlock::release() {
  if (done) (void)mk_event_free(done);
  if (host) (void)mk_host_free(ctx, host);
  done = nullptr;
  host = nullptr;
  dev = DevBuf();
}

Model::~Model() {
  if (!staging_.empty()) (void)mk_synchronize(ctx_);
  if (dplan_) (void)mk_decode_plan_destroy(dplan_);
  for (Staging& st : staging_) {
    (void)mk_event_free(st.done);
    (void)mk_host_free(ctx_, st.host);
  }
}

mk_weight Model::weight(int layer, int which) const {
  if (which == 4) return output_.w();
  if (layer < 0 || layer >= cfg_.n_layer || which < 0 || which > 3) throw std::invalid_argument("weight: bad index");
  const Layer& L = layers_[layer];
  if ((which == 0 && L.qkv.parts.size() != 1) || (which == 2 && L.gateup.parts.size() != 1))
    throw std::invalid_argument("weight: this group is split by type");
  const Weight* w[4] = {&L.qkv.parts[0], &L.wo, &L.gateup.parts[0], &L.down};
  mk_weight r = w[which]->w();
  r.wide = wide_ ? 1 : 0;
  return r;
}

namespace {

void reset_layout(TokenLayout& L, int n) {
  L.n = n;
  L.id.assign(n, 0);
  L.rope_pos.assign(n, 0);
  L.seq.assign(n, 0);
  L.kv_row.assign(n, 0);
  L.n_keys.assign(n, 0);
  L.id_from.assign(n, -1);
  L.logit_rows.clear();
  L.tree = false;
  L.extra_at.clear();
  L.extra.clear();
}

}  // namespace

// A multi-sequence batch (model.cpp:280-323 semantics; validation texts as there). A plain token (parent < 0)
// writes KV row pos of its sequence and attends to rows 0..pos. A tree token writes row kv and attends to what its
// parent attends to, then to its own row. Unrolled: follow the parent links up to the plain token the chain starts
// from; the keys are that token's rows 0..pos, then the rows of the chain's tokens from just below it down to t.
void Model::layout_batch(const BatchToken* batch, int n, int limit) {
  if (n <= 0 || n > limit) throw std::runtime_error("forward: batch size out of range");
  TokenLayout& L = lay_;
  reset_layout(L, n);
  for (int t = 0; t < n; ++t) {
    const BatchToken& b = batch[t];
    const bool child = b.parent >= 0;
    const int row = child ? b.kv : b.pos;
    if (b.seq < 0 || b.seq >= n_seq_ || b.pos < 0 || b.pos >= n_ctx_ || row < 0 || row >= n_ctx_)
      throw std::runtime_error("forward: bad slot");
    if (b.parent >= t || (child && batch[b.parent].seq != b.seq)) throw std::runtime_error("forward: bad tree parent");
    L.id[t] = b.id;
    L.rope_pos[t] = b.pos;
    L.seq[t] = b.seq;
    L.kv_row[t] = row;
    L.tree = L.tree || child;
    if (b.logits) L.logit_rows.push_back(t);
  }
  std::vector<int32_t> chain;
  for (int t = 0; t < n; ++t) {
    int u = t;
    chain.clear();
    while (batch[u].parent >= 0) {  // parents precede their children, so this ends
      chain.push_back(L.kv_row[u]);
      u = batch[u].parent;
    }
    L.n_keys[t] = batch[u].pos + 1;
    if (L.tree) {
      L.extra_at.push_back(static_cast<int32_t>(L.extra.size()));
      L.extra.insert(L.extra.end(), chain.rbegin(), chain.rend());
    }
  }
  if (L.tree) L.extra_at.push_back(static_cast<int32_t>(L.extra.size()));
  if (L.tree && n > kMaxBatch) throw std::runtime_error("forward: tree too deep");
  finish_layout();
}

// n consecutive tokens of one sequence at positions pos.. (model.cpp:249-278 semantics). With parent links (tree
// verification) token t writes row pos + t, sits at RoPE position pos + depth(t), and attends to the prefix rows
// 0..pos-1 and then to the rows of its ancestors from the root down to itself.
void Model::layout_tokens(const int32_t* tokens, int n, int pos, bool all_logits, const int* parent, int seq) {
  if (n <= 0 || n > kMaxBatch) throw std::runtime_error("forward: batch size out of range");
  if (pos + n > n_ctx_) throw std::runtime_error("forward: context full");
  if (seq < 0 || seq >= n_seq_) throw std::runtime_error("forward: bad sequence");
  TokenLayout& L = lay_;
  reset_layout(L, n);
  L.tree = parent != nullptr;
  std::vector<int32_t> depth(static_cast<size_t>(n), 0), chain;
  for (int t = 0; t < n; ++t) {
    L.id[t] = tokens[t];
    L.seq[t] = seq;
    L.kv_row[t] = pos + t;
    if (all_logits || t == n - 1) L.logit_rows.push_back(t);
    if (!parent) {
      L.rope_pos[t] = pos + t;
      L.n_keys[t] = pos + t + 1;
      continue;
    }
    if (parent[t] >= t) throw std::runtime_error("forward: bad tree parent");
    depth[t] = parent[t] < 0 ? 0 : depth[parent[t]] + 1;
    L.rope_pos[t] = pos + depth[t];
    L.n_keys[t] = pos;
    chain.clear();
    for (int a = t; a >= 0; a = parent[a]) chain.push_back(pos + a);
    L.extra_at.push_back(static_cast<int32_t>(L.extra.size()));
    L.extra.insert(L.extra.end(), chain.rbegin(), chain.rend());
  }
  if (L.tree) L.extra_at.push_back(static_cast<int32_t>(L.extra.size()));
  finish_layout();
}

void Model::finish_layout() {
  TokenLayout& L = lay_;
  const size_t cap = static_cast<size_t>(kMaxBatch) * (kMaxBatch + 1) / 2;
  if (L.extra.size() > cap) throw std::runtime_error("forward: tree too deep");
  L.max_keys = 1;
  for (int t = 0; t < L.n; ++t) {
    const int extra = L.tree ? L.extra_at[t + 1] - L.extra_at[t] : 0;
    L.max_keys = std::max(L.max_keys, L.n_keys[t] + extra);
  }
  std::vector<int32_t> seqs(L.seq);
  std::sort(seqs.begin(), seqs.end());
  L.distinct_seqs = std::adjacent_find(seqs.begin(), seqs.end()) == seqs.end();
}

void Model::check_ids() {
  for (int t = 0; t < lay_.n; ++t)
    if (lay_.id_from[t] < 0 && (lay_.id[t] < 0 || lay_.id[t] >= embd_count_))
      throw std::runtime_error("forward: token id out of range");  // model.cpp:332
}

// Copies the layout to the device from the next pinned staging block, without waiting for the device unless that
// block's previous copy is still pending; then, for tokens whose id is produced on the device, gathers those ids.
void Model::upload_layout(const int32_t* dev_ids) {
  check_ids();
  const TokenLayout& L = lay_;
  const size_t T = kDevBatch, B = kMaxBatch;
  if (L.logit_rows.size() > B) throw std::runtime_error("forward: more than 256 logits rows");
  Staging& st = staging_[next_staging_];
  next_staging_ = (next_staging_ + 1) % staging_.size();
  if (!mk_event_done(st.done)) ck(mk_event_wait(ctx_, st.done));
  int32_t* h = st.host;
  std::copy(L.id.begin(), L.id.end(), h);
  std::copy(L.rope_pos.begin(), L.rope_pos.end(), h + T);
  std::copy(L.seq.begin(), L.seq.end(), h + 2 * T);
  std::copy(L.kv_row.begin(), L.kv_row.end(), h + 3 * T);
  std::copy(L.n_keys.begin(), L.n_keys.end(), h + 4 * T);
  std::copy(L.logit_rows.begin(), L.logit_rows.end(), h + 5 * T);
  std::copy(L.id_from.begin(), L.id_from.end(), h + 6 * T);
  size_t words = 7 * T;
  if (L.tree) {
    std::copy(L.extra_at.begin(), L.extra_at.end(), h + 7 * T);
    std::copy(L.extra.begin(), L.extra.end(), h + 7 * T + B + 1);
    words = 7 * T + B + 1 + L.extra.size();
  }
  ck(mk_copy_async(ctx_, layout_.p, h, words * sizeof(int32_t)));
  ck(mk_event_record(ctx_, &st.done));
  if (dev_ids) ck(mk_move_ids(ctx_, d_ids_, nullptr, dev_ids, d_id_from_, L.n));
}

// model.cpp:325-426 on the device.
void Model::run() {
  const int n = lay_.n;
  const auto& c = cfg_;
  const int E = c.n_embd, D = c.head_dim, H = c.n_head, KV = c.n_head_kv, F = c.n_ff;
  const int64_t QKV = static_cast<int64_t>(H + 2 * KV) * D;
  float* x = x_.as<float>();
  float* qkv = qkv_.as<float>();
  float* att = att_.as<float>();
  float* gu = gu_.as<float>();
  void* xq = xq_.p;
  const mk_kv_cache& kv = kv_;
  ck(mk_dequantize_rows(ctx_, embd_type_, embd_rows_.p, embd_row_bytes_, d_ids_, n, E, x));
  // One token: every layer in one persistent launch (same results as the per-step launches below).
  const bool one = dplan_ && n == 1 && !lay_.tree && mk_decode_supported(dplan_, lay_.max_keys);
  const bool persistent = one && decode_ == kDecodePersistent, fused_attn = one && decode_ == kDecodeFusedAttn;
  if (persistent) {
    ck(mk_decode_layers(ctx_, dplan_, 0, c.n_layer, lay_.max_keys));
    dplan_pending_ = true;
  }
  for (int il = 0; il < (persistent ? 0 : c.n_layer); ++il) {
    const Layer& L = layers_[il];
    const float* norms = L.norms.as<float>();
    if (L.row_flow) {
      run_row_layer(L, il);
      continue;
    }
    // Decode steps (n <= 2) fuse rmsnorm / quantization into the matmuls (mk_matmul_f32); same results.
    if (!matmul_group_f32(L.qkv, x, E, norms, n, qkv)) {
      ck(mk_rmsnorm_q8(ctx_, x, nullptr, norms, n, E, c.rms_eps, xq));
      matmul_group(L.qkv, xq, n, qkv);
    }
    if (fused_attn) {  // attention and x += attn_output(att) in one launch
      ck(mk_decode_attn_wo(ctx_, dplan_, il, lay_.max_keys));
      dplan_pending_ = true;
    }
    // Short plain batches of distinct sequences (decode steps): QK-norm, RoPE, the KV write and attention in one
    // launch; otherwise (prompt chunks, trees, shared sequences) the KV rows are written before any token attends.
    // Where attn_output takes BlockQ8 activations, the attention kernels write them beside att (the reference's
    // quantize_acts of att, model.cpp:398-401).
    mk_weight wo = L.wo.w();
    wo.wide = wide_ ? 1 : 0;
    const bool wo_f32 = matmul_f32_ok(wo, n, false);
    int rc = MK_ERR_UNSUPPORTED;
    if (fused_attn) {
      rc = MK_OK;
    } else if (!lay_.tree && lay_.distinct_seqs && n < 16) {
      rc = wo_f32 ? mk_attention_decode(ctx_, qkv, QKV, n, H, norms + 2 * E, norms + 2 * E + D, c.rms_eps,
                                        rope_cos_.as<float>(), rope_sin_.as<float>(), d_rpos_, d_seq_, d_kv_row_,
                                        d_n_keys_, &kv, il, att, static_cast<int64_t>(H) * D, lay_.max_keys)
                  : mk_attention_decode_q8(ctx_, qkv, QKV, n, H, norms + 2 * E, norms + 2 * E + D, c.rms_eps,
                                           rope_cos_.as<float>(), rope_sin_.as<float>(), d_rpos_, d_seq_, d_kv_row_,
                                           d_n_keys_, &kv, il, att, static_cast<int64_t>(H) * D, lay_.max_keys, xq);
    }
    if (rc == MK_ERR_UNSUPPORTED) {
      ck(mk_qk_norm_rope_kv(ctx_, qkv, qkv + static_cast<int64_t>(H) * D, qkv + static_cast<int64_t>(H + KV) * D, QKV,
                            n, H, norms + 2 * E, norms + 2 * E + D, c.rms_eps, rope_cos_.as<float>(),
                            rope_sin_.as<float>(), d_rpos_, d_seq_, d_kv_row_, &kv, il));
      if (wo_f32)
        ck(mk_attention(ctx_, qkv, QKV, att, static_cast<int64_t>(H) * D, n, H, &kv, il, d_seq_, d_n_keys_,
                        lay_.tree ? d_extra_at_ : nullptr, d_extra_, lay_.max_keys));
      else
        ck(mk_attention_q8(ctx_, qkv, QKV, att, static_cast<int64_t>(H) * D, n, H, &kv, il, d_seq_, d_n_keys_,
                           lay_.tree ? d_extra_at_ : nullptr, d_extra_, lay_.max_keys, xq));
    } else {
      ck(rc);
    }
    if (fused_attn)
      ;
    else if (wo_f32)
      ck(mk_matmul_f32(ctx_, &wo, att, static_cast<int64_t>(H) * D, nullptr, 0.0f, n, x, E, 1, 0));
    else
      ck(mk_matmul(ctx_, &wo, xq, n, x, E, 1));  // x += attn_output(att) (model.cpp:398-401)
    mk_weight wd = L.down.w();
    wd.wide = wide_ ? 1 : 0;
    if (L.gateup.silu_pairs && matmul_f32_ok(L.gateup.parts[0].w(), n, true) && matmul_f32_ok(wd, n, false)) {
      // h = silu(gate) * up straight from the gate|up matmul, quantized inside the down matmul.
      mk_weight wg = L.gateup.parts[0].w();
      wg.wide = wide_ ? 1 : 0;
      ck(mk_matmul_f32(ctx_, &wg, x, E, norms + E, c.rms_eps, n, gu, F, 0, 1));
      ck(mk_matmul_f32(ctx_, &wd, gu, F, nullptr, 0.0f, n, x, E, 1, 0));  // x += ffn_down(h)
    } else {
      if (!matmul_group_f32(L.gateup, x, E, norms + E, n, gu)) {
        ck(mk_rmsnorm_q8(ctx_, x, nullptr, norms + E, n, E, c.rms_eps, xq));
        matmul_group(L.gateup, xq, n, gu);
      }
      ck(mk_silu_mul_q8(ctx_, gu, n, F, L.gateup.silu_pairs ? 1 : 0, xq));
      ck(mk_matmul(ctx_, &wd, xq, n, x, E, 1));  // x += ffn_down(...) (model.cpp:412-416)
    }
  }
  const int m = n_out();
  if (m == 0) return;
  if (output_.raw) {  // model.cpp:419-425 over GGUF rows: fp32 normalized rows and their BlockQ8 rows
    float* h = h_.as<float>();
    ck(mk_rmsnorm_rows(ctx_, x, d_out_, output_norm_.as<float>(), m, E, c.rms_eps, h));
    if (!raw_only_type(output_.type)) ck(mk_quantize_q8(ctx_, h, m, E, xq));
    if (output_.rowdot)
      ck(mk_matmul_rows(ctx_, output_.type, output_.packed.p, output_.row_bytes, output_.rows, output_.cols, h, E, xq,
                        m, logits_.as<float>(), c.n_vocab, 0));
    else
      ck(mk_matmul_gguf(ctx_, output_.type, output_.packed.p, output_.row_bytes, output_.rows, output_.cols, xq, m,
                        logits_.as<float>(), c.n_vocab, 0));
    return;
  }
  ck(mk_rmsnorm_q8(ctx_, x, d_out_, output_norm_.as<float>(), m, E, c.rms_eps, xq));
  mk_weight wout = output_.w();
  wout.wide = wide_ ? 1 : 0;
  ck(mk_matmul(ctx_, &wout, xq, m, logits_.as<float>(), c.n_vocab, 0));
}


void Model::matmul_any(const Group& g, const float* xf, int64_t xfs, const void* xq, int n, float* y) {
  for (const Weight& p : g.parts) {
    if (p.raw && p.rowdot) {
      ck(mk_matmul_rows(ctx_, p.type, p.packed.p, p.row_bytes, p.rows, p.cols, xf, xfs, xq, n, y + p.out_off, g.rows,
                        0));
    } else if (p.raw) {
      ck(mk_matmul_gguf(ctx_, p.type, p.packed.p, p.row_bytes, p.rows, p.cols, xq, n, y + p.out_off, g.rows, 0));
    } else {
      mk_weight w = p.w();
      w.wide = wide_ ? 1 : 0;
      ck(mk_matmul(ctx_, &w, xq, n, y + p.out_off, g.rows, 0));
    }
  }
}

// One layer with weights on the row path, as model.cpp:360-416 runs it: every matmul sees the fp32 activations and
// their BlockQ8 rows, gate|up gives [gate | up] per token, and the residual adds go into x.
void Model::run_row_layer(const Layer& L, int il) {
  const int n = lay_.n;
  const auto& c = cfg_;
  const int E = c.n_embd, D = c.head_dim, H = c.n_head, KV = c.n_head_kv, F = c.n_ff;
  const int64_t QKV = static_cast<int64_t>(H + 2 * KV) * D, HD = static_cast<int64_t>(H) * D;
  float* x = x_.as<float>();
  float* h = h_.as<float>();
  float* qkv = qkv_.as<float>();
  float* att = att_.as<float>();
  float* gu = gu_.as<float>();
  void* xq = xq_.p;
  const float* norms = L.norms.as<float>();
  auto single = [&](const Weight& w, const float* xf, int64_t xfs, float* y, int64_t ys) {
    if (w.raw && w.rowdot) {
      ck(mk_matmul_rows(ctx_, w.type, w.packed.p, w.row_bytes, w.rows, w.cols, xf, xfs, xq, n, y, ys, 1));
    } else if (w.raw) {
      ck(mk_matmul_gguf(ctx_, w.type, w.packed.p, w.row_bytes, w.rows, w.cols, xq, n, y, ys, 1));
    } else {
      mk_weight mw = w.w();
      mw.wide = wide_ ? 1 : 0;
      ck(mk_matmul(ctx_, &mw, xq, n, y, ys, 1));
    }
  };
  ck(mk_rmsnorm_rows(ctx_, x, nullptr, norms, n, E, c.rms_eps, h));
  ck(mk_quantize_q8(ctx_, h, n, E, xq));
  matmul_any(L.qkv, h, E, xq, n, qkv);
  ck(mk_qk_norm_rope_kv(ctx_, qkv, qkv + HD, qkv + HD + static_cast<int64_t>(KV) * D, QKV, n, H, norms + 2 * E,
                        norms + 2 * E + D, c.rms_eps, rope_cos_.as<float>(), rope_sin_.as<float>(), d_rpos_, d_seq_,
                        d_kv_row_, &kv_, il));
  ck(mk_attention_q8(ctx_, qkv, QKV, att, HD, n, H, &kv_, il, d_seq_, d_n_keys_,
                     lay_.tree ? d_extra_at_ : nullptr, d_extra_, lay_.max_keys, xq));  // att and its BlockQ8 rows
  single(L.wo, att, HD, x, E);  // x += attn_output(att)
  ck(mk_rmsnorm_rows(ctx_, x, nullptr, norms + E, n, E, c.rms_eps, h));
  ck(mk_quantize_q8(ctx_, h, n, E, xq));
  matmul_any(L.gateup, h, E, xq, n, gu);
  ck(mk_silu_mul_q8(ctx_, gu, n, F, 0, xq));  // BlockQ8 rows of silu(gate) * up ...
  ck(mk_silu_mul_rows(ctx_, gu, n, F));       // ... and the fp32 rows themselves, in place of gate
  single(L.down, gu, 2 * static_cast<int64_t>(F), x, E);  // x += ffn_down(...)
}

void Model::forward(const BatchToken* batch, int n, float* logits) {
  layout_batch(batch, n);
  upload_layout();
  run();
  if (!lay_.logit_rows.empty() && logits)
    ck(mk_download(ctx_, logits, logits_.p, lay_.logit_rows.size() * static_cast<size_t>(cfg_.n_vocab) * sizeof(float)));
  else
    ck(mk_synchronize(ctx_));
  check_device();
}

void Model::enqueue(const BatchToken* batch, int n, const int32_t* id_from, const int32_t* dev_ids, int32_t* dev_top1,
                    int32_t* dev_top2) {
  layout_batch(batch, n);
  bool from_device = false;
  if (id_from && dev_ids)
    for (int t = 0; t < n; ++t)
      if (id_from[t] >= 0) {
        lay_.id_from[t] = id_from[t];
        from_device = true;
      }
  upload_layout(from_device ? dev_ids : nullptr);
  run();
  const int m = n_out();
  if (m > 0 && (dev_top1 || dev_top2)) {
    int32_t* t1 = dev_top1 ? dev_top1 : top_.as<int32_t>();  // the runner-up scan still needs a top-1 output
    ck(mk_argmax_top2(ctx_, logits_.as<float>(), m, cfg_.n_vocab, t1, dev_top2));
  }
}

void Model::forward_top2(const BatchToken* batch, int n, int32_t* top1, int32_t* top2) {
  int32_t* d1 = top_.as<int32_t>();
  int32_t* d2 = d1 + kMaxBatch;
  enqueue(batch, n, nullptr, nullptr, d1, top2 ? d2 : nullptr);
  const int m = n_out();
  if (m > 0 && top1) ck(mk_download(ctx_, top1, d1, m * sizeof(int32_t)));
  if (m > 0 && top2) ck(mk_download(ctx_, top2, d2, m * sizeof(int32_t)));
  if (m == 0 || (!top1 && !top2)) ck(mk_synchronize(ctx_));
  check_device();
}

void Model::forward(const int32_t* tokens, int n, int pos, float* logits, bool all_logits, const int* parent,
                    int seq) {
  layout_tokens(tokens, n, pos, all_logits, parent, seq);
  upload_layout();
  run();
  if (logits)
    ck(mk_download(ctx_, logits, logits_.p, lay_.logit_rows.size() * static_cast<size_t>(cfg_.n_vocab) * sizeof(float)));
  else
    ck(mk_synchronize(ctx_));
  check_device();
}

void Model::move_kv(int from, int to, int seq) {
  if (from == to) return;
  ck(mk_move_kv(ctx_, &kv_, seq, from, to));
}

void Model::kv_row(int layer, int seq, int pos, bool k, uint8_t* out) {
  const auto& c = cfg_;
  const int KV = c.n_head_kv, D = c.head_dim;
  for (int g = 0; g < KV; ++g) {
    const size_t row = ((static_cast<size_t>(layer) * n_seq_ + seq) * KV + g) * n_ctx_ + pos;
    ck(mk_download(ctx_, out + static_cast<size_t>(g) * D, (k ? kc_ : vc_).as<int8_t>() + row * D, D));
    if (k) {  // device K rows are permuted (malkin_hip.h, mk_kv_cache): back to element order
      std::vector<uint8_t> tmp(out + static_cast<size_t>(g) * D, out + static_cast<size_t>(g + 1) * D);
      const int DC = D / 16;
      for (int e = 0; e < D; ++e) out[static_cast<size_t>(g) * D + e] = tmp[DC * (e % 16) + e / 16];
    }
    ck(mk_download(ctx_, out + static_cast<size_t>(KV) * D + 4 * g, (k ? ks_ : vs_).as<float>() + row, 4));
  }
}

void Model::generate_greedy(const int32_t* prompt, int n_prompt, int n_gen, int seq, int32_t* out, GenStats* st,
                            bool use_graph) {
  if (n_prompt <= 0 || n_gen <= 0) throw std::invalid_argument("generate: empty prompt or no tokens");
  if (n_prompt + n_gen > n_ctx_) throw std::runtime_error("forward: context full");
  const int B = kMaxBatch;
  int32_t* d_top1 = top_.as<int32_t>();
  int32_t* d_tokens = top_.as<int32_t>() + B;  // generated ids (n_gen <= B per call segment below)
  int32_t* d_counter = top_.as<int32_t>() + 2 * B;
  std::vector<BatchToken> batch;
  hipStream_t s = static_cast<hipStream_t>(mk_stream(ctx_));

  // Prefill in kDevBatch-token forwards (the reference's engine takes 256 per forward, engine.cpp:381-393; the
  // per-token results are the same either way).
  const auto t0 = Clock::now();
  for (int pos = 0; pos < n_prompt; pos += kDevBatch) {
    const int m = std::min(kDevBatch, n_prompt - pos);
    batch.clear();
    for (int i = 0; i < m; ++i) batch.push_back({prompt[pos + i], seq, pos + i, pos + i + 1 == n_prompt});
    layout_batch(batch.data(), m, kDevBatch);
    upload_layout();
    run();
  }
  ck(mk_argmax_top2(ctx_, logits_.as<float>(), 1, cfg_.n_vocab, d_top1, nullptr));
  int32_t first = 0;
  ck(mk_download(ctx_, &first, d_top1, sizeof first));
  check_device();
  if (st) st->prefill_ms = ms_since(t0);
  out[0] = first;
  if (n_gen == 1) return;

  // Decode: one-token layout resident on the device; greedy_advance feeds each argmax back as the next input.
  batch.assign(1, BatchToken{first, seq, n_prompt, true});
  layout_batch(batch.data(), 1);
  lay_.max_keys = n_prompt + n_gen;  // attention sized for the last step
  upload_layout();
  const int steps = n_gen - 1;
  std::vector<int32_t> toks(steps);
  const auto t1 = Clock::now();
  for (int done = 0; done < steps;) {
    const int seg = std::min(B, steps - done);  // d_tokens holds B ids
    ck(mk_fill(ctx_, d_counter, 0, sizeof(int32_t)));
    auto step = [&] {
      run();
      ck(mk_argmax_top2(ctx_, logits_.as<float>(), 1, cfg_.n_vocab, d_top1, nullptr));
      ck(mk_greedy_advance(ctx_, d_top1, d_ids_, d_rpos_, d_kv_row_, d_n_keys_, d_tokens, d_counter));
    };
    if (use_graph) {
      hipGraph_t g = nullptr;
      hipGraphExec_t ge = nullptr;
      hck(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        step();
      } catch (...) {
        (void)hipStreamEndCapture(s, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      hck(hipStreamEndCapture(s, &g), "hipStreamEndCapture");
      hck(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
      for (int i = 0; i < seg; ++i) hck(hipGraphLaunch(ge, s), "hipGraphLaunch");
      ck(mk_synchronize(ctx_));
      (void)hipGraphExecDestroy(ge);
      (void)hipGraphDestroy(g);
    } else {
      for (int i = 0; i < seg; ++i) step();
    }
    ck(mk_download(ctx_, toks.data() + done, d_tokens, seg * sizeof(int32_t)));
    check_device();
    done += seg;
  }
  if (st) {
    st->decode_ms = ms_since(t1);
    st->decode_forwards = steps;
  }
  std::copy(toks.begin(), toks.end(), out + 1);
}

}  // namespace malkin_hip
