// Qwen3 dense decoder on one MI355X: the device counterpart of the reference's malkin::Model (model.h:11-97).
// Same public API and semantics (BatchToken batches, plain / tree forwards, move_kv, the reference's error texts);
// weights, KV cache, activations and the per-token layout live in HBM and every op is a gfx950 kernel behind the
// C ABI of include/malkin_hip.h.
//
// Host waits: a forward that returns logits or picks to the host waits once for them; enqueue() and move_kv() only
// queue work on the context's stream. Per-forward layouts travel from a ring of pinned host blocks by asynchronous
// copies, so several forwards can be queued back to back (the engine's draft rounds).
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../../include/malkin_hip.h"
#include "gguf.h"

namespace malkin_hip {

struct ModelConfig {  // model.h:11-16
  std::string arch, name;
  int n_layer = 0, n_embd = 0, n_ff = 0, n_head = 0, n_head_kv = 0, head_dim = 0;
  int n_ctx_train = 0, n_vocab = 0;
  float rope_base = 10000.0f, rms_eps = 1e-6f;
  // End-of-generation ids (Tokenizer::is_eog's set, tokenizer.cpp:93-102), ascending, each < n_vocab.
  std::vector<int32_t> eog;
};

// Hyperparameters from the GGUF metadata (the keys of model.cpp:78-101, same defaults and error texts).
ModelConfig read_config(const GgufFile& f);
// End-of-generation ids the metadata names (tokenizer.cpp:93-102), ascending, unique; not yet bounded by the
// vocabulary size.
std::vector<int32_t> read_eog(const GgufFile& f);

// model.h:25-30
struct BatchToken {
  int32_t id;
  int seq, pos;
  bool logits;
  int kv = -1, parent = -1;
};

// Device buffer owned by the model.
struct DevBuf {
  mk_ctx* ctx = nullptr;
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(mk_ctx* c, size_t n);
  DevBuf(DevBuf&& o) noexcept : ctx(o.ctx), p(o.p), bytes(o.bytes) { o.p = nullptr; }
  DevBuf& operator=(DevBuf&& o) noexcept;
  ~DevBuf();
  template <typename T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// What every kernel of one forward needs to know about its tokens. Built on the host from either forward form,
// then copied to the device as one block.
struct TokenLayout {
  int n = 0;
  std::vector<int32_t> id, rope_pos, seq, kv_row, n_keys;  // per token
  std::vector<int32_t> id_from;  // per token: index into a device id array the token's id is read from, or -1
  std::vector<int32_t> logit_rows;  // tokens whose logits are produced, in batch order
  // Tree batches: token t attends to its n_keys[t] contiguous rows, then to rows extra[extra_at[t] .. extra_at[t+1]).
  bool tree = false;
  std::vector<int32_t> extra_at, extra;
  // Derived: the longest key list, and whether no two tokens share a sequence.
  int max_keys = 0;
  bool distinct_seqs = false;
};

class Model {
 public:
  static constexpr int kMaxBatch = 256;  // model.h:35: tokens per forward through the public API
  // Tokens per device forward of a prompt inside generate_greedy: per-token results do not depend on how the
  // prompt is split, and 512-token forwards give the prefill GEMMs twice the workgroups of 256-token ones.
  static constexpr int kDevBatch = 512;

  // wide: the reference's wide Q6_K prefill panels are packed (Engine packs them when RAM allows,
  // engine.cpp:130-145); MALKIN_NO_WIDE turns them off there.
  // no_pack: every matmul on the reference's row path over GGUF rows (its MALKIN_NO_PACK, model.cpp:136).
  // decode: how one-token forwards run their layers where the shape allows (kDecodeSteps: one launch per step;
  // kDecodePersistent: every layer in one launch, mk_decode_layers; kDecodeFusedAttn: each layer's attention and
  // attn_output in one launch, mk_decode_attn_wo). The results are the same.
  enum { kDecodeSteps = 0, kDecodePersistent = 1, kDecodeFusedAttn = 2 };
  Model(mk_ctx* ctx, const GgufFile& f, int n_ctx, int n_seq = 1, bool wide = true, bool no_pack = false,
        int decode = kDecodeSteps);
  ~Model();
  const ModelConfig& cfg() const { return cfg_; }
  int n_ctx() const { return n_ctx_; }
  int n_seq() const { return n_seq_; }
  mk_ctx* ctx() const { return ctx_; }

  // model.h:52 — logits: n_vocab floats per token with .logits set, in batch order (host memory).
  void forward(const BatchToken* batch, int n, float* logits);
  // model.h:58-59
  void forward(const int32_t* tokens, int n, int pos, float* logits, bool all_logits, const int* parent = nullptr,
               int seq = 0);
  // model.h:61. Queued on the stream (no wait): later forwards see the moved rows.
  void move_kv(int from, int to, int seq = 0);

  // Same forward, logits left in device memory; top1/top2 (host, may be null): per logits row, the first maximum
  // and the reference's runner-up (sampler.cpp:27-30, engine.cpp:309-318). Waits once.
  void forward_top2(const BatchToken* batch, int n, int32_t* top1, int32_t* top2);
  // Queues the forward of `batch` without waiting. id_from (host, n entries, may be null): token t takes its id from
  // dev_ids[id_from[t]] at run time when id_from[t] >= 0 (an id another queued kernel produces), else batch[t].id.
  // The picks of the logits rows (in batch order) go to dev_top1 / dev_top2 (device; either may be null).
  void enqueue(const BatchToken* batch, int n, const int32_t* id_from, const int32_t* dev_ids, int32_t* dev_top1,
               int32_t* dev_top2);
  // The last forward's logits rows (device, n_vocab floats each, in batch order); samplers penalize them in place.
  float* dev_logits() const { return logits_.as<float>(); }
  int n_out() const { return static_cast<int>(lay_.logit_rows.size()); }

  // Greedy generation of one sequence (the reference's `malkin bench` protocol, main.cpp:126-143): the prompt in
  // kMaxBatch-token forwards, then n_gen tokens, each from the argmax of the previous forward. The decode steps are
  // captured once as a HIP graph that keeps the token and position on the device.
  struct GenStats {
    double prefill_ms = 0, decode_ms = 0;
    int decode_forwards = 0;
  };
  void generate_greedy(const int32_t* prompt, int n_prompt, int n_gen, int seq, int32_t* out, GenStats* st,
                       bool use_graph = true);

  // KV row of (layer, seq, pos) in the reference's layout (KV*D int8, then KV float scales), for tests.
  void kv_row(int layer, int seq, int pos, bool k, uint8_t* out);

  // Bytes of packed weights resident in HBM, and the GGUF bytes of the matmul weights one decode token reads.
  size_t weight_bytes() const { return weight_bytes_; }
  // Whether one-token forwards run the persistent decode kernel (mk_decode_layers); after a host wait on the model's
  // stream, check_device() raises if one of its launches since the last check timed out in a hand-off wait.
  bool persistent() const { return dplan_ != nullptr && decode_ == kDecodePersistent; }
  bool fused_attn() const { return dplan_ != nullptr && decode_ == kDecodeFusedAttn; }
  void check_device();
  // Packed matmul weight: which = 0 qkv, 1 wo, 2 gate|up, 3 down of `layer`; 4 the LM head.
  mk_weight weight(int layer, int which) const;

 private:
  struct Weight {
    int type = 0;
    int64_t rows = 0, cols = 0;
    int64_t out_off = 0;  // first output row within its group (q|k|v, gate|up)
    bool raw = false;     // kept as GGUF rows (no CDNA layout)
    bool rowdot = false;  // raw: the row path's arithmetic (mk_matmul_rows); else the panel arithmetic on GGUF rows
                          // (mk_matmul_gguf, Q5_K)
    size_t row_bytes = 0;
    DevBuf packed;
    mk_weight w() const;
  };
  // Matrices sharing one input, packed as few weights as possible: consecutive matrices of the same type are
  // concatenated by rows (one launch); a type change (Q4_K_M mixes) starts a new weight.
  struct Group {
    std::vector<Weight> parts;
    int64_t rows = 0;
    // gate|up packed as one weight with rows interleaved by 4 (4 gate rows, then the 4 up rows of the same outputs):
    // the decode matmul then applies silu_mul itself (mk_matmul_f32 silu_pairs).
    bool silu_pairs = false;
  };
  struct Layer {
    DevBuf norms;  // attn_norm[E], ffn_norm[E], q_norm[D], k_norm[D]
    Group qkv, gateup;
    Weight wo, down;
    bool row_flow = false;  // some weight is on the row path: unfused rmsnorm / quantize / silu steps
  };
  // A pinned staging block of the weight loader and its device twin (freed once loading is done, or on unwinding).
  struct LoadBlock {
    mk_ctx* ctx = nullptr;
    uint8_t* host = nullptr;
    void* done = nullptr;  // event after the copy that reads `host`
    DevBuf dev;
    LoadBlock() = default;
    LoadBlock(const LoadBlock&) = delete;
    LoadBlock& operator=(const LoadBlock&) = delete;
    void release();
    ~LoadBlock() { release(); }
  };
  // One pinned host block per in-flight layout copy, reusable once its event has passed.
  struct Staging {
    int32_t* host = nullptr;
    void* done = nullptr;  // event recorded after the copy that reads `host`
  };

  void load_weight(const GgufFile& f, const std::vector<std::string>& names, Weight& w, bool interleave4 = false);
  void load_gateup(const GgufFile& f, const std::string& gate, const std::string& up, Group& g, bool interleave);
  void stream_rows(int64_t rows, size_t row_bytes,
                   const std::function<std::pair<const uint8_t*, int64_t>(int64_t)>& src,
                   const std::function<void(const void*, int64_t, int64_t)>& consume, void* dest);
  // One group's matmul, every part on its own path: packed parts read xq (BlockQ8 rows), row-path parts xf too.
  void matmul_any(const Group& g, const float* xf, int64_t xfs, const void* xq, int n, float* y);
  void load_group(const GgufFile& f, const std::vector<std::string>& names, Group& g);
  void matmul_group(const Group& g, const void* xq, int n, float* y);
  // The group from fp32 rows x (token stride xs) with rmsnorm (norm_w) / quantization inside each matmul; false when
  // a part has no fused kernel for n tokens (nothing launched then).
  bool matmul_group_f32(const Group& g, const float* x, int64_t xs, const float* norm_w, int n, float* y);

  // Layout builders (validation with the reference's error texts), the asynchronous upload, and the layer loop.
  void layout_batch(const BatchToken* batch, int n, int limit = kMaxBatch);
  void layout_tokens(const int32_t* tokens, int n, int pos, bool all_logits, const int* parent, int seq);
  void finish_layout();
  void upload_layout(const int32_t* dev_ids = nullptr);
  void run();
  void run_row_layer(const Layer& L, int il);
  void make_decode_plan();
  void check_ids();

  mk_ctx* ctx_;
  ModelConfig cfg_;
  int n_ctx_, n_seq_;
  bool wide_, no_pack_;
  size_t weight_bytes_ = 0;
  LoadBlock load_[2];
  size_t load_block_bytes_ = 0;
  int embd_type_ = 0;
  int64_t embd_count_ = 0;  // token_embd rows (valid token ids)
  size_t embd_row_bytes_ = 0;
  DevBuf embd_rows_;  // token_embd in GGUF rows (lookup)
  Weight output_;     // LM head (packed token_embd when tied)
  DevBuf output_norm_;
  std::vector<Layer> layers_;
  DevBuf rope_cos_, rope_sin_;  // [n_ctx][D/2]
  DevBuf kc_, vc_, ks_, vs_;    // KV cache: [layer][seq][kv_head][n_ctx] rows of D int8 / one float
  mk_kv_cache kv_{};

  TokenLayout lay_;
  // Device layout block: ids rope_pos seq kv_row n_keys logit_rows id_from [kDevBatch each], extra_at [B + 1],
  // extra [B (B + 1) / 2] with B = kMaxBatch (tree batches come through the public API only).
  DevBuf layout_;
  size_t layout_words_ = 0;
  int32_t *d_ids_, *d_rpos_, *d_seq_, *d_kv_row_, *d_n_keys_, *d_out_, *d_id_from_, *d_extra_at_, *d_extra_;
  std::vector<Staging> staging_;
  size_t next_staging_ = 0;

  // Activations for kMaxBatch tokens.
  DevBuf x_, qkv_, att_, gu_, xq_, logits_, top_;
  mk_decode_plan* dplan_ = nullptr;  // the persistent decode kernel's plan (all layers Q8_0, fused groups)
  bool dplan_pending_ = false;       // launched since the last check_device()
  int decode_ = kDecodeSteps;
  DevBuf h_;  // fp32 normalized rows of the row-path layers (kDevBatch x n_embd)
};

}  // namespace malkin_hip
