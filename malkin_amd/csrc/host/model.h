// Qwen3 dense decoder on one MI355X: the device counterpart of the reference's malkin::Model (model.h:11-97).
// Same public API and semantics (BatchToken batches, plain / tree forwards, move_kv, the reference's error texts);
// weights, KV cache, activations and the per-token layout live in HBM and every op is a gfx950 kernel behind the
// C ABI of include/malkin_hip.h.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../../../include/malkin_hip.h"
#include "gguf.h"

namespace malkin_hip {

struct ModelConfig {  // model.h:11-16
  std::string arch, name;
  int n_layer = 0, n_embd = 0, n_ff = 0, n_head = 0, n_head_kv = 0, head_dim = 0;
  int n_ctx_train = 0, n_vocab = 0;
  float rope_base = 10000.0f, rms_eps = 1e-6f;
};

ModelConfig read_config(const GgufFile& f);  // model.cpp:78-101

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

class Model {
 public:
  static constexpr int kMaxBatch = 256;  // model.h:35

  // wide: the reference's wide Q6_K prefill panels are packed (Engine packs them when RAM allows,
  // engine.cpp:130-145); MALKIN_NO_WIDE turns them off there.
  Model(mk_ctx* ctx, const GgufFile& f, int n_ctx, int n_seq = 1, bool wide = true);
  ~Model();
  const ModelConfig& cfg() const { return cfg_; }
  int n_ctx() const { return n_ctx_; }
  int n_seq() const { return n_seq_; }

  // model.h:52 — logits: n_vocab floats per token with .logits set, in batch order (host memory).
  void forward(const BatchToken* batch, int n, float* logits);
  // model.h:58-59
  void forward(const int32_t* tokens, int n, int pos, float* logits, bool all_logits, const int* parent = nullptr,
               int seq = 0);
  // model.h:61
  void move_kv(int from, int to, int seq = 0);

  // Same forward, logits left in device memory; top1/top2 (host, may be null): per logits row, the first maximum
  // and the reference's runner-up (sampler.cpp:27-30, engine.cpp:309-318).
  void forward_top2(const BatchToken* batch, int n, int32_t* top1, int32_t* top2);
  const float* dev_logits() const { return logits_.as<float>(); }
  int n_out() const { return static_cast<int>(out_.size()); }

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
  // Packed matmul weight: which = 0 qkv, 1 wo, 2 gate|up, 3 down of `layer`; 4 the LM head.
  mk_weight weight(int layer, int which) const;

 private:
  struct Weight {
    int type = 0;
    int64_t rows = 0, cols = 0;
    int64_t out_off = 0;  // first output row within its group (q|k|v, gate|up)
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
  };

  void load_weight(const GgufFile& f, const std::vector<std::string>& names, Weight& w, bool interleave4 = false);
  void load_gateup(const GgufFile& f, const std::string& gate, const std::string& up, Group& g);
  void load_group(const GgufFile& f, const std::vector<std::string>& names, Group& g);
  void matmul_group(const Group& g, const void* xq, int n, float* y);
  // The group from fp32 rows x (token stride xs) with rmsnorm (norm_w) / quantization inside each matmul; false when
  // a part has no fused kernel for n tokens (nothing launched then).
  bool matmul_group_f32(const Group& g, const float* x, int64_t xs, const float* norm_w, int n, float* y);
  void build_layout(const BatchToken* batch, int n);
  void upload_layout(int n);
  void run(int n);  // device forward over the uploaded layout
  void check_ids(const int32_t* ids, int n);

  mk_ctx* ctx_;
  ModelConfig cfg_;
  int n_ctx_, n_seq_;
  bool wide_;
  size_t weight_bytes_ = 0;
  int embd_type_ = 0;
  size_t embd_row_bytes_ = 0;
  DevBuf embd_rows_;  // token_embd in GGUF rows (lookup)
  Weight output_;     // LM head (packed token_embd when tied)
  DevBuf output_norm_;
  std::vector<Layer> layers_;
  DevBuf rope_cos_, rope_sin_;  // [n_ctx][D/2]
  DevBuf kc_, vc_, ks_, vs_;    // KV cache: [layer][seq][kv_head][n_ctx] rows of D int8 / one float

  // Per-token layout (host copies + one device block).
  std::vector<int32_t> ids_, rpos_, seq_, kv_row_, n_keys_, anc_off_, anc_, out_;
  std::vector<int> depth_;
  bool tree_ = false;
  bool distinct_seqs_ = false;  // no two tokens of the batch share a sequence
  int max_keys_ = 0;
  std::vector<int32_t> host_block_;
  DevBuf layout_;
  int32_t *d_ids_, *d_rpos_, *d_seq_, *d_kv_row_, *d_n_keys_, *d_anc_off_, *d_anc_, *d_out_;

  // Activations for kMaxBatch tokens.
  DevBuf x_, qkv_, att_, gu_, xq_, logits_, top_;
};

}  // namespace malkin_hip
