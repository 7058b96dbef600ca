// extern "C" layer of include/malkin_hip.h over the internal launchers.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "ctx.h"
#include "ops.h"

namespace mk {

namespace {
thread_local char g_err[512] = "";
std::atomic<uint64_t> g_host_waits{0};
std::atomic<uint64_t> g_host_bytes{0};
// Pinned blocks from mk_host_alloc (start -> bytes): copies into them count as downloads.
std::mutex g_pinned_m;
std::map<uintptr_t, size_t> g_pinned;
bool pinned(const void* p, size_t bytes) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  std::lock_guard<std::mutex> lk(g_pinned_m);
  auto it = g_pinned.upper_bound(a);
  if (it == g_pinned.begin()) return false;
  --it;
  return a + bytes <= it->first + it->second;
}
}

void count_host_wait() { g_host_waits.fetch_add(1, std::memory_order_relaxed); }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
  set_error("%s: %s", what, hipGetErrorString(e));
  return MK_ERR_HIP;
}

}  // namespace mk

using mk::check;
using mk::guard;
using mk::require;

extern "C" {

const char* mk_last_error(void) { return mk::g_err; }

int mk_init(int device, mk_ctx** out) {
  return guard([&] {
    require(out != nullptr, "mk_init: null output");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw mk::Error(MK_ERR_NO_DEVICE, "no HIP device");
    require(device >= 0 && device < count, "mk_init: bad device index");
    check(hipSetDevice(device), "hipSetDevice");
    auto* c = new mk_ctx;
    c->device = device;
    hipDeviceProp_t p;
    check(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
    std::snprintf(c->name, sizeof c->name, "%s", p.gcnArchName);
    c->n_cu = p.multiProcessorCount;
    check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
    check(hipEventCreate(&c->ev0), "hipEventCreate");
    check(hipEventCreate(&c->ev1), "hipEventCreate");
    c->scratch_bytes = 1 << 20;
    check(hipMalloc(&c->scratch, c->scratch_bytes), "hipMalloc");
    check(hipMalloc(&c->meta, 64), "hipMalloc");
    *out = c;
  });
}

int mk_destroy(mk_ctx* c) {
  return guard([&] {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    (void)hipEventDestroy(c->ev0);
    (void)hipEventDestroy(c->ev1);
    (void)hipStreamDestroy(c->stream);
    (void)hipFree(c->scratch);
    (void)hipFree(c->meta);
    delete c;
  });
}

const char* mk_device_name(const mk_ctx* c) { return c ? c->name : ""; }

int mk_reserve_scratch(mk_ctx* c, size_t bytes) {
  return guard([&] {
    if (bytes <= c->scratch_bytes) return;
    check(hipSetDevice(c->device), "hipSetDevice");
    mk::count_host_wait();
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    void* p = nullptr;
    check(hipMalloc(&p, bytes), "hipMalloc");
    (void)hipFree(c->scratch);
    c->scratch = p;
    c->scratch_bytes = bytes;
  });
}

size_t mk_attention_scratch_bytes(int head_dim, int max_keys, int pairs) {
  return head_dim > 0 && max_keys > 0 && pairs > 0 ? mk::attention_scratch_bytes(head_dim, max_keys, pairs) : 0;
}

int mk_synchronize(mk_ctx* c) {
  return guard([&] {
    mk::count_host_wait();
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

uint64_t mk_host_waits(void) { return mk::g_host_waits.load(std::memory_order_relaxed); }
uint64_t mk_host_bytes(void) { return mk::g_host_bytes.load(std::memory_order_relaxed); }

void* mk_stream(mk_ctx* c) { return c ? c->stream : nullptr; }

int mk_malloc(mk_ctx* c, size_t bytes, void** dev) {
  return guard([&] {
    require(dev != nullptr, "mk_malloc: null output");
    check(hipSetDevice(c->device), "hipSetDevice");
    check(hipMalloc(dev, bytes ? bytes : 1), "hipMalloc");
  });
}

int mk_free(mk_ctx* c, void* dev) {
  return guard([&] {
    if (!dev) return;
    check(hipSetDevice(c->device), "hipSetDevice");
    mk::count_host_wait();
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    check(hipFree(dev), "hipFree");
  });
}

int mk_upload(mk_ctx* c, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    if (!bytes) return;
    check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpy H2D");
    mk::count_host_wait();
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

int mk_download(mk_ctx* c, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    if (!bytes) return;
    check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "hipMemcpy D2H");
    mk::g_host_bytes.fetch_add(bytes, std::memory_order_relaxed);
    mk::count_host_wait();
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  });
}

int mk_host_alloc(mk_ctx* c, size_t bytes, void** host) {
  return guard([&] {
    require(host != nullptr, "mk_host_alloc: null output");
    check(hipSetDevice(c->device), "hipSetDevice");
    check(hipHostMalloc(host, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
    std::lock_guard<std::mutex> lk(mk::g_pinned_m);
    mk::g_pinned[reinterpret_cast<uintptr_t>(*host)] = bytes ? bytes : 1;
  });
}

int mk_host_free(mk_ctx* c, void* host) {
  return guard([&] {
    if (!host) return;
    check(hipSetDevice(c->device), "hipSetDevice");
    mk::count_host_wait();
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    check(hipHostFree(host), "hipHostFree");
    std::lock_guard<std::mutex> lk(mk::g_pinned_m);
    mk::g_pinned.erase(reinterpret_cast<uintptr_t>(host));
  });
}

int mk_copy_async(mk_ctx* c, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    if (!bytes) return;
    check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, c->stream), "hipMemcpyAsync");
    if (mk::pinned(dst, bytes) && !mk::pinned(src, bytes)) mk::g_host_bytes.fetch_add(bytes, std::memory_order_relaxed);
  });
}

int mk_event_record(mk_ctx* c, void** event) {
  return guard([&] {
    require(event != nullptr, "mk_event_record: null event");
    if (!*event) {
      hipEvent_t e = nullptr;
      check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
      *event = e;
    }
    check(hipEventRecord(static_cast<hipEvent_t>(*event), c->stream), "hipEventRecord");
  });
}

int mk_event_done(void* event) {
  if (!event) return 1;
  return hipEventQuery(static_cast<hipEvent_t>(event)) == hipSuccess ? 1 : 0;
}

int mk_event_wait(mk_ctx*, void* event) {
  return guard([&] {
    if (!event) return;
    mk::count_host_wait();
    check(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
  });
}

int mk_event_free(void* event) {
  return guard([&] {
    if (event) check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
  });
}

int mk_fill(mk_ctx* c, void* dev, int v, size_t bytes) {
  return guard([&] { mk::fill(c->stream, dev, v, bytes); });
}

int mk_timer_start(mk_ctx* c) {
  return guard([&] { check(hipEventRecord(c->ev0, c->stream), "hipEventRecord"); });
}

int mk_timer_stop(mk_ctx* c, float* ms) {
  return guard([&] {
    check(hipEventRecord(c->ev1, c->stream), "hipEventRecord");
    mk::count_host_wait();
    check(hipEventSynchronize(c->ev1), "hipEventSynchronize");
    check(hipEventElapsedTime(ms, c->ev0, c->ev1), "hipEventElapsedTime");
  });
}

size_t mk_packed_bytes(int type, int64_t rows, int64_t cols) { return mk::packed_bytes(type, rows, cols); }

int mk_pack_weight(mk_ctx* c, int type, const void* src, size_t srb, int64_t rows, int64_t cols, void* dst) {
  return guard([&] { mk::pack_weight(c->stream, type, src, srb, rows, cols, dst); });
}

int mk_pack_weight_rows(mk_ctx* c, int type, const void* src, size_t srb, int64_t row0, int64_t n_rows, int64_t rows,
                        int64_t cols, void* dst) {
  return guard([&] { mk::pack_weight_rows(c->stream, type, src, srb, row0, n_rows, rows, cols, dst); });
}

int mk_unpack_weight(mk_ctx* c, int type, const void* packed, int64_t rows, int64_t cols, void* dst) {
  return guard([&] { mk::unpack_weight(c->stream, type, packed, rows, cols, dst); });
}

int mk_quantize_q8(mk_ctx* c, const float* x, int n, int64_t k, void* xq) {
  return guard([&] { mk::quantize_q8(c->stream, x, n, k, static_cast<mk::BlockQ8*>(xq)); });
}

int mk_quantize_i8(mk_ctx* c, const float* x, int rows, int n, int8_t* q, float* d) {
  return guard([&] { mk::quantize_i8_rows(c->stream, x, rows, n, q, d); });
}

int mk_dequantize_rows(mk_ctx* c, int type, const void* src, size_t row_bytes, const int32_t* ids, int n, int64_t k,
                       float* dst) {
  return guard([&] { mk::dequantize_rows(c->stream, type, src, row_bytes, ids, n, k, dst); });
}

int mk_matmul(mk_ctx* c, const mk_weight* w, const void* xq, int n, float* y, int64_t ys, int accumulate) {
  return guard([&] {
    require(w != nullptr, "mk_matmul: null weight");
    mk::matmul(c->stream, w->type, w->wide != 0, w->data, w->rows, w->cols, static_cast<const mk::BlockQ8*>(xq), n, y,
               ys, accumulate != 0);
  });
}

int mk_matmul_f32(mk_ctx* c, const mk_weight* w, const float* x, int64_t x_stride, const float* norm_w, float eps,
                  int n, float* y, int64_t ys, int accumulate, int silu_pairs) {
  return guard([&] {
    require(w != nullptr, "mk_matmul_f32: null weight");
    if (!mk::matmul_f32_supported(w->type, w->wide != 0, w->rows, w->cols, n, norm_w != nullptr))
      throw mk::Error(MK_ERR_UNSUPPORTED, "mk_matmul_f32: no fused kernel (needs 1 or 2 tokens, a multiple of 32 "
                                          "columns, <= 8192 with rmsnorm, a Q8_0/Q4_K/Q6_K weight)");
    mk::matmul_f32(c->stream, w->type, w->wide != 0, w->data, w->rows, w->cols, x, x_stride, norm_w, eps, n, y, ys,
                   accumulate != 0, silu_pairs != 0);
  });
}

int mk_rmsnorm(mk_ctx* c, const float* x, const float* w, int rows, int n, float eps, float* y) {
  return guard([&] { mk::rmsnorm(c->stream, x, w, rows, n, eps, y); });
}

int mk_rmsnorm_q8(mk_ctx* c, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                  void* xq) {
  return guard([&] { mk::rmsnorm_q8(c->stream, x, rows_idx, w, rows, n, eps, static_cast<mk::BlockQ8*>(xq)); });
}

int mk_rmsnorm_rows(mk_ctx* c, const float* x, const int32_t* rows_idx, const float* w, int rows, int n, float eps,
                    float* y) {
  return guard([&] { mk::rmsnorm(c->stream, x, w, rows, n, eps, y, rows_idx); });
}

int mk_silu_mul_rows(mk_ctx* c, float* gu, int rows, int64_t n) {
  return guard([&] { mk::silu_mul_rows(c->stream, gu, rows, n); });
}

int mk_matmul_rows(mk_ctx* c, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols, const float* x,
                   int64_t x_stride, const void* xq, int n, float* y, int64_t y_stride, int accumulate) {
  return guard([&] {
    require(w != nullptr && y != nullptr && rows >= 0 && n >= 0, "matmul_rows: bad arguments");
    mk::matmul_rows(c->stream, type, w, row_bytes, rows, cols, x, x_stride, static_cast<const mk::BlockQ8*>(xq), n, y,
                    y_stride, accumulate != 0);
  });
}

int mk_matmul_gguf(mk_ctx* c, int type, const void* w, size_t row_bytes, int64_t rows, int64_t cols, const void* xq,
                   int n, float* y, int64_t y_stride, int accumulate) {
  return guard([&] {
    require(w != nullptr && y != nullptr && rows >= 0 && n >= 0, "matmul_gguf: bad arguments");
    mk::matmul_gguf(c->stream, type, w, row_bytes, rows, cols, static_cast<const mk::BlockQ8*>(xq), n, y, y_stride,
                    accumulate != 0);
  });
}

int mk_silu_mul(mk_ctx* c, int64_t n, float* g, const float* u) {
  return guard([&] { mk::silu_mul(c->stream, n, g, u); });
}

int mk_silu_mul_q8(mk_ctx* c, const float* gu, int rows, int64_t n, int interleave4, void* xq) {
  return guard([&] { mk::silu_mul_q8(c->stream, gu, rows, n, static_cast<mk::BlockQ8*>(xq), interleave4 != 0); });
}

int mk_add(mk_ctx* c, int64_t n, float* x, const float* h) {
  return guard([&] { mk::add(c->stream, n, x, h); });
}

int mk_attend_gqa(mk_ctx* c, const float* q, int G, int D, const int8_t* k, const int8_t* v, size_t stride,
                  ptrdiff_t soff, int n, float scale, float* out, const int32_t* extra, int ne) {
  return guard([&] {
    require(G > 0 && n >= 0 && ne >= 0 && n + ne > 0, "attend_gqa: bad sizes");
    // The batched kernel's layout for one token of sequence 0: n contiguous keys, then ne extra rows. Written into
    // the context's metadata words by a kernel in stream order: no allocation, no host synchronization.
    int32_t* dm = c->meta;
    mk::put4(c->stream, dm, 0, n, 0, ne);
    mk::AttnAddr a{k, v, reinterpret_cast<const char*>(k) + soff, reinterpret_cast<const char*>(v) + soff,
                   0, 0, (int64_t)stride, 0, 0, (int64_t)stride, 0};
    mk::attention(c->stream, q, (int64_t)G * D, out, (int64_t)G * D, 1, G, 1, D, scale, a, dm, dm + 1,
                  ne > 0 ? dm + 2 : nullptr, extra, n + ne, c->scratch, c->scratch_bytes);
  });
}

static mk::KvLayer kv_layer(const mk_kv_cache* kv, int layer) {
  require(kv != nullptr && layer >= 0 && layer < kv->n_layer, "bad KV cache / layer");
  const size_t rows = (size_t)layer * kv->n_seq * kv->n_head_kv * kv->n_ctx;
  return mk::KvLayer{kv->k + rows * kv->head_dim, kv->v + rows * kv->head_dim, kv->k_scale + rows, kv->v_scale + rows};
}

int mk_qk_norm_rope_kv(mk_ctx* c, float* q, float* k, const float* v, int64_t stride, int n, int n_head,
                       const float* q_norm, const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                       const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const mk_kv_cache* kv,
                       int layer) {
  return guard([&] {
    const mk::KvLayer L = kv_layer(kv, layer);
    mk::qk_norm_rope_kv(c->stream, q, k, v, stride, n, n_head, kv->n_head_kv, kv->head_dim, q_norm, k_norm, eps, cos_t,
                        sin_t, rpos, seq, kv_row, L, kv->n_ctx);
  });
}

namespace {

void attention_rows(mk_ctx* c, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int n_head,
                    const mk_kv_cache* kv, int layer, const int32_t* seq, const int32_t* n_keys,
                    const int32_t* anc_off, const int32_t* anc, int max_keys, void* xq) {
  const mk::KvLayer L = kv_layer(kv, layer);
  const int D = kv->head_dim;
  const int64_t rows = (int64_t)kv->n_ctx;
  mk::AttnAddr a{L.k, L.v, reinterpret_cast<const char*>(L.ks), reinterpret_cast<const char*>(L.vs),
                 (int64_t)kv->n_head_kv * rows * D, rows * D, D,
                 (int64_t)kv->n_head_kv * rows * 4, rows * 4, 4, 1};
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));  // model.cpp:208
  mk::attention(c->stream, q, q_stride, out, out_stride, n, n_head, kv->n_head_kv, D, scale, a, seq, n_keys, anc_off,
                anc, max_keys, c->scratch, c->scratch_bytes, static_cast<mk::BlockQ8*>(xq), (int64_t)n_head * D / 32);
}

void attention_decode(mk_ctx* c, const float* qkv, int64_t stride, int n, int n_head, const float* q_norm,
                      const float* k_norm, float eps, const float* cos_t, const float* sin_t, const int32_t* rpos,
                      const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys, const mk_kv_cache* kv,
                      int layer, float* out, int64_t out_stride, int max_keys, void* xq) {
  const mk::KvLayer L = kv_layer(kv, layer);
  const int D = kv->head_dim, KV = kv->n_head_kv;
  require(n_head > 0 && n_head % KV == 0 && max_keys > 0, "mk_attention_decode: bad head layout");
  const int64_t rows = (int64_t)kv->n_ctx;
  mk::AttnAddr a{L.k, L.v, reinterpret_cast<const char*>(L.ks), reinterpret_cast<const char*>(L.vs),
                 (int64_t)KV * rows * D, rows * D, D, (int64_t)KV * rows * 4, rows * 4, 4, 1};
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));  // model.cpp:208
  if (!mk::attention_decode_fused(c->stream, qkv, stride, out, out_stride, n, n_head, KV, D, scale, a, q_norm,
                                  k_norm, eps, cos_t, sin_t, rpos, seq, kv_row, n_keys, L, kv->n_ctx, max_keys,
                                  static_cast<mk::BlockQ8*>(xq), (int64_t)n_head * D / 32))
    throw mk::Error(MK_ERR_UNSUPPORTED, "mk_attention_decode: no fused kernel for this head layout / key count");
}

}  // namespace

int mk_attention_q8(mk_ctx* c, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int n_head,
                    const mk_kv_cache* kv, int layer, const int32_t* seq, const int32_t* n_keys,
                    const int32_t* anc_off, const int32_t* anc, int max_keys, void* xq) {
  return guard([&] {
    require(xq != nullptr, "mk_attention_q8: xq is NULL");
    attention_rows(c, q, q_stride, out, out_stride, n, n_head, kv, layer, seq, n_keys, anc_off, anc, max_keys, xq);
  });
}

int mk_attention_decode_q8(mk_ctx* c, const float* qkv, int64_t stride, int n, int n_head, const float* q_norm,
                           const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                           const int32_t* rpos, const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys,
                           const mk_kv_cache* kv, int layer, float* out, int64_t out_stride, int max_keys, void* xq) {
  return guard([&] {
    require(xq != nullptr, "mk_attention_decode_q8: xq is NULL");
    attention_decode(c, qkv, stride, n, n_head, q_norm, k_norm, eps, cos_t, sin_t, rpos, seq, kv_row, n_keys, kv,
                     layer, out, out_stride, max_keys, xq);
  });
}

int mk_attention(mk_ctx* c, const float* q, int64_t q_stride, float* out, int64_t out_stride, int n, int n_head,
                 const mk_kv_cache* kv, int layer, const int32_t* seq, const int32_t* n_keys, const int32_t* anc_off,
                 const int32_t* anc, int max_keys) {
  return guard([&] {
    attention_rows(c, q, q_stride, out, out_stride, n, n_head, kv, layer, seq, n_keys, anc_off, anc, max_keys,
                   nullptr);
  });
}

int mk_attention_decode(mk_ctx* c, const float* qkv, int64_t stride, int n, int n_head, const float* q_norm,
                        const float* k_norm, float eps, const float* cos_t, const float* sin_t, const int32_t* rpos,
                        const int32_t* seq, const int32_t* kv_row, const int32_t* n_keys, const mk_kv_cache* kv,
                        int layer, float* out, int64_t out_stride, int max_keys) {
  return guard([&] {
    attention_decode(c, qkv, stride, n, n_head, q_norm, k_norm, eps, cos_t, sin_t, rpos, seq, kv_row, n_keys, kv,
                     layer, out, out_stride, max_keys, nullptr);
  });
}

int mk_move_kv(mk_ctx* c, const mk_kv_cache* kv, int seq, int from, int to) {
  return guard([&] {
    require(kv && seq >= 0 && seq < kv->n_seq && from >= 0 && from < kv->n_ctx && to >= 0 && to < kv->n_ctx,
            "move_kv: bad row");
    mk::move_kv_rows(c->stream, kv->k, kv->v, kv->k_scale, kv->v_scale, kv->n_layer, kv->n_seq, kv->n_head_kv,
                     kv->head_dim, kv->n_ctx, seq, from, to);
  });
}

int mk_move_ids(mk_ctx* c, int32_t* dst, const int32_t* dst_index, const int32_t* src, const int32_t* src_index,
                int n) {
  return guard([&] { mk::move_ids(c->stream, dst, dst_index, src, src_index, n); });
}

int mk_greedy_advance(mk_ctx* c, const int32_t* top1, int32_t* ids, int32_t* rpos, int32_t* kv_row, int32_t* n_keys,
                      int32_t* out_tokens, int32_t* counter) {
  return guard([&] { mk::greedy_advance(c->stream, top1, ids, rpos, kv_row, n_keys, out_tokens, counter); });
}

int mk_argmax_top2(mk_ctx* c, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2) {
  return guard([&] { mk::argmax_top2(c->stream, logits, rows, n_vocab, top1, top2, c->scratch, c->scratch_bytes); });
}

int mk_argmax_top2_noalloc(void* stream, const float* logits, int rows, int n_vocab, int32_t* top1, int32_t* top2) {
  return guard([&] { mk::argmax_top2_noalloc(static_cast<hipStream_t>(stream), logits, rows, n_vocab, top1, top2); });
}

int mk_penalize(mk_ctx* c, float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
                const int32_t* pen_off, const int32_t* pen_id, const float* pen_amt) {
  return guard([&] {
    require(logits && n_rows >= 0 && n_vocab > 0 && stride >= n_vocab, "penalize: bad logits");
    mk::penalize(c->stream, logits, stride, rows, n_rows, n_vocab, pen_off, pen_id, pen_amt);
  });
}

int mk_topk(mk_ctx* c, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab, int k,
            float* values, int32_t* ids) {
  return guard([&] {
    require(logits && values && ids && n_rows >= 0 && n_vocab > 0 && stride >= n_vocab, "topk: bad arguments");
    mk::topk(c->stream, logits, stride, rows, n_rows, n_vocab, k, values, ids);
  });
}

size_t mk_sample_cut_workspace(int n_rows, int n_vocab) {
  size_t n = 0;
  return guard([&] { n = mk::sample_cut_workspace(n_rows, n_vocab); }) == MK_OK ? n : 0;
}

int mk_sample_cut(mk_ctx* c, const float* logits, int64_t stride, const int32_t* rows, int n_rows, int n_vocab,
                  const mk_cut_params* params, int cap, float* values, int32_t* ids, int32_t* keep, double* sums,
                  void* workspace, size_t workspace_bytes) {
  return guard([&] {
    require(c && logits && params && values && ids && keep && sums && n_rows >= 0 && n_vocab > 0 &&
                stride >= n_vocab,
            "sample_cut: bad arguments");
    mk::sample_cut(c->stream, logits, stride, rows, n_rows, n_vocab, params, cap, values, ids, keep, sums, workspace,
                   workspace_bytes);
  });
}

int mk_sample_cut_tail(mk_ctx* c, void* workspace, int n_rows, int n_vocab, int row, int from, int count,
                       float* values, int32_t* ids) {
  return guard([&] {
    require(c && workspace && values && ids && n_vocab > 0, "sample_cut_tail: bad arguments");
    mk::sample_cut_tail(c->stream, workspace, n_rows, n_vocab, row, from, count, values, ids);
  });
}

int mk_sample_draw(mk_ctx* c, const float* values, const int32_t* ids, int stride, int n_rows,
                   const mk_draw_params* params, uint64_t* states, int n_states, int32_t* out, int n_out) {
  return guard([&] {
    require(c && n_rows >= 0 && n_states >= 0 && n_out >= 0, "sample_draw: bad arguments");
    require(stride >= 1 && stride <= 1024, "sample_draw: stride outside 1..1024 (mk_topk's candidate limit)");
    if (n_rows == 0) return;
    require(values && ids && params && states && out, "sample_draw: null array");
    mk::sample_draw(c->stream, values, ids, stride, n_rows, params, states, n_states, out, n_out);
  });
}

}  // extern "C"

struct mk_decode_plan {
  mk::DecodeDims d{};
  int n_layer = 0;
  void* layers = nullptr;  // device mk::DecodeLayer[n_layer]
  void* args = nullptr;    // device argument block
  unsigned* sync = nullptr;
  size_t sync_bytes = 0;
};

namespace {

void decode_plan_free(mk_decode_plan* p) {
  if (!p) return;
  if (p->layers) (void)hipFree(p->layers);
  if (p->args) (void)hipFree(p->args);
  if (p->sync) (void)hipFree(p->sync);
  delete p;
}

}  // namespace

int mk_decode_plan_create(mk_ctx* c, const mk_decode_layer* layers, int n_layer, int n_head, float eps,
                          const mk_kv_cache* kv, float* x, float* qkv, void* att, float* h, const float* cos_t,
                          const float* sin_t, const int32_t* rpos, const int32_t* seq, const int32_t* kv_row,
                          const int32_t* n_keys, mk_decode_plan** out) {
  return guard([&] {
    require(c && layers && n_layer > 0 && kv && out && n_layer <= kv->n_layer, "mk_decode_plan_create: bad arguments");
    *out = nullptr;
    mk::DecodeDims d{};
    d.E = (int)layers[0].wo.rows;
    d.H = n_head;
    d.KV = kv->n_head_kv;
    d.D = kv->head_dim;
    d.F = (int)layers[0].down.cols;
    d.n_ctx = kv->n_ctx;
    d.n_seq = kv->n_seq;
    d.eps = eps;
    const int64_t QKV = (int64_t)(d.H + 2 * d.KV) * d.D;
    std::vector<mk::DecodeLayer> dl(n_layer);
    for (int i = 0; i < n_layer; ++i) {
      const mk_decode_layer& L = layers[i];
      const bool shapes = L.qkv.type == MK_Q8_0 && L.wo.type == MK_Q8_0 && L.gate_up.type == MK_Q8_0 &&
                          L.down.type == MK_Q8_0 && L.qkv.rows == QKV && L.qkv.cols == d.E && L.wo.rows == d.E &&
                          L.wo.cols == (int64_t)d.H * d.D && L.gate_up.rows == 2 * (int64_t)d.F &&
                          L.gate_up.cols == d.E && L.down.rows == d.E && L.down.cols == d.F;
      if (!shapes) throw mk::Error(MK_ERR_UNSUPPORTED, "mk_decode_plan_create: weights other than Q8_0 / bad shapes");
      require(L.attn_norm && L.ffn_norm && L.q_norm && L.k_norm, "mk_decode_plan_create: missing norm weights");
      dl[i] = mk::DecodeLayer{L.qkv.data,   L.wo.data,     L.gate_up.data, L.down.data,
                              L.attn_norm,  L.ffn_norm,    L.q_norm,       L.k_norm};
    }
    // Keys are bounded by the context; the smallest row (one key) must fit for the plan to be of any use.
    if (!mk::decode_layers_supported(d, 1))
      throw mk::Error(MK_ERR_UNSUPPORTED, "mk_decode_plan_create: no persistent decode kernel for this model shape");
    std::unique_ptr<mk_decode_plan, void (*)(mk_decode_plan*)> p(new mk_decode_plan, decode_plan_free);
    p->d = d;
    p->n_layer = n_layer;
    p->sync_bytes = mk::decode_sync_bytes(n_layer);
    check(hipMalloc(&p->layers, sizeof(mk::DecodeLayer) * n_layer), "hipMalloc");
    check(hipMalloc(&p->args, mk::decode_args_bytes()), "hipMalloc");
    check(hipMalloc(reinterpret_cast<void**>(&p->sync), p->sync_bytes), "hipMalloc");
    check(hipMemcpy(p->layers, dl.data(), sizeof(mk::DecodeLayer) * n_layer, hipMemcpyHostToDevice), "hipMemcpy");
    check(hipMemset(p->sync, 0, p->sync_bytes), "hipMemset");
    mk::DecodeBufs b{};
    b.layers = static_cast<const mk::DecodeLayer*>(p->layers);
    b.kv0 = mk::KvLayer{kv->k, kv->v, kv->k_scale, kv->v_scale};
    b.x = x, b.qkv = qkv, b.att = att, b.h = h;
    b.cos_t = cos_t, b.sin_t = sin_t, b.rpos = rpos, b.seq = seq, b.kv_row = kv_row, b.n_keys = n_keys;
    b.sync = p->sync;
    // About one poll per microsecond: a wait gives up after about half a second.
    b.spin_max = 1u << 19;
    mk::decode_set_args(p->args, d, b);
    *out = p.release();
  });
}

int mk_decode_plan_destroy(mk_decode_plan* p) {
  return guard([&] {
    if (p) check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    decode_plan_free(p);
  });
}

int mk_decode_supported(const mk_decode_plan* p, int max_keys) {
  if (!p) return 0;
  int ok = 0;
  (void)guard([&] { ok = mk::decode_layers_supported(p->d, max_keys) ? 1 : 0; });
  return ok;
}

int mk_decode_layers(mk_ctx* c, mk_decode_plan* p, int l0, int l1, int max_keys) {
  return guard([&] {
    require(c && p && l0 >= 0 && l1 > l0 && l1 <= p->n_layer, "mk_decode_layers: bad layer range");
    mk::decode_layers(c->stream, p->args, p->d, l0, l1, max_keys);
  });
}

int mk_decode_attn_wo(mk_ctx* c, mk_decode_plan* p, int layer, int max_keys) {
  return guard([&] {
    require(c && p && layer >= 0 && layer < p->n_layer, "mk_decode_attn_wo: bad layer");
    mk::decode_attn_wo(c->stream, p->args, p->d, layer, p->n_layer, max_keys);
  });
}

int mk_decode_check(mk_ctx* c, mk_decode_plan* p) {
  return guard([&] {
    require(c && p, "mk_decode_check: no plan");
    unsigned err = 0;
    const unsigned* word = p->sync + mk::decode_error_word(p->n_layer);
    check(hipMemcpy(&err, word, sizeof err, hipMemcpyDeviceToHost), "hipMemcpy");
    if (err != 0) {
      // Some workgroup may have left without resetting the counters: clear them and the error word.
      check(hipMemset(p->sync, 0, p->sync_bytes), "hipMemset");
      throw mk::Error(MK_ERR_HIP, "mk_decode_layers: a hand-off wait timed out (results of the step are invalid)");
    }
  });
}
