// TEST INFRASTRUCTURE ONLY. A C ABI over the reference's own code, compiled together with the
// reference sources under /root/reference/src by oracle/Makefile into oracle/_ref/. It lets
// tests check the C restatement (liboracle.so) against the real scalar table and LlamaModel,
// and lets bench.py time the reference CPU path. Nothing in the product loads it.
#include "core/dtype.h"
#include "kernels/kernels.h"
#include "model/kv_cache.h"
#include "model/llama.h"
#include "axon/sampler.h"

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <span>
#include <vector>

using axon::BlockQ4_0;
using axon::BlockQ4_1;
using axon::BlockQ6_K;
using axon::BlockQ8_0;

namespace {
const axon::kernels::KernelTable& T() { return axon::kernels::scalar_kernels(); }

struct RefModel {
  std::unique_ptr<axon::model::LlamaModel> model;
  std::vector<std::unique_ptr<axon::model::KVCache>> caches;
};
}  // namespace

extern "C" {

// ---- conversions and blocks (src/core/dtype.cpp) ----
float ref_fp16_to_fp32(std::uint16_t h) { return axon::fp16_to_fp32(h); }
std::uint16_t ref_fp32_to_fp16(float f) { return axon::fp32_to_fp16(f); }
float ref_bf16_to_fp32(std::uint16_t h) { return axon::bf16_to_fp32(h); }
std::uint16_t ref_fp32_to_bf16(float f) { return axon::fp32_to_bf16(f); }
void ref_dequantize_block_q6_k(const void* b, float* out) {
  axon::dequantize_block_q6_k(*static_cast<const BlockQ6_K*>(b), out);
}

// ---- the 30 scalar table entries (src/kernels/kernels.cpp:16-47) ----
void ref_matmul_f32(const float* w, const float* x, float* y, size_t o, size_t i) { T().matmul_f32(w, x, y, o, i); }
void ref_matmul_f16(const std::uint16_t* w, const float* x, float* y, size_t o, size_t i) { T().matmul_f16(w, x, y, o, i); }
void ref_matmul_bf16(const std::uint16_t* w, const float* x, float* y, size_t o, size_t i) { T().matmul_bf16(w, x, y, o, i); }
void ref_matmul_f32_rows(const float* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_f32_rows(w, x, y, r, o, i, s); }
void ref_matmul_f16_rows(const std::uint16_t* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_f16_rows(w, x, y, r, o, i, s); }
void ref_matmul_bf16_rows(const std::uint16_t* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_bf16_rows(w, x, y, r, o, i, s); }
void ref_rmsnorm(const float* x, const float* w, float* y, size_t n, float eps) { T().rmsnorm(x, w, y, n, eps); }
void ref_rope(float* x, size_t n_heads, size_t pos, size_t head_dim, size_t rotary_dim, float theta, int style,
              const float* factors) {
  const axon::kernels::RopeParams p{.head_dim = head_dim,
                                    .rotary_dim = rotary_dim,
                                    .theta = theta,
                                    .style = style == 0 ? axon::kernels::RopeStyle::Normal
                                                        : axon::kernels::RopeStyle::NeoX,
                                    .freq_factors = factors};
  T().rope(x, n_heads, pos, p);
}
void ref_softmax(float* x, size_t n) { T().softmax(x, n); }
void ref_silu_mul(const float* g, const float* u, float* o, size_t n) { T().silu_mul(g, u, o, n); }
void ref_embedding_row(int type, const void* table, size_t n, std::int64_t index, float* out) {
  T().embedding_row(static_cast<axon::DType>(type), table, n, index, out);
}
void ref_attention_kv_heads(const float* q, const float* k, const float* v, float* out, float* scores, size_t n_q,
                            size_t n_past, size_t n_head, size_t n_head_kv, size_t head_dim, float scale, size_t hb,
                            size_t he) {
  T().attention_kv_heads(q, k, v, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale, hb, he);
}
void ref_attention_kv_heads_f16(const float* q, const std::uint16_t* k, const std::uint16_t* v, float* out,
                                float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                                size_t head_dim, float scale, size_t hb, size_t he) {
  T().attention_kv_heads_f16(q, k, v, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale, hb, he);
}
void ref_quantize_row_q8_0(const float* x, void* out, size_t n) {
  T().quantize_row_q8_0(x, static_cast<BlockQ8_0*>(out), n);
}
void ref_matmul_q8_0(const void* w, const float* x, float* y, size_t o, size_t i) { T().matmul_q8_0(static_cast<const BlockQ8_0*>(w), x, y, o, i); }
void ref_matmul_q4_0(const void* w, const float* x, float* y, size_t o, size_t i) { T().matmul_q4_0(static_cast<const BlockQ4_0*>(w), x, y, o, i); }
void ref_matmul_q4_1(const void* w, const float* x, float* y, size_t o, size_t i) { T().matmul_q4_1(static_cast<const BlockQ4_1*>(w), x, y, o, i); }
void ref_matmul_q6_k(const void* w, const float* x, float* y, size_t o, size_t i) { T().matmul_q6_k(static_cast<const BlockQ6_K*>(w), x, y, o, i); }
void ref_matmul_q8_0_q8(const void* w, const void* x, float* y, size_t o, size_t i) { T().matmul_q8_0_q8(static_cast<const BlockQ8_0*>(w), static_cast<const BlockQ8_0*>(x), y, o, i); }
void ref_matmul_q4_0_q8(const void* w, const void* x, float* y, size_t o, size_t i) { T().matmul_q4_0_q8(static_cast<const BlockQ4_0*>(w), static_cast<const BlockQ8_0*>(x), y, o, i); }
void ref_matmul_q4_1_q8(const void* w, const void* x, float* y, size_t o, size_t i) { T().matmul_q4_1_q8(static_cast<const BlockQ4_1*>(w), static_cast<const BlockQ8_0*>(x), y, o, i); }
void ref_matmul_q8_0_rows(const void* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q8_0_rows(static_cast<const BlockQ8_0*>(w), x, y, r, o, i, s); }
void ref_matmul_q4_0_rows(const void* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q4_0_rows(static_cast<const BlockQ4_0*>(w), x, y, r, o, i, s); }
void ref_matmul_q4_1_rows(const void* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q4_1_rows(static_cast<const BlockQ4_1*>(w), x, y, r, o, i, s); }
void ref_matmul_q6_k_rows(const void* w, const float* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q6_k_rows(static_cast<const BlockQ6_K*>(w), x, y, r, o, i, s); }
void ref_matmul_q8_0_q8_rows(const void* w, const void* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q8_0_q8_rows(static_cast<const BlockQ8_0*>(w), static_cast<const BlockQ8_0*>(x), y, r, o, i, s); }
void ref_matmul_q4_0_q8_rows(const void* w, const void* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q4_0_q8_rows(static_cast<const BlockQ4_0*>(w), static_cast<const BlockQ8_0*>(x), y, r, o, i, s); }
void ref_matmul_q4_1_q8_rows(const void* w, const void* x, float* y, size_t r, size_t o, size_t i, size_t s) { T().matmul_q4_1_q8_rows(static_cast<const BlockQ4_1*>(w), static_cast<const BlockQ8_0*>(x), y, r, o, i, s); }

// ---- LlamaModel (src/model/llama.h:83-153) ----
// Returns a handle or null; the error message is copied into err.
// LlamaModel::load on the scalar table; cache_f16 selects CacheType::F16 for every cache.
void* ref_model_load_cache(const char* path, size_t max_seq, size_t max_ctx, size_t max_batch, int n_threads,
                           int exact_activations, int cache_f16, char* err, size_t err_len) {
  axon::model::LoadOptions opts;
  opts.cache = cache_f16 != 0 ? axon::model::CacheType::F16 : axon::model::CacheType::F32;
  opts.max_seq = max_seq;
  opts.max_ctx = max_ctx;
  opts.max_batch = max_batch;
  opts.n_threads = n_threads;
  opts.exact_activations = exact_activations != 0;
  opts.kernels = axon::kernels::KernelSet::Scalar;
  auto model = axon::model::LlamaModel::load(path, opts);
  if (!model) {
    if (err != nullptr && err_len > 0) {
      std::strncpy(err, model.error().message.c_str(), err_len - 1);
      err[err_len - 1] = 0;
    }
    return nullptr;
  }
  auto* h = new RefModel;
  h->model = std::move(*model);
  return h;
}

void* ref_model_load(const char* path, size_t max_seq, size_t max_ctx, size_t max_batch, int n_threads,
                     int exact_activations, char* err, size_t err_len) {
  return ref_model_load_cache(path, max_seq, max_ctx, max_batch, n_threads, exact_activations, 0, err, err_len);
}

void ref_model_free(void* h) { delete static_cast<RefModel*>(h); }

int ref_model_threads(void* h) { return static_cast<RefModel*>(h)->model->n_threads(); }

size_t ref_model_weight_bytes(void* h) { return static_cast<RefModel*>(h)->model->weight_bytes_per_token(); }

// A new cache of the model's type owned by the handle; returns its index.
int ref_cache_new(void* h) {
  auto* m = static_cast<RefModel*>(h);
  m->caches.push_back(std::make_unique<axon::model::KVCache>(m->model->new_cache()));
  return static_cast<int>(m->caches.size()) - 1;
}

size_t ref_cache_pos(void* h, int c) { return static_cast<RefModel*>(h)->caches[c]->pos(); }

void ref_cache_truncate(void* h, int c, size_t pos) { static_cast<RefModel*>(h)->caches[c]->truncate(pos); }

// Fills positions [pos, pos + n) of every layer's K and V with the given rows
// ([n_layer][2][n][row] floats) and advances the cache, as if they had been prefilled.
void ref_cache_fill(void* h, int c, const float* rows, size_t n) {
  auto* m = static_cast<RefModel*>(h);
  auto& cache = *m->caches[c];
  const size_t row = cache.row_floats();
  const size_t pos = cache.pos();
  for (size_t l = 0; l < cache.n_layer(); ++l) {
    if (cache.type() == axon::model::CacheType::F16) {
      for (size_t i = 0; i < n * row; ++i) {
        cache.k16(l)[pos * row + i] = axon::fp32_to_fp16(rows[(l * 2 + 0) * n * row + i]);
        cache.v16(l)[pos * row + i] = axon::fp32_to_fp16(rows[(l * 2 + 1) * n * row + i]);
      }
      continue;
    }
    std::memcpy(cache.k(l) + pos * row, rows + (l * 2 + 0) * n * row, n * row * sizeof(float));
    std::memcpy(cache.v(l) + pos * row, rows + (l * 2 + 1) * n * row, n * row * sizeof(float));
  }
  cache.advance(n);
}

static int copy_logits(const axon::Expected<std::span<const float>>& r, float* out) {
  if (!r) {
    return -1;
  }
  std::memcpy(out, r->data(), r->size() * sizeof(float));
  return 0;
}

int ref_forward(void* h, const std::int32_t* tokens, size_t n, float* logits) {
  auto* m = static_cast<RefModel*>(h);
  return copy_logits(m->model->forward(std::span<const std::int32_t>(tokens, n)), logits);
}

int ref_forward_prefill(void* h, int c, const std::int32_t* tokens, size_t n, float* logits) {
  auto* m = static_cast<RefModel*>(h);
  return copy_logits(m->model->forward_prefill(*m->caches[c], std::span<const std::int32_t>(tokens, n)), logits);
}

int ref_forward_batch(void* h, const int* cache_ids, const std::int32_t* tokens, size_t n, float* logits) {
  auto* m = static_cast<RefModel*>(h);
  std::vector<axon::model::KVCache*> caches(n);
  for (size_t i = 0; i < n; ++i) {
    caches[i] = m->caches[cache_ids[i]].get();
  }
  return copy_logits(m->model->forward_batch(caches, std::span<const std::int32_t>(tokens, n)), logits);
}

// `draws` calls of Sampler::sample (src/sampling/sampler.cpp:160-183) with one configuration,
// seed and row of logits, into out[draws].
void ref_sample(const float* logits, size_t n, const std::int32_t* recent, size_t n_recent, float temperature,
                int top_k, float top_p, float min_p, float repeat_penalty, int repeat_last_n, std::uint64_t seed,
                size_t draws, std::int32_t* out) {
  axon::SamplerConfig cfg;
  cfg.temperature = temperature;
  cfg.top_k = top_k;
  cfg.top_p = top_p;
  cfg.min_p = min_p;
  cfg.repeat_penalty = repeat_penalty;
  cfg.repeat_last_n = repeat_last_n;
  cfg.seed = seed;
  axon::Sampler sampler(cfg, static_cast<std::int32_t>(n));
  for (size_t i = 0; i < draws; ++i)
    out[i] = sampler.sample(std::span<const float>(logits, n), std::span<const std::int32_t>(recent, n_recent));
}

}  // extern "C"
