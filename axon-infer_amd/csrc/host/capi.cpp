// C ABI of the device-resident forward pass (include/axon_model.h).

#include "axon_model.h"

#include "axon_hip.h"
#include "model.h"

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

struct axon_model {
  std::unique_ptr<axon::model::LlamaModel> m;
  std::map<int, std::unique_ptr<axon::model::KVCache>> caches;
  // Per-call argument staging, sized at load for max_batch + 1 rows, so that a pass through
  // this interface allocates no host memory (tests/unit/test_model_forward.cpp:119-128).
  std::vector<axon::model::KVCache*> batch;
  std::vector<std::span<const int32_t>> windows;
  std::vector<axon::sampling::Config> configs;
};

namespace {

thread_local std::string g_error;

int fail(const axon::Error& e) {
  g_error = e.message;
  return e.code == axon::ErrorCode::Device ? AXON_HIP_E_HIP
         : e.code == axon::ErrorCode::Unsupported ? AXON_HIP_E_UNSUPPORTED
                                                  : AXON_HIP_E_INVALID;
}

int fail(const std::string& msg) {
  g_error = msg;
  return AXON_HIP_E_INVALID;
}

axon::model::KVCache* find(axon_model* model, int cache) {
  const auto it = model->caches.find(cache);
  return it == model->caches.end() ? nullptr : it->second.get();
}

int copy_out(const axon::Expected<std::span<const float>>& r, float* logits) {
  if (!r) return fail(r.error());
  if (logits != nullptr) std::memcpy(logits, r->data(), r->size() * sizeof(float));
  return 0;
}

}  // namespace

extern "C" {

const char* axon_model_last_error(void) { return g_error.c_str(); }

int axon_model_load(const char* path, const axon_model_options* options, axon_model** out) {
  *out = nullptr;
  axon::model::LoadOptions o;
  if (options != nullptr) {
    if (options->max_seq) o.max_seq = options->max_seq;
    if (options->max_ctx) o.max_ctx = options->max_ctx;
    if (options->max_batch) o.max_batch = options->max_batch;
    o.max_caches = options->max_caches;
    o.exact_activations = options->exact_activations != 0;
    if (options->cache_type != 0 && options->cache_type != 1)
      return fail("cache_type: expected 0 (F32) or 1 (F16), found " + std::to_string(options->cache_type));
    o.cache = options->cache_type == 1 ? axon::model::CacheType::F16 : axon::model::CacheType::F32;
    o.repack = options->no_repack == 0;
    o.persistent_decode = options->no_persistent == 0;
    if (options->kernels != nullptr && !axon::kernels::parse_kernel_set(options->kernels, o.kernels))
      return fail(std::string("kernels: expected auto, scalar, neon or hip, found '") + options->kernels + "'");
  }
  auto m = axon::model::LlamaModel::load(path, o);
  if (!m) return fail(m.error());
  auto* model = new axon_model{std::move(*m), {}, {}, {}, {}};
  const size_t rows = model->m->max_seq() + model->m->max_batch() + 1;
  model->batch.reserve(rows);
  model->windows.reserve(rows);
  model->configs.reserve(rows);
  *out = model;
  return 0;
}

void axon_model_free(axon_model* model) { delete model; }

int axon_model_get_info(const axon_model* model, axon_model_info* out) {
  const auto& c = model->m->config();
  out->n_layer = c.n_layer;
  out->n_embd = c.n_embd;
  out->n_head = c.n_head;
  out->n_head_kv = c.n_head_kv;
  out->n_ff = c.n_ff;
  out->n_vocab = c.n_vocab;
  out->head_dim = c.head_dim;
  out->rotary_dim = c.rotary_dim;
  out->max_seq = model->m->max_seq();
  out->max_ctx = model->m->max_ctx();
  out->max_batch = model->m->max_batch();
  out->weight_bytes_per_token = model->m->weight_bytes_per_token();
  out->device_bytes = model->m->device_bytes();
  out->kv_bytes_per_position = static_cast<size_t>(c.n_layer) * 2 * c.n_embd_kv() * model->m->kv_element_bytes();
  out->cache_type = model->m->cache_type() == axon::model::CacheType::F16 ? 1 : 0;
  out->persistent_decode = model->m->persistent_decode() ? 1 : 0;
  return 0;
}

int axon_model_set_persistent_decode(axon_model* model, int on) {
  auto r = model->m->set_persistent_decode(on != 0);
  if (!r) return fail(r.error());
  return 0;
}

const char* axon_model_table_name(const axon_model* model) {
  static thread_local std::string name;
  name = std::string(axon::kernels::name(model->m->table()));
  return name.c_str();
}

int axon_model_cache_new(axon_model* model, int* cache) {
  auto c = model->m->new_cache();
  if (!c) return fail(c.error());
  *cache = (*c)->slot();
  model->caches[*cache] = std::move(*c);
  return 0;
}

int axon_model_cache_free(axon_model* model, int cache) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("cache_free: unknown cache " + std::to_string(cache));
  model->m->release_cache(*c);
  model->caches.erase(cache);
  return 0;
}

int axon_model_cache_pos(axon_model* model, int cache, size_t* pos) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("cache_pos: unknown cache " + std::to_string(cache));
  *pos = c->pos();
  return 0;
}

int axon_model_cache_truncate(axon_model* model, int cache, size_t pos) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("cache_truncate: unknown cache " + std::to_string(cache));
  if (!c->truncate(pos)) return fail("truncate: " + std::to_string(pos) + " exceeds the cached " + std::to_string(c->pos()));
  return 0;
}

int axon_model_cache_read(axon_model* model, int cache, size_t layer, int values, size_t n, float* out) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("cache_read: unknown cache " + std::to_string(cache));
  auto r = model->m->read_cache(*c, layer, values != 0, n);
  if (!r) return fail(r.error());
  std::memcpy(out, r->data(), r->size() * sizeof(float));
  return 0;
}

int axon_model_cache_fill(axon_model* model, int cache, const float* rows, size_t n) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("cache_fill: unknown cache " + std::to_string(cache));
  auto r = model->m->fill_cache(*c, rows, n);
  return r ? 0 : fail(r.error());
}

int axon_model_forward(axon_model* model, const int32_t* tokens, size_t n, float* logits) {
  if (logits == nullptr) {
    auto r = model->m->forward_device(std::span<const int32_t>(tokens, n));
    return r ? 0 : fail(r.error());
  }
  return copy_out(model->m->forward(std::span<const int32_t>(tokens, n)), logits);
}

int axon_model_forward_prefill(axon_model* model, int cache, const int32_t* tokens, size_t n, float* logits) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("forward_prefill: unknown cache " + std::to_string(cache));
  if (logits == nullptr) {
    auto r = model->m->forward_prefill_device(*c, std::span<const int32_t>(tokens, n));
    return r ? 0 : fail(r.error());
  }
  return copy_out(model->m->forward_prefill(*c, std::span<const int32_t>(tokens, n)), logits);
}

int axon_model_generate_greedy(axon_model* model, int cache, int32_t token, size_t n, int32_t* out) {
  axon::model::KVCache* c = find(model, cache);
  if (c == nullptr) return fail("generate: unknown cache " + std::to_string(cache));
  if (out == nullptr && n > 0) return fail("generate: out is NULL");
  auto r = model->m->generate_greedy(*c, token, std::span<int32_t>(out, n));
  return r ? 0 : fail(r.error());
}

int axon_model_forward_batch(axon_model* model, const int* caches, const int32_t* tokens, size_t n, float* logits) {
  std::vector<axon::model::KVCache*>& cs = model->batch;
  cs.resize(n);
  for (size_t i = 0; i < n; ++i) {
    cs[i] = find(model, caches[i]);
    if (cs[i] == nullptr) return fail("forward_batch: unknown cache " + std::to_string(caches[i]));
  }
  if (logits == nullptr) {
    auto r = model->m->forward_batch_device(cs, std::span<const int32_t>(tokens, n));
    return r ? 0 : fail(r.error());
  }
  return copy_out(model->m->forward_batch(cs, std::span<const int32_t>(tokens, n)), logits);
}

int axon_model_forward_mixed(axon_model* model, int prefill_cache, const int32_t* prefill, size_t n_prefill,
                             const int* caches, const int32_t* tokens, size_t n, float* logits) {
  axon::model::KVCache* pc = nullptr;
  if (n_prefill != 0) {
    if (prefill == nullptr) return fail("forward_mixed: prefill tokens are NULL");
    pc = find(model, prefill_cache);
    if (pc == nullptr) return fail("forward_mixed: unknown cache " + std::to_string(prefill_cache));
  }
  if (n != 0 && (caches == nullptr || tokens == nullptr)) return fail("forward_mixed: caches or tokens are NULL");
  std::vector<axon::model::KVCache*>& cs = model->batch;
  cs.resize(n);
  for (size_t i = 0; i < n; ++i) {
    cs[i] = find(model, caches[i]);
    if (cs[i] == nullptr) return fail("forward_mixed: unknown cache " + std::to_string(caches[i]));
  }
  const std::span<const int32_t> chunk(prefill, n_prefill), toks(tokens, n);
  if (logits == nullptr) {
    auto r = model->m->forward_mixed_device(pc, chunk, cs, toks);
    return r ? 0 : fail(r.error());
  }
  return copy_out(model->m->forward_mixed(pc, chunk, cs, toks), logits);
}

int axon_model_greedy(axon_model* model, const int32_t* const* recent, const size_t* recent_len, float repeat_penalty,
                      int repeat_last_n, int32_t* ids, size_t n) {
  if (ids == nullptr && n != 0) return fail("greedy: ids is NULL");
  std::vector<std::span<const int32_t>>& windows = model->windows;
  windows.clear();
  if (recent != nullptr) {
    if (recent_len == nullptr) return fail("greedy: recent_len is NULL");
    windows.resize(n);
    for (size_t i = 0; i < n; ++i) {
      if (recent[i] == nullptr && recent_len[i] != 0) return fail("greedy: recent[" + std::to_string(i) + "] is NULL");
      windows[i] = std::span<const int32_t>(recent[i], recent_len[i]);
    }
  }
  auto r = model->m->greedy(std::span<int32_t>(ids, n), windows, repeat_penalty, repeat_last_n);
  return r ? 0 : fail(r.error());
}

static_assert(sizeof(axon_rng) == sizeof(axon::sampling::Rng), "axon_rng mirrors sampling::Rng");

void axon_rng_seed(axon_rng* rng, uint64_t seed) { reinterpret_cast<axon::sampling::Rng*>(rng)->seed(seed); }
uint64_t axon_rng_next(axon_rng* rng) { return reinterpret_cast<axon::sampling::Rng*>(rng)->next(); }
double axon_rng_uniform(axon_rng* rng) { return reinterpret_cast<axon::sampling::Rng*>(rng)->uniform(); }

namespace {
axon::sampling::Config config_of(const axon_sampler_config& c) {
  return axon::sampling::Config{c.temperature, c.top_k, c.top_p, c.min_p, c.repeat_penalty, c.repeat_last_n};
}
}  // namespace

int axon_model_sample(axon_model* model, const axon_sampler_config* configs, axon_rng* rngs,
                      const int32_t* const* recent, const size_t* recent_len, int32_t* ids, size_t n) {
  if (n != 0 && (configs == nullptr || rngs == nullptr || ids == nullptr))
    return fail("sample: configs, generators and ids are required");
  std::vector<axon::sampling::Config>& cs = model->configs;
  cs.resize(n);
  for (size_t i = 0; i < n; ++i) cs[i] = config_of(configs[i]);
  std::vector<std::span<const int32_t>>& windows = model->windows;
  windows.clear();
  if (recent != nullptr) {
    if (recent_len == nullptr) return fail("sample: recent_len is NULL");
    windows.resize(n);
    for (size_t i = 0; i < n; ++i) {
      if (recent[i] == nullptr && recent_len[i] != 0) return fail("sample: recent[" + std::to_string(i) + "] is NULL");
      windows[i] = std::span<const int32_t>(recent[i], recent_len[i]);
    }
  }
  auto r = model->m->sample(std::span<int32_t>(ids, n), cs,
                            std::span<axon::sampling::Rng>(reinterpret_cast<axon::sampling::Rng*>(rngs), n), windows);
  return r ? 0 : fail(r.error());
}

int axon_sample_candidates(const axon_sampler_config* config, axon_rng* rng, const float* logits, const int32_t* ids,
                           size_t n, int32_t* out) {
  if (config == nullptr || rng == nullptr || logits == nullptr || ids == nullptr || out == nullptr || n == 0)
    return fail("sample_candidates: every argument is required and n >= 1");
  if (!(config->temperature > 0.0F)) return fail("sample_candidates: the temperature must be above zero");
  std::vector<double> probs(n);
  *out = axon::sampling::draw(config_of(*config), *reinterpret_cast<axon::sampling::Rng*>(rng), logits, ids, n,
                              probs.data());
  return 0;
}

int axon_model_probe(axon_model* model, int type, int enable) {
  auto r = model->m->set_probe(type, enable != 0);
  return r ? 0 : fail(r.error());
}

int axon_model_probe_read(axon_model* model, double* ms, size_t* launches, double* bytes) {
  auto r = model->m->read_probe();
  if (!r) return fail(r.error());
  *ms = r->ms;
  *launches = r->launches;
  *bytes = r->bytes;
  return 0;
}

}  // extern "C"
