/*
 * axon_model — C ABI of the device-resident forward pass (libaxon_host.so), the caller of the
 * hip table. Mirrors trickymind1324/axon-infer's LlamaModel (src/model/llama.h:87-110):
 * load a GGUF file, open per-sequence KV caches, run forward / forward_prefill / forward_one /
 * forward_batch, read logits [rows][n_vocab] on the host. Weights, activations and KV caches
 * live in HBM; caches are slots of one device pool, named by int ids.
 *
 * Every function returns 0 or a negative status; axon_model_last_error() holds the message
 * (the reference's Expected error, src/model/llama.cpp:322-351 and 269-302).
 */
#ifndef AXON_MODEL_H
#define AXON_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct axon_model axon_model;

/* LoadOptions (src/model/llama.h:24-43). max_caches: KV slots in the device pool
 * (0: max_batch + 1). kernels: "hip" or "auto" (anything else is Unsupported here). */
typedef struct {
  size_t max_seq;
  size_t max_ctx;
  size_t max_batch;
  size_t max_caches;
  int exact_activations;
  const char* kernels;
  /* LoadOptions::cache (src/model/llama.h:40-42, CacheType src/model/config.h:16): 0 F32, 1 F16
   * (keys and values rounded once into an fp16 cache; the cache-free forward stays float). */
  int cache_type;
  /* 1: keep the Q6_K output matrix in its GGUF blocks only. 0 (default): also repack it at upload
   * into 16-byte-aligned planes (axon_hip_q6k_repack) that its matmuls stream; same logits. */
  int no_repack;
  /* 1: one-row cached passes launch each step of a layer on its own. 0 (default): they run every
   * layer as one persistent kernel (axon_hip_decode_layers) where the model's shape allows it;
   * same logits either way. */
  int no_persistent;
} axon_model_options;

typedef struct {
  uint32_t n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab, head_dim, rotary_dim;
  size_t max_seq, max_ctx, max_batch;
  size_t weight_bytes_per_token; /* llama.cpp:151-167 */
  size_t device_bytes;
  size_t kv_bytes_per_position;  /* both K and V, all layers, one sequence */
  int cache_type;                /* 0 F32, 1 F16 */
  int persistent_decode;         /* one-row cached passes run as one persistent kernel */
} axon_model_info;

const char* axon_model_last_error(void);
int axon_model_load(const char* path, const axon_model_options* options, axon_model** out);
void axon_model_free(axon_model* model);
int axon_model_get_info(const axon_model* model, axon_model_info* out);
/* The host library's own operator new calls since it was loaded (libaxon_host.so counts its own,
 * as libaxon_hip.so does with axon_hip_allocation_counts). With those, tests pin the reference's
 * "a forward pass performs no heap allocation" (tests/unit/test_model_forward.cpp:119-128) for
 * every pass after the first of each shape. */
size_t axon_model_host_allocations(void);
/* Turns the persistent decode kernel for one-row cached passes on (1) or off (0); on fails with
 * Unsupported where the model's shape does not allow it. No counterpart in the reference, whose
 * passes have no such kernel. A pass whose kernel gave up waiting for a workgroup that never
 * became resident turns it off by itself: that pass fails, naming the cache slot and position,
 * its cache is rolled back to that position, and later one-row passes run layer by layer until
 * this turns the kernel back on. */
int axon_model_set_persistent_decode(axon_model* model, int on);
/* The name of the kernel table the model runs on ("hip"). */
const char* axon_model_table_name(const axon_model* model);

/* KVCache (src/model/kv_cache.h:17-73): new (a free slot), free, position, truncate. */
int axon_model_cache_new(axon_model* model, int* cache);
int axon_model_cache_free(axon_model* model, int cache);
int axon_model_cache_pos(axon_model* model, int cache, size_t* pos);
int axon_model_cache_truncate(axon_model* model, int cache, size_t pos);
/* Rows [0, n) of layer l's keys (values = 0) or values (1) of a cache, to the host as floats
 * (fp16 elements widened exactly). */
int axon_model_cache_read(axon_model* model, int cache, size_t layer, int values, size_t n, float* out);
/* Writes positions [pos, pos + n) of every layer's keys and values from host floats laid out
 * [n_layer][2][n][n_head_kv * head_dim] (K then V per layer) and advances the cache, as if they
 * had been prefilled; an fp16 cache rounds each value to nearest even once. No counterpart entry
 * in the reference, whose KVCache exposes the same rows as host pointers (kv_cache.h:22-40): this is
 * how a caller restores a saved context into device memory, and how tests start the device and
 * the reference from the same cache contents. */
int axon_model_cache_fill(axon_model* model, int cache, const float* rows, size_t n);

/* The passes. logits: host [n][n_vocab], or NULL to leave them in HBM for axon_model_greedy (or
 * for timing the pass alone). */
int axon_model_forward(axon_model* model, const int32_t* tokens, size_t n, float* logits);
int axon_model_forward_prefill(axon_model* model, int cache, const int32_t* tokens, size_t n, float* logits);
int axon_model_forward_batch(axon_model* model, const int* caches, const int32_t* tokens, size_t n, float* logits);
/* One continuous-batching step as one pass. BatchEngine::step (src/engine/batch.cpp:69-156) runs
 * two: forward_prefill of one prompt chunk, then forward_batch of the sequences in decode.
 * prefill_cache takes prefill[0..n_prefill) at its next positions (n_prefill 0: no chunk, and
 * prefill_cache is ignored); caches[i] takes tokens[i] (n may be 0). The chunk is at most
 * max_seq tokens, n at most max_batch, and prefill_cache is not among caches. Every row equals
 * what those two passes compute, bit for bit. logits: host [(n_prefill != 0) + n][n_vocab], the
 * rows that step observes: the chunk's last row (Sequence::prefill_chunk, sequence.cpp:118),
 * then one row per decode cache; the chunk's other rows get no logits. NULL leaves them in HBM
 * for axon_model_greedy, which then takes (n_prefill != 0) + n ids. */
int axon_model_forward_mixed(axon_model* model, int prefill_cache, const int32_t* prefill, size_t n_prefill,
                             const int* caches, const int32_t* tokens, size_t n, float* logits);

/* Sampler::sample at temperature zero on the device (src/sampling/sampler.cpp:67-102) over the
 * last pass's logits, which may have stayed in HBM (logits NULL): the repetition penalty over
 * each row's recent tokens, then std::ranges::max_element per row. recent: n host pointers to
 * each row's token history (prompt included) with recent_len[i] ids, or NULL for no penalty;
 * the window is its last repeat_last_n ids (at most 4096), and repeat_penalty 1 turns it off.
 * n must be the pass's row count. The pass's logits are consumed (rescaled in place); only the
 * n ids cross to the host. */
int axon_model_greedy(axon_model* model, const int32_t* const* recent, const size_t* recent_len, float repeat_penalty,
                      int repeat_last_n, int32_t* ids, size_t n);

/* Engine::generate (src/engine/engine.cpp:50-58) at temperature zero without a repetition
 * penalty: n greedy steps after `token` on `cache`, the ids into out[n]. Each step's id stays on
 * the device for the next step's embedding, so the steps run without host round trips (with the
 * persistent decode kernel; else as the host loop of forward_prefill and greedy). Stop tokens
 * are the caller's to apply to `out` afterwards; the cache advances by n. */
int axon_model_generate_greedy(axon_model* model, int cache, int32_t token, size_t n, int32_t* out);

/* SamplerConfig (include/axon/sampler.h:10-17) without the seed, which seeds an axon_rng. */
typedef struct {
  float temperature; /* 0 or below: greedy */
  int top_k;         /* 0: every id */
  float top_p;       /* 1: off */
  float min_p;       /* 0: off */
  float repeat_penalty;
  int repeat_last_n;
} axon_sampler_config;

/* The sampler's generator (src/sampling/rng.h:11-45): xoshiro256** seeded through SplitMix64.
 * A seed of 0 is used as given (the reference's Sampler draws a clock seed for 0,
 * sampler.cpp:37-48; that choice stays with the caller). */
typedef struct {
  uint64_t s[4];
} axon_rng;
void axon_rng_seed(axon_rng* rng, uint64_t seed);
uint64_t axon_rng_next(axon_rng* rng);
double axon_rng_uniform(axon_rng* rng);

/* Sampler::sample (src/sampling/sampler.cpp:67-183) over the last pass's n rows, row i with
 * configs[i] and generator rngs[i] (each sequence's own Sampler). On the device: each row's
 * repetition penalty (recent as for axon_model_greedy), the greedy choice for rows at temperature
 * zero, and the top-k candidates of the others, descending, equal logits by ascending id (the
 * reference leaves their order unspecified). On the host: temperature, softmax in double, top-p,
 * min-p and one draw from rngs[i] per stochastic row. When every stochastic row keeps at most
 * 256 candidates after top-k, only the ids and those candidates cross to the host; when one
 * keeps more (top_k 0 keeps the whole vocabulary, sampler.cpp:115-117), every row of the call is
 * sorted whole on the device (axon_hip_sort_rows, the same order) and [n][n_vocab] sorted
 * logits and ids cross instead. The first such call allocates device room for its rows (a later
 * call with more rows, again). The pass's logits are consumed. */
int axon_model_sample(axon_model* model, const axon_sampler_config* configs, axon_rng* rngs,
                      const int32_t* const* recent, const size_t* recent_len, int32_t* ids, size_t n);

/* The host stages of axon_model_sample alone (sampler.cpp:120-183): temperature, softmax,
 * top-p, min-p and the draw over n candidates in top-k order (logits descending). *out = the
 * drawn id. */
int axon_sample_candidates(const axon_sampler_config* config, axon_rng* rng, const float* logits, const int32_t* ids,
                           size_t n, int32_t* out);

/* Kernel-time probe (measurement only): while enabled, the kernel of every matmul on weights of
 * ggml type `type` records its dispatch's start and end on HIP events (axon_hip_probe_next_launch);
 * with type AXON_MODEL_PROBE_ATTENTION, each layer's attention launches are bracketed by events
 * instead (their bytes: the rows' visible K and V rows, q and the output). probe_read returns the
 * summed kernel milliseconds, the launch count and the launches' algorithmic bytes, and resets. */
#define AXON_MODEL_PROBE_ATTENTION (-2)
/* With type AXON_MODEL_PROBE_STEP only the persistent decode kernel's launches are bracketed (a
 * probe of the layers' q|k|v type brackets them too, with every other matmul of that type). */
#define AXON_MODEL_PROBE_STEP (-3)
int axon_model_probe(axon_model* model, int type, int enable);
int axon_model_probe_read(axon_model* model, double* ms, size_t* launches, double* bytes);

#ifdef __cplusplus
}
#endif
#endif
