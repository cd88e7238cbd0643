#pragma once

// The device-resident LlamaModel: the caller of the hip table. It mirrors the contract of
// trickymind1324/axon-infer src/model/llama.h:87-110 (load, forward, forward_prefill,
// forward_one, forward_batch, new_cache) and the op order of LlamaModel::run
// (src/model/llama.cpp:315-639), with every weight, activation and KV cache resident in HBM.
// What crosses to the host per forward: the token ids and row positions in (a few bytes per
// row) and the logits out.
//
// Where the reference calls the table per column chunk and per (sequence, head), this model
// issues whole-matrix launches through the coarse entries of include/axon_hip.h: norm + Q8_0
// quantize, fused q|k|v and gate|up matvecs, rope + bias + KV write, one ragged attention
// launch per layer, residual adds fused into the wo and down matvecs.

#include "axon_hip.h"
#include "expected.h"
#include "gguf.h"
#include "kernels.h"
#include "sampler.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <span>
#include <string>
#include <vector>

namespace axon::model {

// Key/value cache storage (src/model/config.h:16): F32 keeps cached decoding bit-identical to
// the cache-free pass; F16 halves the cache and rounds each key and value once when written.
enum class CacheType : std::uint8_t { F32, F16 };

struct LoadOptions {
  std::size_t max_seq = 512;    // rows per prefill call (llama.h:24-43)
  std::size_t max_ctx = 4096;   // positions per cache, clamped to the training context
  std::size_t max_batch = 1;    // rows per forward_batch call
  std::size_t max_caches = 0;   // KV slots on the device (0: max_batch + 1)
  bool exact_activations = false;
  kernels::KernelSet kernels = kernels::KernelSet::Hip;
  CacheType cache = CacheType::F32;  // llama.h:40-42
  // Repack Q6_K matmul weights (the output matrix) at upload into 16-byte-aligned planes; the
  // native blocks stay for the embedding lookup and the table's entries.
  bool repack = true;
  // Run every layer of a one-row cached pass as one persistent kernel (axon_hip_decode_layers)
  // when the model's shape allows it; otherwise, and with false, one launch per step of a layer.
  bool persistent_decode = true;
};

struct Config {
  std::string arch;
  std::uint32_t n_layer = 0, n_embd = 0, n_head = 0, n_head_kv = 0, n_ff = 0, n_ctx_train = 0;
  std::uint32_t n_vocab = 0, head_dim = 0, rotary_dim = 0;
  float rope_theta = 10000.0f, rms_eps = 1e-5f;
  kernels::RopeStyle rope_style = kernels::RopeStyle::Normal;
  bool tie_embeddings = false, attn_bias = false, llama3 = false;
  std::uint32_t n_embd_q() const { return n_head * head_dim; }
  std::uint32_t n_embd_kv() const { return n_head_kv * head_dim; }
};

// A bound weight: its GGUF view on the host and its copy in HBM.
struct Tensor {
  DType type = DType::F32;
  std::uint64_t ne0 = 0, ne1 = 1;
  std::size_t row_bytes = 0, total_bytes = 0;
  const std::byte* host = nullptr;
  void* dev = nullptr;
  void* planar = nullptr;  // Q6_K: the repacked copy the matmuls stream (axon_hip_q6k_repack)
};

struct Layer {
  Tensor attn_norm, wq, wk, wv, wo, ffn_norm, w_gate, w_up, w_down;
  bool bias = false;
  Tensor bq, bk, bv;
};

// One sequence's KV cache: a slot of the device pool, laid out per layer as K rows then V rows
// [max_ctx][n_head_kv * head_dim] (src/model/kv_cache.cpp:15-18).
class KVCache {
public:
  KVCache(int slot, std::size_t max_ctx) : slot_(slot), max_ctx_(max_ctx) {}
  int slot() const { return slot_; }
  std::size_t pos() const { return pos_; }
  std::size_t max_ctx() const { return max_ctx_; }
  void clear() { pos_ = 0; }
  bool truncate(std::size_t pos);
  void advance(std::size_t n) { pos_ += n; }

private:
  int slot_;
  std::size_t max_ctx_;
  std::size_t pos_ = 0;
};

class LlamaModel {
public:
  static Expected<std::unique_ptr<LlamaModel>> load(const std::string& path, LoadOptions options);
  ~LlamaModel();

  // llama.h:87-110. The returned span points into a host buffer owned by the model, valid
  // until the next forward call; logits are [rows][n_vocab].
  Expected<std::span<const float>> forward(std::span<const std::int32_t> tokens);
  Expected<std::span<const float>> forward_prefill(KVCache& cache, std::span<const std::int32_t> tokens);
  Expected<std::span<const float>> forward_one(KVCache& cache, std::int32_t token);
  Expected<std::span<const float>> forward_batch(std::span<KVCache* const> caches,
                                                 std::span<const std::int32_t> tokens);
  // The same passes with the logits left in HBM (logits_device()), for callers that reduce
  // them on the device or time the forward pass alone.
  Expected<std::size_t> forward_device(std::span<const std::int32_t> tokens);
  Expected<std::size_t> forward_prefill_device(KVCache& cache, std::span<const std::int32_t> tokens);
  Expected<std::size_t> forward_batch_device(std::span<KVCache* const> caches, std::span<const std::int32_t> tokens);
  // One continuous-batching step as one pass (batch.cpp:69-156 runs it as two: forward_prefill
  // of one prompt chunk, then forward_batch of the sequences in decode): `prefill` takes
  // `chunk` at its next positions (it may be null with an empty chunk) and caches[i] takes
  // tokens[i]. Every row is computed as in those two passes, bit for bit; the logits are those
  // that step observes: the chunk's last row (Sequence::prefill_chunk, sequence.cpp:118), then
  // one row per decode cache. The chunk and the decode rows together fit max_seq + max_batch.
  Expected<std::span<const float>> forward_mixed(KVCache* prefill, std::span<const std::int32_t> chunk,
                                                 std::span<KVCache* const> caches, std::span<const std::int32_t> tokens);
  Expected<std::size_t> forward_mixed_device(KVCache* prefill, std::span<const std::int32_t> chunk,
                                             std::span<KVCache* const> caches, std::span<const std::int32_t> tokens);
  const float* logits_device() const { return logits_; }
  // Sampler::sample at temperature zero (src/sampling/sampler.cpp:67-102) over the last pass's
  // logits, on the device: the repetition penalty over each row's recent tokens (recent[r], the
  // sequence's tail, prompt included; empty spans or penalty 1 turn it off), then the first
  // maximum. One id per row of that pass into `ids`, whose size must be that row count. Only the
  // ids cross to the host. The pass's logits are consumed: the penalty rescales them in place.
  static constexpr std::size_t kMaxPenaltyWindow = 4096;
  Expected<std::size_t> greedy(std::span<std::int32_t> ids, std::span<const std::span<const std::int32_t>> recent = {},
                               float repeat_penalty = 1.0F, int repeat_last_n = 64);
  // Engine::generate's loop (src/engine/engine.cpp:50-58) at temperature zero without a
  // repetition penalty, for out.size() tokens after `token`: each step's token is the greedy
  // choice of the previous step's logits (forward_one, then Sampler::sample). On the device the
  // chosen id stays in HBM, where the next step's embedding reads it, so the steps run back to
  // back without a host round trip; the ids come to the host once, at the end. The caller
  // applies stop tokens to `out` afterwards: every id up to the first stop token is the one the
  // host loop would produce, and the cache holds out.size() more positions.
  Expected<std::size_t> generate_greedy(KVCache& cache, std::int32_t token, std::span<std::int32_t> out);
  // Sampler::sample (sampler.cpp:67-183) for each row of the last pass, row r with configs[r] and
  // its own generator rngs[r], as each Sequence holds its own Sampler. On the device: each row's
  // repetition penalty, the greedy choice for rows at temperature zero, and the top-k candidates
  // of the others (at most 256: top_k in 1..256, or a vocabulary of at most 256). On the host:
  // the stages after top-k and one draw per stochastic row. Only the ids and the candidates
  // cross to the host. Consumes the pass's logits, as greedy does.
  Expected<std::size_t> sample(std::span<std::int32_t> ids, std::span<const sampling::Config> configs,
                               std::span<sampling::Rng> rngs, std::span<const std::span<const std::int32_t>> recent = {});

  // A fresh cache in a free device slot, or an error when every slot is taken.
  Expected<std::unique_ptr<KVCache>> new_cache();
  void release_cache(const KVCache& cache);
  // Copies rows [0, n) of layer l's K or V of a cache to the host as floats (tests).
  Expected<std::vector<float>> read_cache(const KVCache& cache, std::size_t layer, bool values, std::size_t n);
  // Writes positions [pos, pos + n) of every layer's K and V from host rows laid out
  // [n_layer][2][n][n_head_kv * head_dim] (K then V per layer) and advances the cache, as if
  // those positions had been prefilled; an fp16 cache takes each float rounded to nearest even
  // once, as its own writes do (kv_cache.h:34-43). For restoring a saved context, and for tests
  // that start the device and a reference from the same cache contents.
  Expected<bool> fill_cache(KVCache& cache, const float* rows, std::size_t n);

  // Kernel-time probe: while enabled, every matmul launch on weights of `type` (one ggml type
  // id) is bracketed by HIP events on the library stream. read_probe sums the bracketed device
  // time, the launches and their algorithmic bytes (weights + Q8_0 or float input + output,
  // the output counted twice when the launch accumulates into it).
  Expected<bool> set_probe(int type, bool enable);
  struct ProbeTotals {
    double ms = 0;
    std::size_t launches = 0;
    double bytes = 0;
  };
  Expected<ProbeTotals> read_probe();

  const Config& config() const { return cfg_; }
  const kernels::KernelTable& table() const { return *kernels_; }
  std::size_t weight_bytes_per_token() const { return weight_bytes_; }
  std::size_t device_bytes() const { return device_bytes_; }
  std::size_t max_ctx() const { return max_ctx_; }
  std::size_t max_seq() const { return max_seq_; }
  std::size_t max_batch() const { return max_batch_; }
  CacheType cache_type() const { return cache_type_; }
  // Whether one-row cached passes run as the persistent kernel, and if not, why.
  bool persistent_decode() const { return step_ok_; }
  // Turns the persistent kernel for one-row passes on or off (on: Unsupported when the model's
  // shape does not allow it). A pass whose kernel gave up turns it off (check_persistent_status).
  Expected<bool> set_persistent_decode(bool on);
  const std::string& persistent_decode_reason() const { return step_reason_; }
  std::size_t kv_element_bytes() const { return cache_type_ == CacheType::F16 ? 2 : 4; }

private:
  LlamaModel() = default;
  struct Row {
    std::int32_t token;
    std::int32_t pos;
    int slot;
  };
  // Runs every row through the layers; the final norm and the output matmul run on rows
  // [first_logit, rows.size()) only, whose logits are the pass's.
  Expected<std::size_t> run(std::span<const Row> rows, bool copy_logits, std::size_t first_logit = 0);
  // The row builders check their arguments as llama.cpp:269-302, 322-351 do and write rows_
  // from index `at`, returning the row count (rows_ holds max_rows entries from load on).
  Expected<std::size_t> mixed_rows(KVCache* prefill, std::span<const std::int32_t> chunk,
                                   std::span<KVCache* const> caches, std::span<const std::int32_t> tokens);
  Expected<std::span<const float>> forward_rows(std::span<const std::int32_t> tokens, bool copy_logits);
  Expected<std::size_t> prefill_rows(const KVCache& cache, std::span<const std::int32_t> tokens, std::size_t at);
  Expected<std::size_t> batch_rows(std::span<KVCache* const> caches, std::span<const std::int32_t> tokens,
                                   std::size_t at);
  std::vector<Row> rows_;
  Error device_error(const char* what) const;
  int mm(const Tensor& w, const float* x, const void* xq, float* y, std::size_t n, bool accumulate);
  double step_bytes(std::size_t n_vis) const;
  bool q8_path(const Tensor& w) const;
  // The repetition penalty of one (penalty, window) setting on the rows with select[r] set (all
  // rows when select is empty), on the device (sampler.cpp:73-97). `reuse`: another call follows,
  // so wait until the staging has been copied.
  Expected<bool> penalize(std::size_t n, std::span<const std::span<const std::int32_t>> recent, float penalty,
                          int repeat_last_n, std::span<const std::uint8_t> select, bool reuse = false);

  std::unique_ptr<GgufFile> file_;
  Config cfg_;
  const kernels::KernelTable* kernels_ = nullptr;
  std::vector<Layer> layers_;
  Tensor token_embd_, output_norm_, output_, rope_freqs_;
  bool have_rope_freqs_ = false;
  std::size_t max_seq_ = 0, max_ctx_ = 0, max_batch_ = 0, max_rows_ = 0, n_slots_ = 0;
  bool exact_ = false;
  CacheType cache_type_ = CacheType::F32;
  std::size_t weight_bytes_ = 0, device_bytes_ = 0;

  // Device memory.
  void* weights_ = nullptr;
  void* planar_ = nullptr;  // the repacked Q6_K output matrix
  float* rope_table_ = nullptr;
  void* kv_ = nullptr;        // n_slots_ cache slots of slot_elems_ elements (float or fp16)
  float* kv_free_ = nullptr;  // the cache-free forward's keys and values: float, max_seq positions
  std::size_t slot_elems_ = 0;
  float *x_ = nullptr, *h_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *attn_ = nullptr;
  float *gate_ = nullptr, *up_ = nullptr, *tmp_ = nullptr, *logits_ = nullptr, *scores_ = nullptr;
  void* xq_ = nullptr;
  void* rowinfo_ = nullptr;      // device: ids[R] | pos[R] | n_vis[R] | (8-aligned) cache_off[R]
  void* rowinfo_host_ = nullptr; // pinned staging of the same
  std::size_t scores_floats_ = 0;
  std::uint64_t* argmax_scratch_ = nullptr;
  std::size_t argmax_words_ = 0;  // its length in 8-byte keys
  std::int32_t* ids_ = nullptr;
  std::int32_t* gen_ids_ = nullptr;  // generate_greedy's ids: [max_ctx + 1]
  void* cand_ = nullptr;  // top-k candidates: [rows][k] logits, then [rows][k] ids
  // Every candidate of each row when a row keeps more than AXON_HIP_MAX_TOPK of them (top_k 0):
  // [rows][n_vocab] sorted logits then ids, and the sort's workspace. Allocated by the first
  // such sample call for its row count, and again only for a call with more rows.
  void* sort_out_ = nullptr;
  void* sort_work_ = nullptr;
  std::size_t sort_rows_ = 0;
  std::vector<std::byte> cand_host_;
  std::vector<double> probs_;
  void* window_ = nullptr;       // device: recent ids [R][kMaxPenaltyWindow] | lengths [R]
  void* window_host_ = nullptr;  // pinned staging of the same
  std::size_t last_rows_ = 0;  // rows of the last pass's logits, 0 after a failed pass
  std::vector<float> logits_host_;
  std::vector<std::uint8_t> sample_done_, sample_select_;
  // Probe state (set_probe / read_probe).
  int probe_type_ = -1;
  static constexpr int kProbeAttention = -2;  // AXON_MODEL_PROBE_ATTENTION (axon_model.h)
  static constexpr int kProbeStep = -3;       // AXON_MODEL_PROBE_STEP (axon_model.h)
  std::vector<void*> probe_events_;
  std::size_t probe_used_ = 0;
  std::vector<double> probe_bytes_;
  void probe_begin(const Tensor& w);
  // out_bytes_override >= 0 replaces the float output bytes (a launch that writes Q8_0 blocks).
  void probe_end(const Tensor& w, std::size_t n_rows, std::size_t n_out_total, bool accumulate,
                 double out_bytes_override = -1.0);
  void probe_cancel();
  std::vector<bool> slot_used_;
  std::vector<KVCache*> slot_cache_;  // the cache object of each used slot (new_cache to release_cache)
  // The persistent decode kernel (axon_hip_decode_layers): its shape, the device array of layer
  // records, its workspace and phase count, and the status word in pinned host memory.
  Expected<bool> setup_persistent_decode();
  Expected<bool> check_persistent_status();
  Expected<bool> step_reserve(std::size_t passes);
  bool step_ok_ = false;
  // The cache of the last persistent pass not yet checked, and the position it started at.
  KVCache* step_pending_ = nullptr;
  std::size_t step_pending_pos_ = 0;
  std::string step_reason_;
  axon_hip_decode_shape step_shape_{};
  void* step_layers_ = nullptr;
  void* step_work_ = nullptr;
  std::size_t step_work_bytes_ = 0;
  std::uint64_t step_epoch_ = 0;
  std::uint32_t* step_status_ = nullptr;
};

}  // namespace axon::model
