#include "model.h"

#include "axon_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>

namespace axon::model {

namespace {

std::string fmt_shape(std::uint64_t a, std::uint64_t b) { return std::to_string(a) + "x" + std::to_string(b); }

// An fp16 bit pattern widened to float, exactly (subnormals are m * 2^-24).
float half_to_float(std::uint16_t h) {
  const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
  const std::uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  std::uint32_t bits;
  if (e == 0x1fu) {
    bits = sign | 0x7f800000u | (m << 13);
  } else if (e != 0) {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  } else {
    const float f = std::ldexp(static_cast<float>(m), -24);
    std::memcpy(&bits, &f, 4);
    bits |= sign;
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// float to fp16 bits, rounding to nearest even; overflow to infinity, NaN stays NaN (the
// payload's top ten bits, at least 1), as src/core/dtype.cpp fp32_to_fp16 specifies.
std::uint16_t float_to_half(float f) {
  std::uint32_t b;
  std::memcpy(&b, &f, 4);
  const auto sign = static_cast<std::uint16_t>((b >> 16) & 0x8000u);
  const std::uint32_t a = b & 0x7fffffffu;
  if (a >= 0x7f800000u) {
    const std::uint32_t payload = (a >> 13) & 0x3ffu;
    return static_cast<std::uint16_t>(sign | 0x7c00u | (a == 0x7f800000u ? 0u : (payload != 0 ? payload : 1u)));
  }
  if (a >= 0x477ff000u) return static_cast<std::uint16_t>(sign | 0x7c00u);  // at or past 65520: infinity
  if (a >= 0x38800000u) {  // a normal half: rebias the exponent, round the 13 dropped bits
    std::uint32_t m = a - 0x38000000u;
    m += 0xfffu + ((m >> 13) & 1u);
    return static_cast<std::uint16_t>(sign | (m >> 13));
  }
  // A subnormal half (or zero): the value in units of 2^-24, rounded to nearest even (scaling by
  // a power of two is exact).
  float mag;
  std::memcpy(&mag, &a, 4);
  return static_cast<std::uint16_t>(sign | static_cast<std::uint16_t>(std::nearbyint(mag * 16777216.0f)));
}

bool matmul_type(DType t) {
  switch (t) {
  case DType::F32: case DType::F16: case DType::BF16: case DType::Q8_0: case DType::Q4_0: case DType::Q4_1:
  case DType::Q6_K:
    return true;
  }
  return false;
}

enum class Kind { Matmul, Norm };

// Binds one tensor with the exact shape and dtype checks of src/model/weights.cpp:15-67.
Expected<Tensor> bind_tensor(const GgufFile& f, const std::string& name, Kind kind, std::uint64_t ne0, std::uint64_t ne1) {
  const GgufTensor* t = f.tensor(name);
  if (t == nullptr) return make_error(ErrorCode::InvalidArgument, name + ": missing");
  const std::uint64_t got1 = t->n_dims > 1 ? t->ne[1] : 1;
  if (t->ne[0] != ne0 || got1 != ne1 || t->ne[2] != 1 || t->ne[3] != 1)
    return make_error(ErrorCode::InvalidArgument,
                      name + ": expected shape " + fmt_shape(ne0, ne1) + ", found " + fmt_shape(t->ne[0], got1));
  if (kind == Kind::Norm && t->type != DType::F32)
    return make_error(ErrorCode::Unsupported, name + ": expected F32, found type " + std::to_string(int(t->type)));
  if (kind == Kind::Matmul && !matmul_type(t->type))
    return make_error(ErrorCode::Unsupported, name + ": unsupported matmul type " + std::to_string(int(t->type)));
  const std::size_t row = row_bytes_of(t->type, ne0);
  if (row == 0)
    return make_error(ErrorCode::InvalidArgument, name + ": row length " + std::to_string(ne0) + " is not a whole number of blocks");
  Tensor out;
  out.type = t->type;
  out.ne0 = ne0;
  out.ne1 = ne1;
  out.row_bytes = row;
  out.total_bytes = row * ne1;
  out.host = t->data;
  return out;
}

// The model's shape from the file's metadata. The keys, their defaults and the detection of
// tied embeddings, Q/K/V bias and llama3 rope factors are the GGUF contract the reference reads
// (src/model/config.cpp:27-123); the validation is this library's.
Expected<Config> config_of(const GgufFile& f) {
  Config c;
  c.arch = f.string_or("general.architecture", "");
  if (c.arch != "llama" && c.arch != "qwen2")
    return make_error(ErrorCode::Unsupported, "model architecture '" + c.arch + "' is not supported (llama, qwen2)");
  c.rope_style = c.arch == "qwen2" ? kernels::RopeStyle::NeoX : kernels::RopeStyle::Normal;
  const std::string ns = c.arch + ".";

  // Required extents first, then the ones that default to a value derived from them.
  struct Extent {
    const char* name;
    std::uint32_t* field;
  };
  for (const Extent& e : {Extent{"block_count", &c.n_layer}, Extent{"embedding_length", &c.n_embd},
                          Extent{"attention.head_count", &c.n_head}, Extent{"feed_forward_length", &c.n_ff},
                          Extent{"context_length", &c.n_ctx_train}}) {
    const GgufValue* v = f.meta(ns + e.name);
    if (v == nullptr || v->kind != GgufValue::Kind::UInt || v->u > 0xffffffffull)
      return make_error(ErrorCode::InvalidArgument, ns + e.name + " is absent or not an unsigned 32-bit value");
    *e.field = static_cast<std::uint32_t>(v->u);
  }
  if (c.n_layer * std::uint64_t{c.n_embd} * c.n_head * c.n_ff == 0)
    return make_error(ErrorCode::InvalidArgument,
                      "model shape has an empty extent: " + std::to_string(c.n_layer) + " layers, width " +
                          std::to_string(c.n_embd) + ", " + std::to_string(c.n_head) + " heads, feed-forward " +
                          std::to_string(c.n_ff));
  c.n_head_kv = static_cast<std::uint32_t>(f.uint_or(ns + "attention.head_count_kv", c.n_head));
  c.head_dim = static_cast<std::uint32_t>(f.uint_or(ns + "attention.key_length", c.n_embd / c.n_head));
  c.rotary_dim = static_cast<std::uint32_t>(f.uint_or(ns + "rope.dimension_count", c.head_dim));
  c.rope_theta = static_cast<float>(f.float_or(ns + "rope.freq_base", 10000.0));
  c.rms_eps = static_cast<float>(f.float_or(ns + "attention.layer_norm_rms_epsilon", 1e-5));
  if (c.n_head_kv == 0 || c.n_head % c.n_head_kv != 0)
    return make_error(ErrorCode::InvalidArgument, std::to_string(c.n_head_kv) + " key/value heads cannot serve " +
                                                      std::to_string(c.n_head) + " query heads in equal groups");
  if (c.head_dim == 0 || c.head_dim % 2 != 0)
    return make_error(ErrorCode::InvalidArgument, "head size " + std::to_string(c.head_dim) + " is not a positive even number");
  if (c.rotary_dim == 0 || c.rotary_dim % 2 != 0 || c.rotary_dim > c.head_dim)
    return make_error(ErrorCode::InvalidArgument, "rotary width " + std::to_string(c.rotary_dim) +
                                                      " must be positive, even and within the head size " +
                                                      std::to_string(c.head_dim));

  // The vocabulary is the embedding's row count; the declared sizes must agree with it.
  const GgufTensor* embd = f.tensor("token_embd.weight");
  if (embd == nullptr) return make_error(ErrorCode::InvalidArgument, "the token embedding (token_embd.weight) is absent");
  if (embd->n_dims != 2 || embd->ne[0] != c.n_embd)
    return make_error(ErrorCode::InvalidArgument, "token_embd.weight rows are " + std::to_string(embd->ne[0]) +
                                                      " wide, not the model width " + std::to_string(c.n_embd));
  c.n_vocab = static_cast<std::uint32_t>(embd->ne[1]);
  const std::string vocab_rows = std::to_string(c.n_vocab) + " embedding rows";
  if (const GgufValue* vs = f.meta(ns + "vocab_size"); vs != nullptr && vs->u != c.n_vocab)
    return make_error(ErrorCode::InvalidArgument, ns + "vocab_size says " + std::to_string(vs->u) + " for " + vocab_rows);
  if (const GgufValue* toks = f.meta("tokenizer.ggml.tokens"); toks != nullptr && toks->array_size != c.n_vocab)
    return make_error(ErrorCode::InvalidArgument,
                      "the tokenizer lists " + std::to_string(toks->array_size) + " tokens for " + vocab_rows);
  c.tie_embeddings = f.tensor("output.weight") == nullptr;
  c.attn_bias = f.tensor("blk.0.attn_q.bias") != nullptr;
  c.llama3 = f.tensor("rope_freqs.weight") != nullptr;
  return c;
}

std::size_t align_up(std::size_t v, std::size_t a) { return (v + a - 1) / a * a; }

}  // namespace

bool KVCache::truncate(std::size_t pos) {
  if (pos > pos_) return false;
  pos_ = pos;
  return true;
}

Error LlamaModel::device_error(const char* what) const {
  return make_error(ErrorCode::Device, std::string(what) + ": " + axon_hip_last_error());
}

Expected<std::unique_ptr<LlamaModel>> LlamaModel::load(const std::string& path, LoadOptions options) {
  if (options.max_seq == 0) return make_error(ErrorCode::InvalidArgument, "max_seq: expected at least 1, found 0");
  if (options.max_ctx < options.max_seq)
    return make_error(ErrorCode::InvalidArgument, "max_ctx is smaller than max_seq");
  auto file = GgufFile::open(path);
  if (!file) return file.error();
  auto cfg = config_of(*file);
  if (!cfg) return make_error(cfg.error().code, path + ": " + cfg.error().message);
  auto table = kernels::select(options.kernels);
  if (!table) return table.error();

  std::unique_ptr<LlamaModel> m(new LlamaModel());
  m->cfg_ = *cfg;
  m->kernels_ = *table;
  const Config& c = m->cfg_;
  // As llama.cpp:203-208: a cache longer than the training context is clamped, not refused.
  m->max_ctx_ = std::min<std::size_t>(options.max_ctx, c.n_ctx_train);
  m->max_seq_ = std::min(options.max_seq, m->max_ctx_);
  m->max_batch_ = std::max<std::size_t>(1, options.max_batch);
  // A mixed pass carries a prompt chunk and a decode batch.
  m->max_rows_ = m->max_seq_ + m->max_batch_;
  m->n_slots_ = options.max_caches != 0 ? options.max_caches : m->max_batch_ + 1;
  m->exact_ = options.exact_activations;
  m->cache_type_ = options.cache;

  // Bind (weights.cpp:71-127).
  const std::uint64_t d = c.n_embd, dq = c.n_embd_q(), dkv = c.n_embd_kv(), ff = c.n_ff;
#define BIND(target, name, kind, a, b)                                                            \
  do {                                                                                             \
    auto bound = bind_tensor(*file, name, kind, a, b);                                                    \
    if (!bound) return make_error(bound.error().code, path + ": " + bound.error().message);        \
    (target) = *bound;                                                                             \
  } while (0)
  BIND(m->token_embd_, "token_embd.weight", Kind::Matmul, d, c.n_vocab);
  BIND(m->output_norm_, "output_norm.weight", Kind::Norm, d, 1);
  if (c.tie_embeddings) {
    m->output_ = m->token_embd_;
  } else {
    BIND(m->output_, "output.weight", Kind::Matmul, d, c.n_vocab);
  }
  if (c.llama3) {
    BIND(m->rope_freqs_, "rope_freqs.weight", Kind::Norm, c.rotary_dim / 2, 1);
    m->have_rope_freqs_ = true;
  }
  m->layers_.resize(c.n_layer);
  for (std::uint32_t i = 0; i < c.n_layer; ++i) {
    Layer& L = m->layers_[i];
    const std::string p = "blk." + std::to_string(i) + ".";
    BIND(L.attn_norm, p + "attn_norm.weight", Kind::Norm, d, 1);
    BIND(L.wq, p + "attn_q.weight", Kind::Matmul, d, dq);
    BIND(L.wk, p + "attn_k.weight", Kind::Matmul, d, dkv);
    BIND(L.wv, p + "attn_v.weight", Kind::Matmul, d, dkv);
    BIND(L.wo, p + "attn_output.weight", Kind::Matmul, dq, d);
    BIND(L.ffn_norm, p + "ffn_norm.weight", Kind::Norm, d, 1);
    BIND(L.w_gate, p + "ffn_gate.weight", Kind::Matmul, d, ff);
    BIND(L.w_up, p + "ffn_up.weight", Kind::Matmul, d, ff);
    BIND(L.w_down, p + "ffn_down.weight", Kind::Matmul, ff, d);
    if (c.attn_bias) {
      BIND(L.bq, p + "attn_q.bias", Kind::Norm, dq, 1);
      BIND(L.bk, p + "attn_k.bias", Kind::Norm, dkv, 1);
      BIND(L.bv, p + "attn_v.bias", Kind::Norm, dkv, 1);
      L.bias = true;
    }
  }
#undef BIND

  // Bytes one token reads (llama.cpp:151-167): one embedding row, the output norm and matrix,
  // the rope factors, and every layer tensor.
  std::size_t wb = m->token_embd_.row_bytes + m->output_norm_.total_bytes + m->output_.total_bytes;
  if (m->have_rope_freqs_) wb += m->rope_freqs_.total_bytes;
  for (const Layer& L : m->layers_) {
    wb += L.attn_norm.total_bytes + L.wq.total_bytes + L.wk.total_bytes + L.wv.total_bytes + L.wo.total_bytes +
          L.ffn_norm.total_bytes + L.w_gate.total_bytes + L.w_up.total_bytes + L.w_down.total_bytes;
    if (L.bias) wb += L.bq.total_bytes + L.bk.total_bytes + L.bv.total_bytes;
  }
  m->weight_bytes_ = wb;

  // Upload every bound tensor into one HBM allocation, each at a 256-byte boundary.
  std::vector<Tensor*> all = {&m->token_embd_, &m->output_norm_};
  if (!c.tie_embeddings) all.push_back(&m->output_);
  if (m->have_rope_freqs_) all.push_back(&m->rope_freqs_);
  for (Layer& L : m->layers_) {
    for (Tensor* t : {&L.attn_norm, &L.wq, &L.wk, &L.wv, &L.wo, &L.ffn_norm, &L.w_gate, &L.w_up, &L.w_down})
      all.push_back(t);
    if (L.bias) {
      all.push_back(&L.bq);
      all.push_back(&L.bk);
      all.push_back(&L.bv);
    }
  }
  std::size_t total = 0;
  std::vector<std::size_t> offs;
  for (Tensor* t : all) {
    offs.push_back(total);
    total = align_up(total + t->total_bytes, 256);
  }
  if (axon_hip_malloc(&m->weights_, total) != AXON_HIP_OK) return m->device_error("weights");
  for (std::size_t i = 0; i < all.size(); ++i) {
    all[i]->dev = static_cast<std::byte*>(m->weights_) + offs[i];
    if (axon_hip_memcpy_h2d(all[i]->dev, all[i]->host, all[i]->total_bytes) != AXON_HIP_OK)
      return m->device_error("weight upload");
  }
  if (c.tie_embeddings) m->output_ = m->token_embd_;
  m->device_bytes_ = total;
  // The one-time repack of the Q6_K output matrix (the f2 row of the build plan): planes of
  // aligned 16-byte slices, checked against the native blocks by dequantization in the tests.
  if (options.repack && m->output_.type == DType::Q6_K) {
    const std::size_t pb = axon_hip_q6k_planar_bytes(m->output_.ne1, m->output_.ne0);
    if (pb != 0) {
      if (axon_hip_malloc(&m->planar_, pb) != AXON_HIP_OK ||
          axon_hip_q6k_repack(m->output_.dev, m->output_.ne1, m->output_.ne0, m->planar_) != AXON_HIP_OK ||
          axon_hip_synchronize() != AXON_HIP_OK)
        return m->device_error("Q6_K repack");
      m->output_.planar = m->planar_;
      m->device_bytes_ += pb;
    }
  }

  // cos/sin table [pos][rotary_dim/2], evaluated in double with the host libm exactly as
  // src/kernels/ref/rope.cpp:19-26 does, then rounded to float.
  {
    const std::size_t half = c.rotary_dim / 2;
    std::vector<float> tab(m->max_ctx_ * half * 2);
    const auto theta = static_cast<double>(c.rope_theta);
    const auto rot = static_cast<double>(c.rotary_dim);
    const float* factors = m->have_rope_freqs_ ? reinterpret_cast<const float*>(m->rope_freqs_.host) : nullptr;
    for (std::size_t i = 0; i < half; ++i) {
      double inv_freq = std::pow(theta, -static_cast<double>(2 * i) / rot);
      if (factors != nullptr) inv_freq /= static_cast<double>(factors[i]);
      for (std::size_t pos = 0; pos < m->max_ctx_; ++pos) {
        const double angle = static_cast<double>(pos) * inv_freq;
        tab[(pos * half + i) * 2] = static_cast<float>(std::cos(angle));
        tab[(pos * half + i) * 2 + 1] = static_cast<float>(std::sin(angle));
      }
    }
    if (axon_hip_malloc(reinterpret_cast<void**>(&m->rope_table_), tab.size() * 4) != AXON_HIP_OK ||
        axon_hip_memcpy_h2d(m->rope_table_, tab.data(), tab.size() * 4) != AXON_HIP_OK)
      return m->device_error("rope table");
    m->device_bytes_ += tab.size() * 4;
  }

  // Activations for max_rows rows (activations.h:18-55), the KV pool, row metadata.
  const std::size_t R = m->max_rows_;
  const std::size_t widest = std::max({d, dq, ff});
  struct Buf {
    float** p;
    std::size_t floats;
  };
  const Buf bufs[] = {{&m->x_, R * d},       {&m->h_, R * d},   {&m->q_, R * dq},     {&m->k_, R * dkv},
                      {&m->v_, R * dkv},     {&m->attn_, R * dq}, {&m->gate_, R * ff}, {&m->up_, R * ff},
                      {&m->tmp_, R * widest}, {&m->logits_, R * c.n_vocab}};
  for (const Buf& b : bufs) {
    if (axon_hip_malloc(reinterpret_cast<void**>(b.p), b.floats * 4) != AXON_HIP_OK) return m->device_error("activations");
    m->device_bytes_ += b.floats * 4;
  }
  if (axon_hip_malloc(&m->xq_, R * (widest / 32) * sizeof(BlockQ8_0) + 64) != AXON_HIP_OK)
    return m->device_error("activation blocks");
  const std::size_t info_bytes = align_up(12 * R, 8) + 8 * R;
  // The greedy keys: argmax_rows' partials for R rows, or one key per workgroup of the planar
  // Q6_K output (generate_greedy), whichever is more.
  m->argmax_words_ = std::max(axon_hip_argmax_scratch_words(R), axon_hip_q6k_argmax_parts(c.n_vocab));
  if (axon_hip_malloc(reinterpret_cast<void**>(&m->argmax_scratch_), m->argmax_words_ * 8) != AXON_HIP_OK ||
      axon_hip_malloc(reinterpret_cast<void**>(&m->ids_), R * 4) != AXON_HIP_OK ||
      axon_hip_malloc(reinterpret_cast<void**>(&m->gen_ids_), (m->max_ctx_ + 1) * 4) != AXON_HIP_OK ||
      axon_hip_malloc(&m->cand_, R * AXON_HIP_MAX_TOPK * 8) != AXON_HIP_OK)
    return m->device_error("sampling scratch");
  const std::size_t window_bytes = R * (kMaxPenaltyWindow + 1) * 4;
  if (axon_hip_malloc(&m->window_, window_bytes) != AXON_HIP_OK ||
      axon_hip_host_malloc(&m->window_host_, window_bytes) != AXON_HIP_OK)
    return m->device_error("penalty windows");
  if (axon_hip_malloc(&m->rowinfo_, info_bytes) != AXON_HIP_OK ||
      axon_hip_host_malloc(&m->rowinfo_host_, info_bytes) != AXON_HIP_OK)
    return m->device_error("row table");
  m->slot_elems_ = static_cast<std::size_t>(c.n_layer) * 2 * m->max_ctx_ * dkv;
  const std::size_t pool = m->n_slots_ * m->slot_elems_ * m->kv_element_bytes();
  if (axon_hip_malloc(&m->kv_, pool) != AXON_HIP_OK) return m->device_error("kv pool");
  // The cache-free forward (llama.cpp:379-383) keeps its keys and values in float whatever
  // the cache type, laid out as a slot of max_seq positions.
  const std::size_t free_bytes = static_cast<std::size_t>(c.n_layer) * 2 * m->max_seq_ * dkv * 4;
  if (axon_hip_malloc(reinterpret_cast<void**>(&m->kv_free_), free_bytes) != AXON_HIP_OK)
    return m->device_error("kv (cache-free pass)");
  m->device_bytes_ += pool + free_bytes;
  axon_hip_attention_rows_args probe{};
  probe.n_head = c.n_head;
  probe.n_kv = c.n_head_kv;
  probe.head_dim = c.head_dim;
  probe.max_vis = static_cast<std::uint32_t>(m->max_ctx_);
  m->scores_floats_ = 0;
  for (std::size_t rows = 1; rows <= R; ++rows)
    m->scores_floats_ = std::max(m->scores_floats_, axon_hip_attention_scratch_floats(&probe, rows));
  if (m->scores_floats_ != 0 &&
      axon_hip_malloc(reinterpret_cast<void**>(&m->scores_), m->scores_floats_ * 4) != AXON_HIP_OK)
    return m->device_error("attention scratch");
  m->slot_used_.assign(m->n_slots_, false);
  m->slot_cache_.assign(m->n_slots_, nullptr);
  if (options.persistent_decode) {
    auto st = m->setup_persistent_decode();
    if (!st) return st.error();
  } else {
    m->step_reason_ = "turned off by LoadOptions::persistent_decode";
  }
  // Host staging that every pass reuses: the row list, the logits of max_rows rows, and the
  // sampler's per-row flags, so that a pass allocates no host memory.
  m->rows_.resize(R);
  m->logits_host_.reserve(R * c.n_vocab);
  m->sample_done_.reserve(R);
  m->sample_select_.reserve(R);
  m->cand_host_.reserve(R * AXON_HIP_MAX_TOPK * 8);
  m->probs_.reserve(AXON_HIP_MAX_TOPK);
  m->file_ = std::make_unique<GgufFile>(std::move(*file));
  return m;
}

LlamaModel::~LlamaModel() {
  axon_hip_synchronize();
  for (void* p : {static_cast<void*>(x_), static_cast<void*>(h_), static_cast<void*>(q_), static_cast<void*>(k_),
                  static_cast<void*>(v_), static_cast<void*>(attn_), static_cast<void*>(gate_),
                  static_cast<void*>(up_), static_cast<void*>(tmp_), static_cast<void*>(logits_),
                  static_cast<void*>(scores_), static_cast<void*>(argmax_scratch_), static_cast<void*>(ids_),
                  static_cast<void*>(gen_ids_), cand_, sort_out_, sort_work_, window_,
                  xq_, rowinfo_, kv_, static_cast<void*>(kv_free_),
                  static_cast<void*>(rope_table_), weights_, planar_}) {
    if (p != nullptr) axon_hip_free(p);
  }
  if (rowinfo_host_ != nullptr) axon_hip_host_free(rowinfo_host_);
  if (step_layers_ != nullptr) axon_hip_free(step_layers_);
  if (step_work_ != nullptr) axon_hip_free(step_work_);
  if (step_status_ != nullptr) axon_hip_host_free(step_status_);
  if (window_host_ != nullptr) axon_hip_host_free(window_host_);
  for (void* e : probe_events_) axon_hip_event_destroy(e);
}

Expected<bool> LlamaModel::set_probe(int type, bool enable) {
  if (!enable) {
    probe_type_ = -1;
    return true;
  }
  if (probe_events_.empty()) {
    probe_events_.resize(2 * 8192, nullptr);
    for (void*& e : probe_events_) {
      if (axon_hip_event_create(&e) != AXON_HIP_OK) return device_error("probe events");
    }
  }
  probe_type_ = type;
  probe_used_ = 0;
  probe_bytes_.clear();
  return true;
}

void LlamaModel::probe_begin(const Tensor& w) {
  if (static_cast<int>(w.type) != probe_type_ || 2 * probe_used_ + 2 > probe_events_.size()) return;
  axon_hip_probe_next_launch(probe_events_[2 * probe_used_], probe_events_[2 * probe_used_ + 1]);
}

void LlamaModel::probe_cancel() { axon_hip_probe_next_launch(nullptr, nullptr); }

void LlamaModel::probe_end(const Tensor& w, std::size_t n_rows, std::size_t n_out_total, bool accumulate,
                           double out_bytes_override) {
  if (static_cast<int>(w.type) != probe_type_ || 2 * probe_used_ + 2 > probe_events_.size()) return;
  axon_hip_probe_next_launch(nullptr, nullptr);
  const double in_bytes = q8_path(w) ? static_cast<double>(n_rows) * (w.ne0 / 32) * sizeof(BlockQ8_0)
                                     : static_cast<double>(n_rows) * w.ne0 * 4.0;
  const double out_bytes = out_bytes_override >= 0
                               ? out_bytes_override
                               : static_cast<double>(n_rows) * n_out_total * 4.0 * (accumulate ? 2 : 1);
  probe_bytes_.push_back(static_cast<double>(w.row_bytes) * n_out_total + in_bytes + out_bytes);
  ++probe_used_;
}

Expected<LlamaModel::ProbeTotals> LlamaModel::read_probe() {
  ProbeTotals t;
  if (axon_hip_synchronize() != AXON_HIP_OK) return device_error("synchronize");
  for (std::size_t i = 0; i < probe_used_; ++i) {
    float ms = 0;
    if (axon_hip_event_elapsed_ms(probe_events_[2 * i], probe_events_[2 * i + 1], &ms) != AXON_HIP_OK)
      return device_error("probe elapsed");
    t.ms += ms;
    t.bytes += probe_bytes_[i];
  }
  t.launches = probe_used_;
  probe_used_ = 0;
  probe_bytes_.clear();
  return t;
}

Expected<std::unique_ptr<KVCache>> LlamaModel::new_cache() {
  for (std::size_t s = 0; s < n_slots_; ++s) {
    if (!slot_used_[s]) {
      slot_used_[s] = true;
      auto cache = std::make_unique<KVCache>(static_cast<int>(s), max_ctx_);
      slot_cache_[s] = cache.get();
      return cache;
    }
  }
  return make_error(ErrorCode::OutOfRange, "new_cache: all " + std::to_string(n_slots_) + " device KV slots are in use");
}

void LlamaModel::release_cache(const KVCache& cache) {
  if (cache.slot() >= 0 && static_cast<std::size_t>(cache.slot()) < n_slots_) {
    slot_used_[cache.slot()] = false;
    slot_cache_[cache.slot()] = nullptr;
  }
  if (step_pending_ == &cache) step_pending_ = nullptr;
}

Expected<std::vector<float>> LlamaModel::read_cache(const KVCache& cache, std::size_t layer, bool values, std::size_t n) {
  if (layer >= cfg_.n_layer || n > max_ctx_) return make_error(ErrorCode::InvalidArgument, "read_cache: out of range");
  const std::size_t dkv = cfg_.n_embd_kv();
  std::vector<float> out(n * dkv);
  const std::size_t at = cache.slot() * slot_elems_ + (2 * layer + (values ? 1 : 0)) * max_ctx_ * dkv;
  if (cache_type_ == CacheType::F32) {
    if (axon_hip_memcpy_d2h(out.data(), static_cast<const float*>(kv_) + at, out.size() * 4) != AXON_HIP_OK)
      return device_error("read_cache");
    return out;
  }
  std::vector<std::uint16_t> bits(n * dkv);
  if (axon_hip_memcpy_d2h(bits.data(), static_cast<const std::uint16_t*>(kv_) + at, bits.size() * 2) != AXON_HIP_OK)
    return device_error("read_cache");
  for (std::size_t i = 0; i < bits.size(); ++i) out[i] = half_to_float(bits[i]);
  return out;
}

Expected<bool> LlamaModel::fill_cache(KVCache& cache, const float* rows, std::size_t n) {
  if (cache.slot() < 0 || static_cast<std::size_t>(cache.slot()) >= n_slots_)
    return make_error(ErrorCode::InvalidArgument, "fill_cache: the cache was built for a different model");
  if (cache.pos() + n > max_ctx_)
    return make_error(ErrorCode::InvalidArgument, "context overflow: " + std::to_string(cache.pos()) + " cached + " +
                                                      std::to_string(n) + " filled positions exceed " +
                                                      std::to_string(max_ctx_));
  if (n == 0) return true;
  if (rows == nullptr) return make_error(ErrorCode::InvalidArgument, "fill_cache: no rows");
  const std::size_t dkv = cfg_.n_embd_kv();
  const std::size_t span = n * dkv;
  std::vector<std::uint16_t> half(cache_type_ == CacheType::F16 ? span : 0);
  for (std::size_t l = 0; l < cfg_.n_layer; ++l) {
    for (std::size_t kv = 0; kv < 2; ++kv) {
      const float* src = rows + (2 * l + kv) * span;
      const std::size_t at = cache.slot() * slot_elems_ + (2 * l + kv) * max_ctx_ * dkv + cache.pos() * dkv;
      int rc;
      if (cache_type_ == CacheType::F32) {
        rc = axon_hip_memcpy_h2d(static_cast<float*>(kv_) + at, src, span * 4);
      } else {
        for (std::size_t i = 0; i < span; ++i) half[i] = float_to_half(src[i]);
        rc = axon_hip_memcpy_h2d(static_cast<std::uint16_t*>(kv_) + at, half.data(), span * 2);
      }
      if (rc != AXON_HIP_OK) return device_error("fill_cache");
    }
  }
  cache.advance(n);
  return true;
}

Expected<bool> LlamaModel::setup_persistent_decode() {
  const Config& c = cfg_;
  auto reason = [&](const char* why) {
    step_reason_ = why;
    return true;
  };
  if (exact_) return reason("exact activations (float matmul inputs)");
  if (c.rope_style != kernels::RopeStyle::Normal) return reason("NeoX rotary layout");
  if (c.head_dim != 64) return reason("a head size other than 64");
  for (const Layer& L : layers_) {
    if (!q8_path(L.wq) || !q8_path(L.wo) || !q8_path(L.w_gate) || !q8_path(L.w_down))
      return reason("a layer matrix outside Q8_0 / Q4_0 / Q4_1");
    if (L.wq.type != L.wk.type || L.wk.type != L.wv.type || L.w_gate.type != L.w_up.type ||
        L.wq.type != layers_[0].wq.type || L.wo.type != layers_[0].wo.type || L.w_gate.type != layers_[0].w_gate.type ||
        L.w_down.type != layers_[0].w_down.type)
      return reason("matrix types that differ within a role or across layers");
  }
  axon_hip_decode_shape& sh = step_shape_;
  sh.n_layer = c.n_layer;
  sh.n_embd = c.n_embd;
  sh.n_head = c.n_head;
  sh.n_head_kv = c.n_head_kv;
  sh.n_ff = c.n_ff;
  sh.rotary_dim = c.rotary_dim;
  sh.type_qkv = static_cast<int>(layers_[0].wq.type);
  sh.type_o = static_cast<int>(layers_[0].wo.type);
  sh.type_gate_up = static_cast<int>(layers_[0].w_gate.type);
  sh.type_down = static_cast<int>(layers_[0].w_down.type);
  sh.max_ctx = static_cast<std::uint32_t>(max_ctx_);
  sh.cache_f16 = cache_type_ == CacheType::F16 ? 1 : 0;
  if (const char* why = axon_hip_decode_layers_unsupported(&sh); why != nullptr)
    return reason(why);
  const std::size_t dkv = c.n_embd_kv();
  std::vector<axon_hip_decode_layer> recs(c.n_layer);
  for (std::size_t l = 0; l < c.n_layer; ++l) {
    const Layer& L = layers_[l];
    axon_hip_decode_layer& r = recs[l];
    r.wq = L.wq.dev;
    r.wk = L.wk.dev;
    r.wv = L.wv.dev;
    r.wo = L.wo.dev;
    r.w_gate = L.w_gate.dev;
    r.w_up = L.w_up.dev;
    r.w_down = L.w_down.dev;
    r.attn_norm = static_cast<const float*>(L.attn_norm.dev);
    r.ffn_norm = static_cast<const float*>(L.ffn_norm.dev);
    if (L.bias) {
      r.bq = static_cast<const float*>(L.bq.dev);
      r.bk = static_cast<const float*>(L.bk.dev);
      r.bv = static_cast<const float*>(L.bv.dev);
    }
    r.k_layer_off = static_cast<std::int64_t>(2 * l) * static_cast<std::int64_t>(max_ctx_ * dkv);
    r.v_layer_off = r.k_layer_off + static_cast<std::int64_t>(max_ctx_ * dkv);
  }
  step_work_bytes_ = axon_hip_decode_layers_workspace_bytes(&sh);
  if (axon_hip_malloc(&step_layers_, recs.size() * sizeof(axon_hip_decode_layer)) != AXON_HIP_OK ||
      axon_hip_memcpy_h2d(step_layers_, recs.data(), recs.size() * sizeof(axon_hip_decode_layer)) != AXON_HIP_OK ||
      axon_hip_malloc(&step_work_, step_work_bytes_) != AXON_HIP_OK ||
      axon_hip_memset(step_work_, 0, step_work_bytes_) != AXON_HIP_OK ||
      axon_hip_host_malloc(reinterpret_cast<void**>(&step_status_), sizeof(std::uint32_t)) != AXON_HIP_OK)
    return device_error("persistent decode setup");
  *step_status_ = 0;
  step_epoch_ = 0;
  device_bytes_ += recs.size() * sizeof(axon_hip_decode_layer) + step_work_bytes_;
  step_ok_ = true;
  step_reason_.clear();
  return true;
}

// After a synchronization (every pass issued so far has ended): a persistent-kernel pass that
// gave up waiting for another workgroup's output voids that pass. Its cache goes back to the
// position the pass started at (a pass whose logits stayed in HBM has already advanced it, and
// the rows it wrote there are not the pass's results), the workspace is reset, and later one-row
// passes of this model run layer by layer: a grid that could not become resident once (a CU
// mask, another process holding CUs) is likely to fail again, and every such pass would cost a
// full poll limit. set_persistent_decode(true) turns the kernel back on. The error names the
// cache slot and the position.
Expected<bool> LlamaModel::check_persistent_status() {
  if (step_status_ == nullptr || *reinterpret_cast<volatile std::uint32_t*>(step_status_) == 0) {
    step_pending_ = nullptr;
    return true;
  }
  const std::uint32_t st = *step_status_;
  std::string where;
  if (step_pending_ != nullptr) {
    if (step_pending_->pos() > step_pending_pos_) step_pending_->truncate(step_pending_pos_);
    where = " at position " + std::to_string(step_pending_pos_) + " of the cache in slot " +
            std::to_string(step_pending_->slot()) + " (rolled back to that position)";
  }
  step_pending_ = nullptr;
  if (axon_hip_memset(step_work_, 0, step_work_bytes_) != AXON_HIP_OK) return device_error("persistent decode reset");
  step_epoch_ = 0;
  *step_status_ = 0;
  step_ok_ = false;
  step_reason_ = "the persistent kernel gave up waiting for another workgroup (status " + std::to_string(st) +
                 "); one-row passes run layer by layer";
  return make_error(ErrorCode::Device, "a one-row pass's persistent kernel gave up waiting for another workgroup (status " +
                                           std::to_string(st) + ")" + where +
                                           "; that pass's results are void, and later one-row passes run layer by layer");
}

// The phase tags of `passes` more persistent passes must not pass 2^32 (the kernel tags words
// with the low 32 bits of epoch + phase): before they would, at a synchronization, the
// workspace is zeroed and the epoch restarts (about 54 million steps of a 16-layer model).
Expected<bool> LlamaModel::step_reserve(std::size_t passes) {
  const std::uint64_t phases = 5ull * cfg_.n_layer * passes;
  if (step_epoch_ + phases <= 0xffffffffull) return true;
  if (axon_hip_synchronize() != AXON_HIP_OK) return device_error("synchronize");
  if (auto st = check_persistent_status(); !st) return st.error();
  if (axon_hip_memset(step_work_, 0, step_work_bytes_) != AXON_HIP_OK) return device_error("persistent decode reset");
  step_epoch_ = 0;
  if (phases > 0xffffffffull) return make_error(ErrorCode::InvalidArgument, "generate: too many steps in one call");
  return true;
}

Expected<bool> LlamaModel::set_persistent_decode(bool on) {
  if (axon_hip_synchronize() != AXON_HIP_OK) return device_error("synchronize");
  if (auto st = check_persistent_status(); !st) return st.error();
  if (!on) {
    step_ok_ = false;
    step_reason_ = "turned off by set_persistent_decode";
    return true;
  }
  if (step_ok_) return true;
  if (step_work_ == nullptr) {  // never set up (LoadOptions::persistent_decode was false)
    auto st = setup_persistent_decode();
    if (!st) return st.error();
    if (!step_ok_) return make_error(ErrorCode::Unsupported, "persistent decode: " + step_reason_);
    return true;
  }
  if (axon_hip_memset(step_work_, 0, step_work_bytes_) != AXON_HIP_OK) return device_error("persistent decode reset");
  step_epoch_ = 0;
  *step_status_ = 0;
  step_ok_ = true;
  step_reason_.clear();
  return true;
}

// Algorithmic HBM bytes of one persistent decode step over n_vis positions: every layer's
// weights and norm vectors, the K and V rows read (the new one included) and written, the
// activation row in and out.
double LlamaModel::step_bytes(std::size_t n_vis) const {
  const Config& c = cfg_;
  const double dkv = static_cast<double>(c.n_embd_kv()), d = static_cast<double>(c.n_embd);
  double b = 0;
  for (const Layer& L : layers_) {
    for (const Tensor* w : {&L.wq, &L.wk, &L.wv, &L.wo, &L.w_gate, &L.w_up, &L.w_down})
      b += static_cast<double>(w->row_bytes) * w->ne1;
    const double kv_elem = cache_type_ == CacheType::F16 ? 2 : 4;
    b += 2 * d * 4 + 2 * dkv * kv_elem * (static_cast<double>(n_vis) + 1);
  }
  return b + 2 * d * 4;
}

bool LlamaModel::q8_path(const Tensor& w) const {
  return !exact_ && (w.type == DType::Q8_0 || w.type == DType::Q4_0 || w.type == DType::Q4_1);
}

// Y = X W^T for one weight (matmul_columns, llama.cpp:30-101), whole matrix per launch;
// with accumulate, Y += X W^T (the residual add of llama.cpp:594-595, 621-623).
int LlamaModel::mm(const Tensor& w, const float* x, const void* xq, float* y, std::size_t n, bool accumulate) {
  const std::size_t n_out = w.ne1, n_in = w.ne0;
  if (q8_path(w)) {
    const void* ws[1] = {w.dev};
    float* ys[1] = {y};
    const std::size_t no[1] = {n_out};
    probe_begin(w);
    const int rc =
        axon_hip_matmul_q8_fused(static_cast<int>(w.type), xq, n, n_in, 1, ws, ys, no, no, accumulate ? 1 : 0);
    probe_end(w, n, n_out, accumulate);
    return rc;
  }
  probe_begin(w);
  float* out = accumulate ? tmp_ : y;
  const kernels::KernelTable& k = *kernels_;
  const bool one = n == 1;
  switch (w.type) {
  case DType::F32: {
    const auto* p = static_cast<const float*>(w.dev);
    one ? k.matmul_f32(p, x, out, n_out, n_in) : k.matmul_f32_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  case DType::F16: {
    const auto* p = static_cast<const std::uint16_t*>(w.dev);
    one ? k.matmul_f16(p, x, out, n_out, n_in) : k.matmul_f16_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  case DType::BF16: {
    const auto* p = static_cast<const std::uint16_t*>(w.dev);
    one ? k.matmul_bf16(p, x, out, n_out, n_in) : k.matmul_bf16_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  case DType::Q8_0: {
    const auto* p = static_cast<const BlockQ8_0*>(w.dev);
    one ? k.matmul_q8_0(p, x, out, n_out, n_in) : k.matmul_q8_0_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  case DType::Q4_0: {
    const auto* p = static_cast<const BlockQ4_0*>(w.dev);
    one ? k.matmul_q4_0(p, x, out, n_out, n_in) : k.matmul_q4_0_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  case DType::Q4_1: {
    const auto* p = static_cast<const BlockQ4_1*>(w.dev);
    one ? k.matmul_q4_1(p, x, out, n_out, n_in) : k.matmul_q4_1_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  case DType::Q6_K: {
    if (w.planar != nullptr) {
      const int rc = axon_hip_matmul_q6_k_planar(w.planar, x, out, n, n_out, n_in, n_out);
      if (rc != AXON_HIP_OK) return rc;
      break;
    }
    const auto* p = static_cast<const BlockQ6_K*>(w.dev);
    one ? k.matmul_q6_k(p, x, out, n_out, n_in) : k.matmul_q6_k_rows(p, x, out, n, n_out, n_in, n_out);
    break;
  }
  }
  probe_end(w, n, n_out, false);
  return accumulate ? axon_hip_add(y, tmp_, n * n_out) : AXON_HIP_OK;
}

Expected<std::size_t> LlamaModel::run(std::span<const Row> rows, bool copy_logits, std::size_t first_logit) {
  const std::size_t n = rows.size();
  const Config& c = cfg_;
  const std::size_t d = c.n_embd, dq = c.n_embd_q(), dkv = c.n_embd_kv(), ff = c.n_ff;
  const std::size_t R = max_rows_;
  // Row table: ids | pos | n_vis | cache_off (llama.cpp:360: each row's own position).
  auto* ids = static_cast<std::int32_t*>(rowinfo_host_);
  std::int32_t* pos = ids + R;
  std::int32_t* nvis = pos + R;
  auto* coff = reinterpret_cast<std::int64_t*>(static_cast<std::byte*>(rowinfo_host_) + align_up(12 * R, 8));
  last_rows_ = 0;
  // The cache-free forward's rows all name slot n_slots_: its keys and values go to the float
  // area kv_free_ (max_seq positions per layer); cached passes use the pool in the cache type
  // (llama.cpp:379-383, 520-563).
  const bool free_pass = n > 0 && rows[0].slot == static_cast<int>(n_slots_);
  void* const kv = free_pass ? static_cast<void*>(kv_free_) : kv_;
  const int kv_f16 = !free_pass && cache_type_ == CacheType::F16 ? 1 : 0;
  const std::size_t layer_ctx = free_pass ? max_seq_ : max_ctx_;
  // The previous call's row table may still be in flight when its logits stayed on the device.
  if (axon_hip_synchronize() != AXON_HIP_OK) return device_error("synchronize");
  if (auto st = check_persistent_status(); !st) return st.error();
  std::uint32_t max_vis = 0;
  for (std::size_t i = 0; i < n; ++i) {
    ids[i] = rows[i].token;
    pos[i] = rows[i].pos;
    nvis[i] = rows[i].pos + 1;
    coff[i] = free_pass ? 0 : static_cast<std::int64_t>(rows[i].slot) * static_cast<std::int64_t>(slot_elems_);
    max_vis = std::max<std::uint32_t>(max_vis, static_cast<std::uint32_t>(nvis[i]));
  }
  const std::size_t info_bytes = align_up(12 * R, 8) + 8 * R;
  if (axon_hip_memcpy_h2d_async(rowinfo_, rowinfo_host_, info_bytes) != AXON_HIP_OK) return device_error("row table");
  const auto* d_ids = static_cast<const std::int32_t*>(rowinfo_);
  const std::int32_t* d_pos = d_ids + R;
  const std::int32_t* d_nvis = d_pos + R;
  const auto* d_coff = reinterpret_cast<const std::int64_t*>(static_cast<const std::byte*>(rowinfo_) + align_up(12 * R, 8));

  const float scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));
  const float eps = c.rms_eps;
#define DEV(call)                                                  \
  do {                                                             \
    if ((call) != AXON_HIP_OK) return device_error(#call);         \
  } while (0)

  DEV(axon_hip_embedding_rows(static_cast<int>(token_embd_.type), token_embd_.dev, d, d_ids, n, x_));
  // Decode-sized calls (up to four rows) fold the norms, quantizations, RoPE, KV write and
  // SiLU into the matvec launches (axon_hip_matvec_fused); other calls run them apart.
  const bool fuse = n <= 4 && !exact_;
  const auto fused_ok = [&](const Tensor& w, int in_mode, std::size_t n_in, bool silu) {
    return fuse && q8_path(w) && axon_hip_matvec_fused_supported(static_cast<int>(w.type), in_mode, n, n_in, silu) == 1;
  };
  const auto fused_args = [&](const Tensor& w) {
    axon_hip_matvec_fused_args fa{};
    fa.type = static_cast<int>(w.type);
    fa.n_rows = n;
    fa.n_in = w.ne0;
    fa.eps = eps;
    return fa;
  };
  // One row of a cached pass: every layer in one persistent kernel.
  const bool persistent = step_ok_ && n == 1 && !free_pass;
  if (persistent) {
    if (auto st = step_reserve(1); !st) return st.error();
    // Until the next synchronization checks the status word, this pass may yet turn out void:
    // its cache and starting position, to roll back to.
    step_pending_ = slot_cache_[static_cast<std::size_t>(rows[0].slot)];
    step_pending_pos_ = static_cast<std::size_t>(rows[0].pos);
    axon_hip_decode_layers_args sa{};
    sa.layers = static_cast<const axon_hip_decode_layer*>(step_layers_);
    sa.eps = eps;
    sa.scale = scale;
    sa.rope_table = rope_table_;
    sa.x = x_;
    sa.cache = static_cast<float*>(kv_);
    sa.cache_off = coff[0];
    sa.pos = pos[0];
    sa.work = step_work_;
    sa.epoch = &step_epoch_;
    sa.status = step_status_;
    // The probe counts the whole kernel as one launch of the layers' q|k|v type.
    const bool probed = (probe_type_ == kProbeStep || probe_type_ == step_shape_.type_qkv) &&
                        2 * probe_used_ + 2 <= probe_events_.size();
    if (probed) axon_hip_probe_next_launch(probe_events_[2 * probe_used_], probe_events_[2 * probe_used_ + 1]);
    const int rc = axon_hip_decode_layers(&step_shape_, &sa);
    if (probed) axon_hip_probe_next_launch(nullptr, nullptr);
    if (rc != AXON_HIP_OK) return device_error("decode_layers");
    if (probed) {
      probe_bytes_.push_back(step_bytes(static_cast<std::size_t>(pos[0]) + 1));
      ++probe_used_;
    }
  }
  for (std::size_t l = 0; l < (persistent ? 0 : c.n_layer); ++l) {
    const Layer& L = layers_[l];
    const std::int64_t k_layer = static_cast<std::int64_t>(2 * l) * layer_ctx * dkv;
    const std::int64_t v_layer = k_layer + static_cast<std::int64_t>(layer_ctx * dkv);

    // attention block (llama.cpp:500-595)
    const bool qkv_q8 = q8_path(L.wq) && q8_path(L.wk) && q8_path(L.wv) && L.wq.type == L.wk.type &&
                        L.wk.type == L.wv.type;
    if (qkv_q8 && c.rope_style == kernels::RopeStyle::Normal && fused_ok(L.wq, 2, d, false)) {
      // attn_norm, quantize, q|k|v, bias, RoPE and the KV write in one launch.
      axon_hip_matvec_fused_args fa = fused_args(L.wq);
      fa.n_seg = 3;
      fa.w[0] = L.wq.dev;
      fa.w[1] = L.wk.dev;
      fa.w[2] = L.wv.dev;
      fa.n_out[0] = dq;
      fa.n_out[1] = dkv;
      fa.n_out[2] = dkv;
      fa.in_mode = 2;
      fa.x = x_;
      fa.x_stride = d;
      fa.norm_w = static_cast<const float*>(L.attn_norm.dev);
      fa.out_mode = 3;
      fa.y[0] = q_;
      fa.y_stride[0] = dq;
      if (L.bias) {
        fa.bias[0] = static_cast<const float*>(L.bq.dev);
        fa.bias[1] = static_cast<const float*>(L.bk.dev);
        fa.bias[2] = static_cast<const float*>(L.bv.dev);
      }
      fa.rope_table = rope_table_;
      fa.rot_half = c.rotary_dim / 2;
      fa.head_dim = c.head_dim;
      fa.pos = d_pos;
      fa.cache_off = d_coff;
      fa.cache = kv;
      fa.cache_f16 = kv_f16;
      fa.k_layer_off = k_layer;
      fa.v_layer_off = v_layer;
      probe_begin(L.wq);
      DEV(axon_hip_matvec_fused(&fa));
      probe_end(L.wq, n, dq + 2 * dkv, false);
    } else {
      const bool need_q8 = q8_path(L.wq) || q8_path(L.wk) || q8_path(L.wv);
      const bool need_f = !q8_path(L.wq) || !q8_path(L.wk) || !q8_path(L.wv);
      DEV(axon_hip_rmsnorm_rows(x_, static_cast<const float*>(L.attn_norm.dev), need_f ? h_ : nullptr,
                                need_q8 ? xq_ : nullptr, d, n, eps));
      // Up to 64 rows: q|k|v with the bias, RoPE and KV write in the matmul's epilogue.
      bool roped = false;
      if (qkv_q8 && c.rope_style == kernels::RopeStyle::Normal && rope_table_ != nullptr) {
        axon_hip_matvec_fused_args fa = fused_args(L.wq);
        fa.n_seg = 3;
        fa.w[0] = L.wq.dev;
        fa.w[1] = L.wk.dev;
        fa.w[2] = L.wv.dev;
        fa.n_out[0] = dq;
        fa.n_out[1] = dkv;
        fa.n_out[2] = dkv;
        fa.in_mode = 0;
        fa.xq = xq_;
        fa.out_mode = 3;
        fa.y[0] = q_;
        fa.y_stride[0] = dq;
        if (L.bias) {
          fa.bias[0] = static_cast<const float*>(L.bq.dev);
          fa.bias[1] = static_cast<const float*>(L.bk.dev);
          fa.bias[2] = static_cast<const float*>(L.bv.dev);
        }
        fa.rope_table = rope_table_;
        fa.rot_half = c.rotary_dim / 2;
        fa.head_dim = c.head_dim;
        fa.pos = d_pos;
        fa.cache_off = d_coff;
        fa.cache = kv;
        fa.cache_f16 = kv_f16;
        fa.k_layer_off = k_layer;
        fa.v_layer_off = v_layer;
        probe_begin(L.wq);
        const int rc = axon_hip_matmul_q8_qkv_rope(&fa);
        if (rc == AXON_HIP_OK) {
          probe_end(L.wq, n, dq + 2 * dkv, false);
          roped = true;
        } else if (rc == AXON_HIP_E_UNSUPPORTED) {
          probe_cancel();  // refused: nothing was launched
        } else {
          return device_error("matmul_q8_qkv_rope");
        }
      }
      if (!roped) {
        if (qkv_q8) {
          const void* ws[3] = {L.wq.dev, L.wk.dev, L.wv.dev};
          float* ys[3] = {q_, k_, v_};
          const std::size_t no[3] = {dq, dkv, dkv};
          probe_begin(L.wq);
          DEV(axon_hip_matmul_q8_fused(static_cast<int>(L.wq.type), xq_, n, d, 3, ws, ys, no, no, 0));
          probe_end(L.wq, n, dq + 2 * dkv, false);
        } else {
          DEV(mm(L.wq, h_, xq_, q_, n, false));
          DEV(mm(L.wk, h_, xq_, k_, n, false));
          DEV(mm(L.wv, h_, xq_, v_, n, false));
        }
        axon_hip_rope_rows_args ra{};
        ra.q = q_;
        ra.k = k_;
        ra.v = v_;
        if (L.bias) {
          ra.bq = static_cast<const float*>(L.bq.dev);
          ra.bk = static_cast<const float*>(L.bk.dev);
          ra.bv = static_cast<const float*>(L.bv.dev);
        }
        ra.pos = d_pos;
        ra.q_stride = static_cast<std::uint32_t>(dq);
        ra.k_stride = static_cast<std::uint32_t>(dkv);
        ra.n_head = c.n_head;
        ra.n_kv = c.n_head_kv;
        ra.head_dim = c.head_dim;
        ra.rotary_dim = c.rotary_dim;
        ra.neox = c.rope_style == kernels::RopeStyle::NeoX ? 1 : 0;
        ra.theta = c.rope_theta;
        ra.table = rope_table_;
        ra.cache = kv;
        ra.cache_f16 = kv_f16;
        ra.cache_off = d_coff;
        ra.k_layer_off = k_layer;
        ra.v_layer_off = v_layer;
        DEV(axon_hip_rope_rows(&ra, n));
      }
    }

    const bool wo_fused = fused_ok(L.wo, 0, dq, false);
    axon_hip_attention_rows_args aa{};
    aa.q = q_;
    aa.out = attn_;
    aa.q_stride = static_cast<std::uint32_t>(dq);
    aa.out_stride = static_cast<std::uint32_t>(dq);
    aa.kv = kv;
    aa.f16 = kv_f16;
    aa.k_off = d_coff;
    aa.v_off = d_coff;
    aa.n_vis = d_nvis;
    aa.k_layer_off = k_layer;
    aa.v_layer_off = v_layer;
    aa.n_head = c.n_head;
    aa.n_kv = c.n_head_kv;
    aa.head_dim = c.head_dim;
    aa.scale = scale;
    aa.scratch = scores_;
    aa.max_vis = max_vis;
    // wo's Q8_0 input, quantized in the attention epilogue.
    aa.outq = q8_path(L.wo) ? xq_ : nullptr;
    // The attention probe brackets the layer's attention launches with events on the stream.
    const bool attn_probed = probe_type_ == kProbeAttention && 2 * probe_used_ + 2 <= probe_events_.size();
    if (attn_probed && axon_hip_event_record(probe_events_[2 * probe_used_]) != AXON_HIP_OK)
      return device_error("attention probe");
    DEV(axon_hip_attention_rows(&aa, n));
    if (attn_probed) {
      if (axon_hip_event_record(probe_events_[2 * probe_used_ + 1]) != AXON_HIP_OK) return device_error("attention probe");
      // Algorithmic bytes: each row's K and V rows over its visible positions, q in, the output.
      double kv_rows = 0;
      for (std::size_t i = 0; i < n; ++i) kv_rows += nvis[i];
      const double elem = kv_f16 ? 2.0 : 4.0;
      probe_bytes_.push_back(kv_rows * 2.0 * static_cast<double>(dkv) * elem + 2.0 * static_cast<double>(n * dq) * 4.0);
      ++probe_used_;
    }

    if (wo_fused) {
      axon_hip_matvec_fused_args fa = fused_args(L.wo);
      fa.n_seg = 1;
      fa.w[0] = L.wo.dev;
      fa.n_out[0] = d;
      fa.in_mode = 0;
      fa.xq = xq_;
      fa.out_mode = 1;
      fa.y[0] = x_;
      fa.y_stride[0] = d;
      probe_begin(L.wo);
      DEV(axon_hip_matvec_fused(&fa));
      probe_end(L.wo, n, d, true);
    } else {
      DEV(mm(L.wo, attn_, xq_, x_, n, true));
    }

    // feed-forward block (llama.cpp:598-623)
    const bool gu_q8 = q8_path(L.w_gate) && q8_path(L.w_up) && L.w_gate.type == L.w_up.type;
    if (gu_q8 && fused_ok(L.w_gate, 2, d, true) && fused_ok(L.w_down, 1, ff, false)) {
      // ffn_norm, quantize, gate|up and SiLU * up in one launch; quantize, down and the
      // residual add in the next.
      axon_hip_matvec_fused_args fa = fused_args(L.w_gate);
      fa.n_seg = 2;
      fa.w[0] = L.w_gate.dev;
      fa.w[1] = L.w_up.dev;
      fa.n_out[0] = ff;
      fa.n_out[1] = ff;
      fa.in_mode = 2;
      fa.x = x_;
      fa.x_stride = d;
      fa.norm_w = static_cast<const float*>(L.ffn_norm.dev);
      fa.out_mode = 2;
      fa.y[0] = gate_;
      fa.y_stride[0] = ff;
      // The SiLU epilogue also writes down's Q8_0 input when the launch shape allows it (whole
      // blocks per workgroup in LDS); down then reads blocks instead of quantizing h itself.
      const bool down_q8 = q8_path(L.w_down) && ff % 32 == 0 && fused_ok(L.w_down, 0, ff, false);
      fa.outq = down_q8 ? xq_ : nullptr;
      probe_begin(L.w_gate);
      int rc = axon_hip_matvec_fused(&fa);
      if (rc == AXON_HIP_E_UNSUPPORTED && fa.outq != nullptr) {
        fa.outq = nullptr;
        rc = axon_hip_matvec_fused(&fa);
      }
      DEV(rc);
      probe_end(L.w_gate, n, 2 * ff, false);
      axon_hip_matvec_fused_args fd = fused_args(L.w_down);
      fd.n_seg = 1;
      fd.w[0] = L.w_down.dev;
      fd.n_out[0] = d;
      fd.in_mode = fa.outq != nullptr ? 0 : 1;
      fd.xq = xq_;
      fd.x = gate_;
      fd.x_stride = ff;
      fd.out_mode = 1;
      fd.y[0] = x_;
      fd.y_stride[0] = d;
      probe_begin(L.w_down);
      DEV(axon_hip_matvec_fused(&fd));
      probe_end(L.w_down, n, d, true);
      continue;
    }
    const bool ff_q8 = q8_path(L.w_gate) || q8_path(L.w_up);
    const bool ff_f = !q8_path(L.w_gate) || !q8_path(L.w_up);
    DEV(axon_hip_rmsnorm_rows(x_, static_cast<const float*>(L.ffn_norm.dev), ff_f ? h_ : nullptr,
                              ff_q8 ? xq_ : nullptr, d, n, eps));
    // gate|up, SiLU and down's Q8_0 input in one tile launch, the blocks into tmp_ (xq_ is
    // still being read as its input); the launcher refuses decode-sized calls whose FFN is too
    // narrow to fill the chip, and those run the matmul and silu_mul apart.
    const void* down_xq = xq_;
    bool swiglu = false;
    if (gu_q8 && q8_path(L.w_down) && ff % 32 == 0) {
      probe_begin(L.w_gate);
      const int rc = axon_hip_matmul_q8_swiglu(static_cast<int>(L.w_gate.type), xq_, n, d, L.w_gate.dev, L.w_up.dev,
                                               ff, nullptr, tmp_);
      if (rc == AXON_HIP_OK) {
        // Its output is down's Q8_0 blocks, not 2 * ff floats per row.
        probe_end(L.w_gate, n, 2 * ff, false, static_cast<double>(n) * (ff / 32) * sizeof(BlockQ8_0));
      } else {
        probe_cancel();  // refused: nothing was launched, so no event pair was recorded
      }
      if (rc == AXON_HIP_OK) {
        swiglu = true;
        down_xq = tmp_;
      } else if (rc != AXON_HIP_E_UNSUPPORTED) {
        return device_error("matmul_q8_swiglu");
      }
    }
    if (!swiglu) {
      if (gu_q8) {
        const void* ws[2] = {L.w_gate.dev, L.w_up.dev};
        float* ys[2] = {gate_, up_};
        const std::size_t no[2] = {ff, ff};
        probe_begin(L.w_gate);
        DEV(axon_hip_matmul_q8_fused(static_cast<int>(L.w_gate.type), xq_, n, d, 2, ws, ys, no, no, 0));
        probe_end(L.w_gate, n, 2 * ff, false);
      } else {
        DEV(mm(L.w_gate, h_, xq_, gate_, n, false));
        DEV(mm(L.w_up, h_, xq_, up_, n, false));
      }
      if (q8_path(L.w_down)) {
        DEV(axon_hip_silu_mul_rows(gate_, up_, nullptr, xq_, ff, n));
      } else {
        DEV(axon_hip_silu_mul_rows(gate_, up_, gate_, nullptr, ff, n));
      }
    }
    DEV(mm(L.w_down, gate_, down_xq, x_, n, true));
  }
  // The final norm and the output matmul for the rows whose logits the pass returns.
  float* const x_out = x_ + first_logit * d;
  const std::size_t n_out = n - first_logit;
  if (!exact_ && n_out <= 4 && q8_path(output_) &&
      axon_hip_matvec_fused_supported(static_cast<int>(output_.type), 2, n_out, d, false) == 1) {
    axon_hip_matvec_fused_args fa = fused_args(output_);
    fa.n_rows = n_out;
    fa.n_seg = 1;
    fa.w[0] = output_.dev;
    fa.n_out[0] = c.n_vocab;
    fa.in_mode = 2;
    fa.x = x_out;
    fa.x_stride = d;
    fa.norm_w = static_cast<const float*>(output_norm_.dev);
    fa.out_mode = 0;
    fa.y[0] = logits_;
    fa.y_stride[0] = c.n_vocab;
    probe_begin(output_);
    DEV(axon_hip_matvec_fused(&fa));
    probe_end(output_, n_out, c.n_vocab, false);
  } else {
    const bool out_q8 = q8_path(output_);
    DEV(axon_hip_rmsnorm_rows(x_out, static_cast<const float*>(output_norm_.dev), out_q8 ? nullptr : h_,
                              out_q8 ? xq_ : nullptr, d, n_out, eps));
    DEV(mm(output_, h_, xq_, logits_, n_out, false));
  }
  if (copy_logits) {
    logits_host_.resize(n_out * c.n_vocab);
    DEV(axon_hip_memcpy_d2h(logits_host_.data(), logits_, logits_host_.size() * 4));
    if (auto st = check_persistent_status(); !st) return st.error();
  }
#undef DEV
  (void)R;
  last_rows_ = n_out;
  return n_out;
}

Expected<std::size_t> LlamaModel::greedy(std::span<std::int32_t> ids,
                                         std::span<const std::span<const std::int32_t>> recent,
                                         float repeat_penalty, int repeat_last_n) {
  const std::size_t n = last_rows_;
  if (n == 0) return make_error(ErrorCode::InvalidArgument, "greedy: no logits from a forward pass");
  if (ids.size() != n)
    return make_error(ErrorCode::InvalidArgument,
                      "greedy: " + std::to_string(ids.size()) + " ids for " + std::to_string(n) + " rows of logits");
  if (!recent.empty() && recent.size() != n)
    return make_error(ErrorCode::InvalidArgument,
                      "greedy: " + std::to_string(recent.size()) + " recent windows for " + std::to_string(n) + " rows");
  last_rows_ = 0;
  auto p = penalize(n, recent, repeat_penalty, repeat_last_n, {});
  if (!p) return p.error();
  if (axon_hip_argmax_rows(logits_, cfg_.n_vocab, n, cfg_.n_vocab, argmax_scratch_, ids_) != AXON_HIP_OK)
    return device_error("greedy");
  // A synchronous copy on the library stream: the staging above is free again when it returns.
  if (axon_hip_memcpy_d2h(ids.data(), ids_, n * 4) != AXON_HIP_OK) return device_error("greedy");
  if (auto st = check_persistent_status(); !st) return st.error();
  return n;
}

Expected<std::size_t> LlamaModel::generate_greedy(KVCache& cache, std::int32_t token, std::span<std::int32_t> out) {
  const std::size_t n = out.size();
  const Config& c = cfg_;
  if (n == 0) return std::size_t{0};
  if (cache.slot() < 0 || static_cast<std::size_t>(cache.slot()) >= n_slots_ || cache.max_ctx() != max_ctx_)
    return make_error(ErrorCode::InvalidArgument, "generate: the cache was built for a different model");
  if (token < 0 || static_cast<std::uint32_t>(token) >= c.n_vocab)
    return make_error(ErrorCode::InvalidArgument, "forward: token id " + std::to_string(token) + " outside the vocabulary");
  if (cache.pos() + n > max_ctx_)
    return make_error(ErrorCode::InvalidArgument, "context overflow: " + std::to_string(n) + " steps from position " +
                                                      std::to_string(cache.pos()) + " exceed " + std::to_string(max_ctx_));
  if (!step_ok_) {
    // Without the persistent kernel, the host loop of forward_one and greedy.
    std::int32_t tok = token;
    for (std::size_t i = 0; i < n; ++i) {
      auto r = forward_prefill_device(cache, std::span<const std::int32_t>(&tok, 1));
      if (!r) return r.error();
      auto g = greedy(std::span<std::int32_t>(&tok, 1));
      if (!g) return g.error();
      out[i] = tok;
    }
    return n;
  }
  if (axon_hip_synchronize() != AXON_HIP_OK) return device_error("synchronize");
  if (auto st = check_persistent_status(); !st) return st.error();
  if (auto st = step_reserve(n); !st) return st.error();
  last_rows_ = 0;
  if (axon_hip_memcpy_h2d(gen_ids_, &token, 4) != AXON_HIP_OK) return device_error("generate");
  const std::size_t d = c.n_embd;
  const std::int64_t coff = static_cast<std::int64_t>(cache.slot()) * static_cast<std::int64_t>(slot_elems_);
  const float scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));
  const bool out_fused = !exact_ && q8_path(output_) &&
                         axon_hip_matvec_fused_supported(static_cast<int>(output_.type), 2, 1, d, false) == 1;
  // The planar Q6_K output leaves greedy keys behind, and one launch then takes the choice and
  // the next step's embedding (two launches fewer per token).
  const bool out_keys = !out_fused && output_.type == DType::Q6_K && output_.planar != nullptr &&
                        axon_hip_q6k_argmax_parts(c.n_vocab) <= argmax_words_;
  bool embedded = false;  // x_ already holds the embedding of gen_ids_[i]
  for (std::size_t i = 0; i < n; ++i) {
    // Step i: the embedding of gen_ids_[i] (the previous step's choice), every layer in one
    // launch, the output norm and matrix, the greedy choice into gen_ids_[i + 1].
    if (!embedded &&
        axon_hip_embedding_rows(static_cast<int>(token_embd_.type), token_embd_.dev, d, gen_ids_ + i, 1, x_) !=
            AXON_HIP_OK)
      return device_error("generate: embedding");
    embedded = false;
    axon_hip_decode_layers_args sa{};
    sa.layers = static_cast<const axon_hip_decode_layer*>(step_layers_);
    sa.eps = c.rms_eps;
    sa.scale = scale;
    sa.rope_table = rope_table_;
    sa.x = x_;
    sa.cache = static_cast<float*>(kv_);
    sa.cache_off = coff;
    sa.pos = static_cast<std::int32_t>(cache.pos() + i);
    sa.work = step_work_;
    sa.epoch = &step_epoch_;
    sa.status = step_status_;
    if (axon_hip_decode_layers(&step_shape_, &sa) != AXON_HIP_OK) return device_error("generate: decode_layers");
    if (out_fused) {
      axon_hip_matvec_fused_args fa{};
      fa.type = static_cast<int>(output_.type);
      fa.n_rows = 1;
      fa.n_in = d;
      fa.eps = c.rms_eps;
      fa.n_seg = 1;
      fa.w[0] = output_.dev;
      fa.n_out[0] = c.n_vocab;
      fa.in_mode = 2;
      fa.x = x_;
      fa.x_stride = d;
      fa.norm_w = static_cast<const float*>(output_norm_.dev);
      fa.out_mode = 0;
      fa.y[0] = logits_;
      fa.y_stride[0] = c.n_vocab;
      if (axon_hip_matvec_fused(&fa) != AXON_HIP_OK) return device_error("generate: output");
    } else if (out_keys) {
      if (axon_hip_rmsnorm_rows(x_, static_cast<const float*>(output_norm_.dev), h_, nullptr, d, 1, c.rms_eps) !=
              AXON_HIP_OK ||
          axon_hip_matmul_q6_k_planar_argmax(output_.planar, h_, logits_, c.n_vocab, d, argmax_scratch_,
                                             argmax_words_) != AXON_HIP_OK)
        return device_error("generate: output");
      // The choice into gen_ids_[i + 1] and its embedding, the next step's input (after the
      // last step it goes unused).
      if (axon_hip_argmax_embed(logits_, argmax_scratch_, axon_hip_q6k_argmax_parts(c.n_vocab), gen_ids_ + i + 1,
                                static_cast<int>(token_embd_.type), token_embd_.dev, token_embd_.ne1, d,
                                x_) != AXON_HIP_OK)
        return device_error("generate: greedy");
      embedded = true;
      continue;
    } else {
      const bool out_q8 = q8_path(output_);
      if (axon_hip_rmsnorm_rows(x_, static_cast<const float*>(output_norm_.dev), out_q8 ? nullptr : h_,
                                out_q8 ? xq_ : nullptr, d, 1, c.rms_eps) != AXON_HIP_OK ||
          mm(output_, h_, xq_, logits_, 1, false) != AXON_HIP_OK)
        return device_error("generate: output");
    }
    if (axon_hip_argmax_rows(logits_, c.n_vocab, 1, c.n_vocab, argmax_scratch_, gen_ids_ + i + 1) != AXON_HIP_OK)
      return device_error("generate: greedy");
  }
  if (axon_hip_memcpy_d2h(out.data(), gen_ids_ + 1, n * 4) != AXON_HIP_OK) return device_error("generate");
  if (auto st = check_persistent_status(); !st) return st.error();
  cache.advance(n);
  return n;
}

Expected<bool> LlamaModel::penalize(std::size_t n, std::span<const std::span<const std::int32_t>> recent,
                                    float penalty, int repeat_last_n, std::span<const std::uint8_t> select,
                                    bool reuse) {
  // sampler.cpp:73: the penalty runs when it is not 1 and the window is not empty.
  std::size_t width = 0;
  if (penalty != 1.0F && repeat_last_n > 0) {
    for (std::size_t r = 0; r < recent.size(); ++r)
      if (select.empty() || select[r] != 0)
        width = std::max(width, std::min(recent[r].size(), static_cast<std::size_t>(repeat_last_n)));
  }
  if (width > kMaxPenaltyWindow)
    return make_error(ErrorCode::InvalidArgument, "sampling: a penalty window of " + std::to_string(width) +
                                                      " ids exceeds " + std::to_string(kMaxPenaltyWindow));
  if (width == 0) return true;
  // Row r's window is the last min(len, repeat_last_n) ids of its history, packed [n][width];
  // rows outside the selection get an empty window.
  auto* win = static_cast<std::int32_t*>(window_host_);
  auto* len = reinterpret_cast<std::uint32_t*>(win + n * width);
  for (std::size_t r = 0; r < n; ++r) {
    const std::size_t w =
        select.empty() || select[r] != 0 ? std::min(recent[r].size(), static_cast<std::size_t>(repeat_last_n)) : 0;
    std::copy(recent[r].end() - static_cast<std::ptrdiff_t>(w), recent[r].end(), win + r * width);
    len[r] = static_cast<std::uint32_t>(w);
  }
  auto* dwin = static_cast<std::int32_t*>(window_);
  auto* dlen = reinterpret_cast<std::uint32_t*>(dwin + n * width);
  // The copy from the pinned staging runs in stream order; a following call rewrites the
  // staging, so it waits for the stream first.
  if (axon_hip_memcpy_h2d_async(window_, window_host_, n * (width + 1) * 4) != AXON_HIP_OK ||
      axon_hip_repeat_penalty_rows(logits_, cfg_.n_vocab, n, cfg_.n_vocab, dwin, dlen, width, penalty) != AXON_HIP_OK ||
      (reuse && axon_hip_synchronize() != AXON_HIP_OK))
    return device_error("sampling: repetition penalty");
  return true;
}

Expected<std::size_t> LlamaModel::sample(std::span<std::int32_t> ids, std::span<const sampling::Config> configs,
                                         std::span<sampling::Rng> rngs,
                                         std::span<const std::span<const std::int32_t>> recent) {
  const std::size_t n = last_rows_;
  const std::size_t V = cfg_.n_vocab;
  if (n == 0) return make_error(ErrorCode::InvalidArgument, "sample: no logits from a forward pass");
  if (ids.size() != n || configs.size() != n || rngs.size() != n)
    return make_error(ErrorCode::InvalidArgument, "sample: " + std::to_string(ids.size()) + " ids, " +
                                                      std::to_string(configs.size()) + " configs and " +
                                                      std::to_string(rngs.size()) + " generators for " +
                                                      std::to_string(n) + " rows of logits");
  if (!recent.empty() && recent.size() != n)
    return make_error(ErrorCode::InvalidArgument,
                      "sample: " + std::to_string(recent.size()) + " recent windows for " + std::to_string(n) + " rows");
  std::size_t k_max = 0;
  bool any_greedy = false;
  for (std::size_t r = 0; r < n; ++r) {
    if (configs[r].temperature <= 0.0F) {
      any_greedy = true;
      continue;
    }
    k_max = std::max(k_max, sampling::kept_after_top_k(configs[r], V));
  }
  // Up to AXON_HIP_MAX_TOPK candidates a row come from the top-k kernel; beyond that every row
  // is sorted whole (the same order, so a row's first top_k candidates are the same either way).
  const bool whole = k_max > AXON_HIP_MAX_TOPK;
  if (whole && n > sort_rows_) {
    for (void** p : {&sort_out_, &sort_work_}) {
      if (*p != nullptr) axon_hip_free(*p);
      *p = nullptr;
    }
    sort_rows_ = 0;
    if (axon_hip_malloc(&sort_out_, n * V * 8) != AXON_HIP_OK ||
        axon_hip_malloc(&sort_work_, axon_hip_sort_rows_work_bytes(V, n)) != AXON_HIP_OK)
      return device_error("sample: whole-vocabulary candidates");
    sort_rows_ = n;
  }
  const std::size_t width = whole ? V : k_max;  // candidates a row holds on the device
  last_rows_ = 0;
  // The penalty, once per distinct (penalty, window) setting among the rows.
  if (!recent.empty()) {
    std::vector<std::uint8_t>& done = sample_done_;
    std::vector<std::uint8_t>& select = sample_select_;
    done.assign(n, 0);
    select.assign(n, 0);
    for (std::size_t r = 0; r < n; ++r) {
      if (done[r] != 0) continue;
      for (std::size_t q = r; q < n; ++q) {
        select[q] = configs[q].repeat_penalty == configs[r].repeat_penalty &&
                    configs[q].repeat_last_n == configs[r].repeat_last_n;
        done[q] |= select[q];
      }
      const bool more = std::find(done.begin(), done.end(), 0) != done.end();
      auto p = penalize(n, recent, configs[r].repeat_penalty, configs[r].repeat_last_n, select, more);
      if (!p) return p.error();
      std::fill(select.begin(), select.end(), 0);
    }
  }
  void* cand = whole ? sort_out_ : cand_;
  auto* cand_logits = static_cast<float*>(cand);
  auto* cand_ids = reinterpret_cast<std::int32_t*>(cand_logits + n * width);
  if (any_greedy && axon_hip_argmax_rows(logits_, V, n, V, argmax_scratch_, ids_) != AXON_HIP_OK)
    return device_error("sample");
  if (k_max != 0 && (whole ? axon_hip_sort_rows(logits_, V, n, V, sort_work_, cand_logits, cand_ids)
                           : axon_hip_topk_rows(logits_, V, n, V, k_max, cand_logits, cand_ids)) != AXON_HIP_OK)
    return device_error("sample");
  // Synchronous copies on the library stream.
  if (any_greedy && axon_hip_memcpy_d2h(ids.data(), ids_, n * 4) != AXON_HIP_OK) return device_error("sample");
  if (auto st = check_persistent_status(); !st) return st.error();
  if (k_max == 0) return n;
  cand_host_.resize(n * width * 8);
  if (axon_hip_memcpy_d2h(cand_host_.data(), cand, n * width * 8) != AXON_HIP_OK) return device_error("sample");
  const auto* hl = reinterpret_cast<const float*>(cand_host_.data());
  const auto* hi = reinterpret_cast<const std::int32_t*>(hl + n * width);
  probs_.resize(k_max);
  for (std::size_t r = 0; r < n; ++r) {
    if (configs[r].temperature <= 0.0F) continue;
    std::size_t kept = sampling::kept_after_top_k(configs[r], V);
    while (kept > 1 && hi[r * width + kept - 1] < 0) --kept;  // NaN logits are never candidates
    ids[r] = sampling::draw(configs[r], rngs[r], hl + r * width, hi + r * width, kept, probs_.data());
  }
  return n;
}

Expected<std::span<const float>> LlamaModel::forward(std::span<const std::int32_t> tokens) {
  return forward_rows(tokens, true);
}

Expected<std::size_t> LlamaModel::forward_device(std::span<const std::int32_t> tokens) {
  auto r = forward_rows(tokens, false);
  if (!r) return r.error();
  return tokens.size();
}

Expected<std::span<const float>> LlamaModel::forward_rows(std::span<const std::int32_t> tokens, bool copy_logits) {
  if (tokens.empty()) return make_error(ErrorCode::InvalidArgument, "forward: empty token sequence");
  if (tokens.size() > max_seq_)
    return make_error(ErrorCode::InvalidArgument, "forward: " + std::to_string(tokens.size()) + " tokens exceed max_seq");
  for (std::size_t i = 0; i < tokens.size(); ++i) {
    if (tokens[i] < 0 || static_cast<std::uint32_t>(tokens[i]) >= cfg_.n_vocab)
      return make_error(ErrorCode::InvalidArgument, "forward: token id " + std::to_string(tokens[i]) + " outside the vocabulary");
    rows_[i] = Row{tokens[i], static_cast<std::int32_t>(i), static_cast<int>(n_slots_)};
  }
  auto r = run(std::span<const Row>(rows_.data(), tokens.size()), copy_logits);
  if (!r) return r.error();
  return std::span<const float>(logits_host_);
}

Expected<std::size_t> LlamaModel::prefill_rows(const KVCache& cache, std::span<const std::int32_t> tokens,
                                               std::size_t at) {
  if (tokens.empty()) return make_error(ErrorCode::InvalidArgument, "forward: empty token sequence");
  if (tokens.size() > max_seq_)
    return make_error(ErrorCode::InvalidArgument, "forward: " + std::to_string(tokens.size()) + " tokens exceed max_seq");
  if (cache.pos() + tokens.size() > cache.max_ctx())
    return make_error(ErrorCode::InvalidArgument, "context overflow: " + std::to_string(cache.pos()) + " cached + " +
                                                      std::to_string(tokens.size()) + " new tokens exceed " +
                                                      std::to_string(cache.max_ctx()));
  for (std::size_t i = 0; i < tokens.size(); ++i) {
    if (tokens[i] < 0 || static_cast<std::uint32_t>(tokens[i]) >= cfg_.n_vocab)
      return make_error(ErrorCode::InvalidArgument, "forward: token id " + std::to_string(tokens[i]) + " outside the vocabulary");
    rows_[at + i] = Row{tokens[i], static_cast<std::int32_t>(cache.pos() + i), cache.slot()};
  }
  return tokens.size();
}

Expected<std::span<const float>> LlamaModel::forward_prefill(KVCache& cache, std::span<const std::int32_t> tokens) {
  auto rows = prefill_rows(cache, tokens, 0);
  if (!rows) return rows.error();
  auto r = run(std::span<const Row>(rows_.data(), *rows), true);
  if (!r) return r.error();
  cache.advance(tokens.size());
  return std::span<const float>(logits_host_);
}

Expected<std::size_t> LlamaModel::forward_prefill_device(KVCache& cache, std::span<const std::int32_t> tokens) {
  auto rows = prefill_rows(cache, tokens, 0);
  if (!rows) return rows.error();
  auto r = run(std::span<const Row>(rows_.data(), *rows), false);
  if (!r) return r.error();
  cache.advance(tokens.size());
  return *r;
}

Expected<std::span<const float>> LlamaModel::forward_one(KVCache& cache, std::int32_t token) {
  return forward_prefill(cache, std::span<const std::int32_t>(&token, 1));
}

Expected<std::size_t> LlamaModel::batch_rows(std::span<KVCache* const> caches, std::span<const std::int32_t> tokens,
                                             std::size_t at) {
  // The checks of llama.cpp:269-302.
  if (caches.empty() || caches.size() != tokens.size())
    return make_error(ErrorCode::InvalidArgument, "forward_batch: " + std::to_string(caches.size()) + " caches for " +
                                                      std::to_string(tokens.size()) + " tokens");
  if (caches.size() > max_batch_)
    return make_error(ErrorCode::InvalidArgument, "forward_batch: " + std::to_string(caches.size()) +
                                                      " sequences exceed max_batch " + std::to_string(max_batch_));
  for (std::size_t i = 0; i < caches.size(); ++i) {
    const KVCache* cache = caches[i];
    if (cache == nullptr || cache->slot() < 0 || static_cast<std::size_t>(cache->slot()) >= n_slots_ ||
        cache->max_ctx() != max_ctx_)
      return make_error(ErrorCode::InvalidArgument, "forward_batch: cache " + std::to_string(i) + " was built for a different model");
    if (cache->pos() >= cache->max_ctx())
      return make_error(ErrorCode::InvalidArgument, "context overflow: cache " + std::to_string(i) + " holds " +
                                                        std::to_string(cache->pos()) + " of " +
                                                        std::to_string(cache->max_ctx()) + " positions");
    for (std::size_t j = 0; j < i; ++j) {
      if (caches[j] == cache || caches[j]->slot() == cache->slot())
        return make_error(ErrorCode::InvalidArgument, "forward_batch: cache " + std::to_string(i) + " appears twice");
    }
    if (tokens[i] < 0 || static_cast<std::uint32_t>(tokens[i]) >= cfg_.n_vocab)
      return make_error(ErrorCode::InvalidArgument, "forward: token id " + std::to_string(tokens[i]) + " outside the vocabulary");
    rows_[at + i] = Row{tokens[i], static_cast<std::int32_t>(cache->pos()), cache->slot()};
  }
  return tokens.size();
}

Expected<std::span<const float>> LlamaModel::forward_batch(std::span<KVCache* const> caches,
                                                           std::span<const std::int32_t> tokens) {
  auto rows = batch_rows(caches, tokens, 0);
  if (!rows) return rows.error();
  auto r = run(std::span<const Row>(rows_.data(), *rows), true);
  if (!r) return r.error();
  for (KVCache* cache : caches) cache->advance(1);
  return std::span<const float>(logits_host_);
}

Expected<std::size_t> LlamaModel::forward_batch_device(std::span<KVCache* const> caches,
                                                       std::span<const std::int32_t> tokens) {
  auto rows = batch_rows(caches, tokens, 0);
  if (!rows) return rows.error();
  auto r = run(std::span<const Row>(rows_.data(), *rows), false);
  if (!r) return r.error();
  for (KVCache* cache : caches) cache->advance(1);
  return *r;
}

Expected<std::size_t> LlamaModel::mixed_rows(KVCache* prefill, std::span<const std::int32_t> chunk,
                                             std::span<KVCache* const> caches, std::span<const std::int32_t> tokens) {
  if (chunk.empty() && tokens.empty()) return make_error(ErrorCode::InvalidArgument, "forward_mixed: no rows");
  std::size_t n = 0;
  if (!chunk.empty()) {
    if (prefill == nullptr || prefill->slot() < 0 || static_cast<std::size_t>(prefill->slot()) >= n_slots_ ||
        prefill->max_ctx() != max_ctx_)
      return make_error(ErrorCode::InvalidArgument, "forward_mixed: the prefill cache was built for a different model");
    for (KVCache* c : caches) {
      if (c == prefill || (c != nullptr && c->slot() == prefill->slot()))
        return make_error(ErrorCode::InvalidArgument, "forward_mixed: the prefill cache is also in the decode batch");
    }
    auto p = prefill_rows(*prefill, chunk, 0);
    if (!p) return p.error();
    n = *p;
  }
  if (!tokens.empty() || !caches.empty()) {
    auto b = batch_rows(caches, tokens, n);  // after the chunk: at most max_seq + max_batch rows
    if (!b) return b.error();
    n += *b;
  }
  return n;
}

Expected<std::span<const float>> LlamaModel::forward_mixed(KVCache* prefill, std::span<const std::int32_t> chunk,
                                                           std::span<KVCache* const> caches,
                                                           std::span<const std::int32_t> tokens) {
  auto rows = mixed_rows(prefill, chunk, caches, tokens);
  if (!rows) return rows.error();
  auto r = run(std::span<const Row>(rows_.data(), *rows), true, chunk.empty() ? 0 : chunk.size() - 1);
  if (!r) return r.error();
  if (!chunk.empty()) prefill->advance(chunk.size());
  for (KVCache* cache : caches) cache->advance(1);
  return std::span<const float>(logits_host_);
}

Expected<std::size_t> LlamaModel::forward_mixed_device(KVCache* prefill, std::span<const std::int32_t> chunk,
                                                       std::span<KVCache* const> caches,
                                                       std::span<const std::int32_t> tokens) {
  auto rows = mixed_rows(prefill, chunk, caches, tokens);
  if (!rows) return rows.error();
  auto r = run(std::span<const Row>(rows_.data(), *rows), false, chunk.empty() ? 0 : chunk.size() - 1);
  if (!r) return r.error();
  if (!chunk.empty()) prefill->advance(chunk.size());
  for (KVCache* cache : caches) cache->advance(1);
  return *r;
}

}  // namespace axon::model
