/*
 * TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h). The forward pass restated from
 * src/model/llama.cpp:315-639 and the sampler from src/sampling/sampler.cpp:66-183. Single
 * threaded: the reference splits columns and heads across threads so that no reduction ever
 * crosses a thread (llama.cpp:310-314), which makes one thread give the same bits.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static size_t max3(size_t a, size_t b, size_t c) {
  size_t m = a > b ? a : b;
  return m > c ? m : c;
}

/* Floats per activation buffer, as src/model/activations.h:36-55 lays them out. */
typedef struct {
  float *x, *h, *q, *k, *v, *attn, *gate, *up, *scores;
  ora_block_q8_0* xq;
} acts;

size_t ora_workspace_floats(const ora_model* m, size_t seq, size_t ctx) {
  const size_t d = m->n_embd, dq = (size_t)m->n_head * m->head_dim;
  const size_t dkv = (size_t)m->n_head_kv * m->head_dim, ff = m->n_ff;
  const size_t widest = max3(d, dq, ff);
  const size_t xq_bytes = seq * (widest / 32) * sizeof(ora_block_q8_0);
  return seq * (2 * d + 2 * dq + 2 * dkv + 2 * ff + ctx) + (xq_bytes + 3) / 4 + 16;
}

static acts carve(const ora_model* m, float* ws, size_t seq, size_t ctx) {
  const size_t d = m->n_embd, dq = (size_t)m->n_head * m->head_dim;
  const size_t dkv = (size_t)m->n_head_kv * m->head_dim, ff = m->n_ff;
  acts a;
  a.x = ws; ws += seq * d;
  a.h = ws; ws += seq * d;
  a.q = ws; ws += seq * dq;
  a.k = ws; ws += seq * dkv;
  a.v = ws; ws += seq * dkv;
  a.attn = ws; ws += seq * dq;
  a.gate = ws; ws += seq * ff;
  a.up = ws; ws += seq * ff;
  a.scores = ws; ws += seq * ctx;
  a.xq = (ora_block_q8_0*)ws;
  return a;
}

static int needs_q8(const ora_model* m, const ora_tensor* w) {
  return !m->exact_activations && (w->type == ORA_Q8_0 || w->type == ORA_Q4_0 || w->type == ORA_Q4_1);
}

static size_t row_bytes(const ora_tensor* w) {
  switch (w->type) {
  case ORA_F32: return w->ne0 * 4;
  case ORA_F16: case ORA_BF16: return w->ne0 * 2;
  case ORA_Q8_0: return w->ne0 / 32 * 34;
  case ORA_Q4_0: return w->ne0 / 32 * 18;
  case ORA_Q4_1: return w->ne0 / 32 * 20;
  case ORA_Q6_K: return w->ne0 / 256 * 210;
  default: return 0;
  }
}

/* llama.cpp:30-101 matmul_columns over every column: rows are independent, and the _rows
 * entries are the single-row entries looped (ref/quant.cpp:111-139), so one row at a time. */
static void matmul(const ora_model* m, const ora_tensor* w, const float* x, const ora_block_q8_0* xq,
                   float* y, size_t n_rows, size_t y_stride) {
  const size_t n_in = w->ne0, n_out = w->ne1, nb = n_in / 32;
  const int exact = m->exact_activations;
  (void)row_bytes;
  for (size_t r = 0; r < n_rows; ++r) {
    const float* xr = x + r * n_in;
    const ora_block_q8_0* xqr = xq != NULL ? xq + r * nb : NULL;
    float* yr = y + r * y_stride;
    switch (w->type) {
    case ORA_F32: ora_matmul_f32(w->data, xr, yr, n_out, n_in); break;
    case ORA_F16: ora_matmul_f16(w->data, xr, yr, n_out, n_in); break;
    case ORA_BF16: ora_matmul_bf16(w->data, xr, yr, n_out, n_in); break;
    case ORA_Q8_0:
      if (exact) ora_matmul_q8_0(w->data, xr, yr, n_out, n_in);
      else ora_matmul_q8_0_q8(w->data, xqr, yr, n_out, n_in);
      break;
    case ORA_Q4_0:
      if (exact) ora_matmul_q4_0(w->data, xr, yr, n_out, n_in);
      else ora_matmul_q4_0_q8(w->data, xqr, yr, n_out, n_in);
      break;
    case ORA_Q4_1:
      if (exact) ora_matmul_q4_1(w->data, xr, yr, n_out, n_in);
      else ora_matmul_q4_1_q8(w->data, xqr, yr, n_out, n_in);
      break;
    case ORA_Q6_K: ora_matmul_q6_k(w->data, xr, yr, n_out, n_in); break;
    default: break;
    }
  }
}

/* llama.cpp:401-417: the input is quantized once per launch that feeds quantized weights. */
static int quantize_input(const ora_model* m, const float* x, const ora_tensor* w, size_t seq,
                          ora_block_q8_0* xq) {
  if (!needs_q8(m, w)) return 0;
  const size_t n_in = w->ne0, nb = n_in / 32;
  for (size_t r = 0; r < seq; ++r) ora_quantize_row_q8_0(x + r * n_in, xq + r * nb, n_in);
  return 1;
}

/* mm_fused (llama.cpp:433-468): every segment reads the same input, quantized at most once. */
static void mm_fused(const ora_model* m, const ora_tensor* const* ws, float* const* ys, size_t n_seg,
                     const float* x, size_t seq, ora_block_q8_0* xq) {
  int quantized = 0;
  for (size_t s = 0; s < n_seg && !quantized; ++s) quantized = quantize_input(m, x, ws[s], seq, xq);
  for (size_t s = 0; s < n_seg; ++s) {
    matmul(m, ws[s], x, quantized ? xq : NULL, ys[s], seq, ws[s]->ne1);
  }
}

static void mm(const ora_model* m, const ora_tensor* w, const float* x, float* y, size_t seq,
               ora_block_q8_0* xq) {
  const ora_tensor* one[1] = {w};
  float* out[1] = {y};
  mm_fused(m, one, out, 1, x, seq, xq);
}

static void add_bias(float* rows, const ora_tensor* bias, size_t n_rows) {
  const float* b = bias->data;
  const size_t n = bias->ne0;
  for (size_t r = 0; r < n_rows; ++r)
    for (size_t i = 0; i < n; ++i) rows[r * n + i] += b[i];
}

static void add_rows(float* x, const float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] += y[i];
}

static void rmsnorm_rows(const ora_model* m, const float* x, const ora_tensor* w, float* out,
                         size_t seq) {
  const size_t n = w->ne0;
  for (size_t r = 0; r < seq; ++r) ora_rmsnorm(x + r * n, w->data, out + r * n, n, m->rms_eps);
}

static size_t cache_at(const ora_model* m, const ora_cache* c, size_t l, int values) {
  return (2 * l + (size_t)values) * c->max_ctx * ((size_t)m->n_head_kv * m->head_dim);
}
static float* cache_k(const ora_model* m, ora_cache* c, size_t l) { return (float*)c->base + cache_at(m, c, l, 0); }
static float* cache_v(const ora_model* m, ora_cache* c, size_t l) { return (float*)c->base + cache_at(m, c, l, 1); }
static uint16_t* cache_k16(const ora_model* m, ora_cache* c, size_t l) {
  return (uint16_t*)c->base + cache_at(m, c, l, 0);
}
static uint16_t* cache_v16(const ora_model* m, ora_cache* c, size_t l) {
  return (uint16_t*)c->base + cache_at(m, c, l, 1);
}

/* llama.cpp:525-532, 559-563: rows of float keys and values rounded once into an fp16 cache. */
static void round_in(uint16_t* dst, const float* src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = ora_fp32_to_fp16(src[i]);
}

/* The one forward pass, llama.cpp:315-639. batch != NULL is forward_batch: row i is its own
 * sequence at batch[i]->pos. Otherwise cache may be NULL (cache-free reference pass). */
static int run(const ora_model* m, const int32_t* tokens, size_t seq, ora_cache* cache,
               ora_cache* const* batch, float* ws, float* logits) {
  if (seq == 0) return -1;
  for (size_t i = 0; i < seq; ++i)
    if (tokens[i] < 0 || (uint32_t)tokens[i] >= m->n_vocab) return -2;
  const size_t n_past = cache != NULL ? cache->pos : 0;
  if (cache != NULL && n_past + seq > cache->max_ctx) return -3;
  const size_t d = m->n_embd, hd = m->head_dim, nh = m->n_head, nkv = m->n_head_kv;
  const size_t kv_row = nkv * hd, q_row = nh * hd;
  size_t total = n_past + seq;
  if (batch != NULL) {
    total = 0;
    for (size_t i = 0; i < seq; ++i) {
      if (batch[i]->pos >= batch[i]->max_ctx) return -3;
      if (batch[i]->pos + 1 > total) total = batch[i]->pos + 1;
    }
  }
  /* llama.cpp:381-382: an fp16 cache stages the new keys and values in float (a.k, a.v). */
  const int half_cache = (cache != NULL && cache->f16) || (batch != NULL && batch[0]->f16);
  if (batch != NULL)
    for (size_t i = 0; i < seq; ++i)
      if (batch[i]->f16 != batch[0]->f16) return -4;
  acts a = carve(m, ws, seq, total);
  const float scale = 1.0f / sqrtf((float)hd);

  for (size_t i = 0; i < seq; ++i)
    ora_embedding_row(m->token_embd.type, m->token_embd.data, d, tokens[i], a.x + i * d);

  for (size_t l = 0; l < m->n_layer; ++l) {
    const ora_layer* w = &m->layers[l];
    const int direct = cache != NULL && !half_cache;
    float* k_base = direct ? cache_k(m, cache, l) : a.k;
    float* v_base = direct ? cache_v(m, cache, l) : a.v;
    float* k_new = direct ? k_base + n_past * kv_row : a.k;
    float* v_new = direct ? v_base + n_past * kv_row : a.v;

    rmsnorm_rows(m, a.x, &w->attn_norm, a.h, seq);
    {
      const ora_tensor* qkv[3] = {&w->wq, &w->wk, &w->wv};
      float* outs[3] = {a.q, k_new, v_new};
      mm_fused(m, qkv, outs, 3, a.h, seq, a.xq);
    }
    if (w->bq.data != NULL && w->bk.data != NULL && w->bv.data != NULL) {
      add_bias(a.q, &w->bq, seq);
      add_bias(k_new, &w->bk, seq);
      add_bias(v_new, &w->bv, seq);
    }
    for (size_t i = 0; i < seq; ++i) {
      const size_t pos = batch != NULL ? batch[i]->pos : n_past + i;
      ora_rope(a.q + i * q_row, nh, pos, hd, m->rotary_dim, m->rope_theta, m->rope_style, m->rope_freqs);
      ora_rope(k_new + i * kv_row, nkv, pos, hd, m->rotary_dim, m->rope_theta, m->rope_style,
               m->rope_freqs);
    }
    if (batch != NULL) {
      /* llama.cpp:520-556: each row's key and value into its own cache, then one call per
       * (sequence, head) over that cache. */
      for (size_t i = 0; i < seq; ++i) {
        ora_cache* c = batch[i];
        if (half_cache) {
          round_in(cache_k16(m, c, l) + c->pos * kv_row, k_new + i * kv_row, kv_row);
          round_in(cache_v16(m, c, l) + c->pos * kv_row, v_new + i * kv_row, kv_row);
        } else {
          memcpy(cache_k(m, c, l) + c->pos * kv_row, k_new + i * kv_row, kv_row * sizeof(float));
          memcpy(cache_v(m, c, l) + c->pos * kv_row, v_new + i * kv_row, kv_row * sizeof(float));
        }
      }
      for (size_t b = 0; b < seq; ++b) {
        ora_cache* c = batch[b];
        for (size_t h = 0; h < nh; ++h) {
          if (half_cache)
            ora_attention_kv_heads_f16(a.q + b * q_row, cache_k16(m, c, l), cache_v16(m, c, l),
                                       a.attn + b * q_row, a.scores, 1, c->pos, nh, nkv, hd, scale, h, h + 1);
          else
            ora_attention_kv_heads(a.q + b * q_row, cache_k(m, c, l), cache_v(m, c, l), a.attn + b * q_row,
                                   a.scores, 1, c->pos, nh, nkv, hd, scale, h, h + 1);
        }
      }
    } else if (half_cache) {
      /* llama.cpp:557-563 then 566-590: the chunk's rows rounded in, then every row attends over
       * the fp16 cache. */
      round_in(cache_k16(m, cache, l) + n_past * kv_row, k_new, seq * kv_row);
      round_in(cache_v16(m, cache, l) + n_past * kv_row, v_new, seq * kv_row);
      for (size_t h = 0; h < nh; ++h) {
        ora_attention_kv_heads_f16(a.q, cache_k16(m, cache, l), cache_v16(m, cache, l), a.attn, a.scores, seq,
                                   n_past, nh, nkv, hd, scale, h, h + 1);
      }
    } else {
      /* llama.cpp:566-590: rows are computed independently, so all rows in one call. */
      for (size_t h = 0; h < nh; ++h) {
        ora_attention_kv_heads(a.q, k_base, v_base, a.attn, a.scores, seq, n_past, nh, nkv, hd, scale,
                               h, h + 1);
      }
    }
    mm(m, &w->wo, a.attn, a.h, seq, a.xq);
    add_rows(a.x, a.h, seq * d);

    rmsnorm_rows(m, a.x, &w->ffn_norm, a.h, seq);
    {
      /* llama.cpp:600-620: gate and up from one quantized input, SiLU product in place. */
      const int quantized = quantize_input(m, a.h, &w->w_gate, seq, a.xq);
      matmul(m, &w->w_gate, a.h, quantized ? a.xq : NULL, a.gate, seq, m->n_ff);
      matmul(m, &w->w_up, a.h, quantized ? a.xq : NULL, a.up, seq, m->n_ff);
      for (size_t r = 0; r < seq; ++r)
        ora_silu_mul(a.gate + r * m->n_ff, a.up + r * m->n_ff, a.gate + r * m->n_ff, m->n_ff);
    }
    mm(m, &w->w_down, a.gate, a.h, seq, a.xq);
    add_rows(a.x, a.h, seq * d);
  }
  rmsnorm_rows(m, a.x, &m->output_norm, a.h, seq);
  mm(m, &m->output, a.h, logits, seq, a.xq);
  if (cache != NULL) cache->pos += seq;
  if (batch != NULL)
    for (size_t i = 0; i < seq; ++i) batch[i]->pos += 1;
  return 0;
}

int ora_forward(const ora_model* m, const int32_t* tokens, size_t n_tokens, ora_cache* cache,
                float* workspace, float* logits) {
  return run(m, tokens, n_tokens, cache, NULL, workspace, logits);
}

int ora_forward_batch(const ora_model* m, const int32_t* tokens, size_t n, ora_cache* const* caches,
                      float* workspace, float* logits) {
  return run(m, tokens, n, NULL, caches, workspace, logits);
}

/* ---- sampler: src/sampling/rng.h:11-45, src/sampling/sampler.cpp:69-183 ------------------ */

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void ora_rng_seed(ora_rng* r, uint64_t seed) {
  uint64_t x = seed;
  for (int i = 0; i < 4; ++i) {
    x += 0x9E3779B97F4A7C15ULL;
    uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    r->s[i] = z ^ (z >> 31);
  }
}

uint64_t ora_rng_next(ora_rng* r) {
  uint64_t* s = r->s;
  const uint64_t result = rotl64(s[1] * 5, 7) * 9;
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return result;
}

double ora_rng_uniform(ora_rng* r) { return (double)(ora_rng_next(r) >> 11) * 0x1.0p-53; }

static const float* g_sort_logits;
/* Descending by logit; equal logits by ascending id. The reference's std::partial_sort leaves
 * equal logits in an unspecified order, so only tie-free logit rows are comparable. */
static int by_logit_desc(const void* pa, const void* pb) {
  const int32_t a = *(const int32_t*)pa, b = *(const int32_t*)pb;
  const float la = g_sort_logits[a], lb = g_sort_logits[b];
  if (la > lb) return -1;
  if (la < lb) return 1;
  return a < b ? -1 : (a > b);
}

void ora_repeat_penalty(float* sl, size_t n, const int32_t* recent, size_t n_recent, float penalty,
                        int repeat_last_n, uint8_t* touched) {
  if (penalty == 1.0f || repeat_last_n <= 0 || n_recent == 0) return;
  const size_t window = n_recent < (size_t)repeat_last_n ? n_recent : (size_t)repeat_last_n;
  const int32_t* tail = recent + (n_recent - window);
  for (size_t t = 0; t < window; ++t) {
    const int32_t id = tail[t];
    if (id < 0 || (size_t)id >= n || touched[id]) continue;
    touched[id] = 1;
    float* logit = &sl[id];
    *logit = *logit > 0.0f ? *logit / penalty : *logit * penalty;
  }
  for (size_t t = 0; t < window; ++t)
    if (tail[t] >= 0 && (size_t)tail[t] < n) touched[tail[t]] = 0;
}

int32_t ora_sample(const ora_sampler_config* c, ora_rng* rng, const float* logits, int32_t n_vocab,
                   const int32_t* recent, size_t n_recent, float* sl, int32_t* order, double* probs,
                   uint8_t* touched) {
  const size_t n = (size_t)n_vocab;
  memcpy(sl, logits, n * sizeof(float));
  ora_repeat_penalty(sl, n, recent, n_recent, c->repeat_penalty, c->repeat_last_n, touched);
  if (c->temperature <= 0.0f) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
      if (sl[i] > sl[best]) best = i; /* max_element: first of equal maxima */
    return (int32_t)best;
  }
  for (size_t i = 0; i < n; ++i) order[i] = (int32_t)i;
  g_sort_logits = sl;
  qsort(order, n, sizeof(int32_t), by_logit_desc);
  size_t kept = n;
  if (c->top_k > 0 && (size_t)c->top_k < n) kept = (size_t)c->top_k;
  const double max_logit = (double)sl[order[0]];
  const double temperature = (double)c->temperature;
  double sum = 0.0;
  for (size_t i = 0; i < kept; ++i) {
    probs[i] = exp(((double)sl[order[i]] - max_logit) / temperature);
    sum += probs[i];
  }
  for (size_t i = 0; i < kept; ++i) probs[i] /= sum;
  if (c->top_p < 1.0f) {
    double cumulative = 0.0;
    size_t cut = kept;
    for (size_t i = 0; i < kept; ++i) {
      cumulative += probs[i];
      if (cumulative >= (double)c->top_p) { cut = i + 1; break; }
    }
    kept = cut;
  }
  if (c->min_p > 0.0f) {
    const double floor_p = (double)c->min_p * probs[0];
    size_t cut = kept;
    for (size_t i = 1; i < kept; ++i)
      if (probs[i] < floor_p) { cut = i; break; }
    kept = cut;
  }
  double remaining = 0.0;
  for (size_t i = 0; i < kept; ++i) remaining += probs[i];
  const double u = ora_rng_uniform(rng) * remaining;
  double cumulative = 0.0;
  for (size_t i = 0; i < kept; ++i) {
    cumulative += probs[i];
    if (u < cumulative) return order[i];
  }
  return order[kept - 1];
}
