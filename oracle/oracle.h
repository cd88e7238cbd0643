/*
 * TEST INFRASTRUCTURE ONLY. This is the CPU oracle: a plain-C restatement of the
 * reference scalar kernel table (trickymind1324/axon-infer, src/kernels/ref/ and
 * src/core/dtype.cpp) and of the forward pass that drives it (src/model/llama.cpp).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker. The product (libaxon_hip.so, libaxon_host.so) never links it.
 *
 * Every reduction runs in the reference's order (sequential, float, no contraction), so
 * with gcc -ffp-contract=off on x86-64 the outputs are the reference scalar table's bits.
 *
 * Parity pinning, per function (see tests/test_oracle_*.py):
 *   fp16/bf16 conversions ... exhaustive round trip + reference fixtures (kernels: embedding, matmul f16 and bf16)
 *   dequantize_* ............ fixtures quant/row.*.dequant, embedding_*.rows (bit-exact)
 *   quantize_row_q8_0 ....... fixtures quant/row.q8_0.bin, act.q8_0.bin (byte-exact)
 *   matmul_*_q8 ............. fixtures quant/matmul_*.yq/.ysq + closed-form single block
 *   matmul_q6_k ............. fixtures quant/matmul_q6_k.y/.ys
 *   float matmuls ........... fixtures kernels/matmul_*.y
 *   rmsnorm/softmax/silu .... fixtures kernels/rmsnorm_*, softmax_*, silu_mul
 *   rope .................... fixtures kernels/rope_{normal,neox,llama3}
 *   attention ............... fixtures kernels/attention_*, GQA==MHA, one-position identity
 *   model forward ........... fixtures model/synthetic-2l*.logits (F32 GGUF, 1e-4) and
 *                             the reference's own LlamaModel built under oracle/_ref
 *   all table entries ....... bit-exact against the reference's own scalar table (oracle/_ref)
 *   sampler (rng, penalty, greedy, top-k/top-p/min-p draws) ... the reference's sampler test
 *                             cases (test_sampler.cpp:35-135), np.argmax (first maximum) on NaN-free
 *                             rows, hand-worked NaN rows, and the reference's own Sampler
 *                             (oracle/_ref) draw for draw on random rows, windows and seeds
 */
#ifndef AXON_ORACLE_H
#define AXON_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Block layouts, byte-identical to src/core/dtype.h:85-120. */
#define ORA_QK 32
#define ORA_QK_K 256
typedef struct { uint16_t d; int8_t qs[32]; } ora_block_q8_0;               /* 34 B */
typedef struct { uint16_t d; uint8_t qs[16]; } ora_block_q4_0;              /* 18 B */
typedef struct { uint16_t d; uint16_t m; uint8_t qs[16]; } ora_block_q4_1;  /* 20 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } ora_block_q6_k; /* 210 B */

/* ggml type ids (src/core/dtype.h:17-49), the subset the table handles. */
enum { ORA_F32 = 0, ORA_F16 = 1, ORA_Q4_0 = 2, ORA_Q4_1 = 3, ORA_Q8_0 = 8, ORA_Q6_K = 14, ORA_BF16 = 30 };

float ora_fp16_to_fp32(uint16_t bits);
uint16_t ora_fp32_to_fp16(float value);
float ora_bf16_to_fp32(uint16_t bits);
uint16_t ora_fp32_to_bf16(float value);

void ora_dequantize_block_q8_0(const ora_block_q8_0* b, float* out);
void ora_dequantize_block_q4_0(const ora_block_q4_0* b, float* out);
void ora_dequantize_block_q4_1(const ora_block_q4_1* b, float* out);
void ora_dequantize_block_q6_k(const ora_block_q6_k* b, float* out);
void ora_quantize_row_q8_0(const float* x, ora_block_q8_0* out, size_t n);

/* The 30 KernelTable entries (src/kernels/kernels.h:33-128), same argument order. */
void ora_matmul_f32(const float* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_f16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_bf16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_f32_rows(const float* w, const float* x, float* y, size_t n_rows, size_t n_out,
                         size_t n_in, size_t y_stride);
void ora_matmul_f16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                         size_t n_in, size_t y_stride);
void ora_matmul_bf16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                          size_t n_in, size_t y_stride);
void ora_rmsnorm(const float* x, const float* weight, float* y, size_t n, float eps);
/* style 0 = Normal, 1 = NeoX; freq_factors may be NULL */
void ora_rope(float* x, size_t n_heads, size_t pos, size_t head_dim, size_t rotary_dim, float theta,
              int style, const float* freq_factors);
void ora_softmax(float* x, size_t n);
void ora_silu_mul(const float* gate, const float* up, float* out, size_t n);
void ora_embedding_row(int type, const void* table, size_t n, int64_t index, float* out);
void ora_attention(const float* q, const float* k, const float* v, float* out, float* scores,
                   size_t seq, size_t n_head, size_t n_head_kv, size_t head_dim, float scale);
void ora_attention_kv(const float* q, const float* k_cache, const float* v_cache, float* out,
                      float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                      size_t head_dim, float scale);
void ora_attention_kv_heads(const float* q, const float* k_cache, const float* v_cache, float* out,
                            float* scores, size_t n_q, size_t n_past, size_t n_head,
                            size_t n_head_kv, size_t head_dim, float scale, size_t head_begin,
                            size_t head_end);
void ora_attention_kv_heads_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                float* out, float* scores, size_t n_q, size_t n_past, size_t n_head,
                                size_t n_head_kv, size_t head_dim, float scale, size_t head_begin,
                                size_t head_end);
void ora_matmul_q8_0(const ora_block_q8_0* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_q4_0(const ora_block_q4_0* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_q8_0_q8(const ora_block_q8_0* w, const ora_block_q8_0* xq, float* y, size_t n_out,
                        size_t n_in);
void ora_matmul_q4_0_q8(const ora_block_q4_0* w, const ora_block_q8_0* xq, float* y, size_t n_out,
                        size_t n_in);
void ora_matmul_q8_0_rows(const ora_block_q8_0* w, const float* x, float* y, size_t n_rows,
                          size_t n_out, size_t n_in, size_t y_stride);
void ora_matmul_q4_0_rows(const ora_block_q4_0* w, const float* x, float* y, size_t n_rows,
                          size_t n_out, size_t n_in, size_t y_stride);
void ora_matmul_q8_0_q8_rows(const ora_block_q8_0* w, const ora_block_q8_0* xq, float* y,
                             size_t n_rows, size_t n_out, size_t n_in, size_t y_stride);
void ora_matmul_q4_0_q8_rows(const ora_block_q4_0* w, const ora_block_q8_0* xq, float* y,
                             size_t n_rows, size_t n_out, size_t n_in, size_t y_stride);
void ora_matmul_q4_1(const ora_block_q4_1* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_q4_1_q8(const ora_block_q4_1* w, const ora_block_q8_0* xq, float* y, size_t n_out,
                        size_t n_in);
void ora_matmul_q4_1_rows(const ora_block_q4_1* w, const float* x, float* y, size_t n_rows,
                          size_t n_out, size_t n_in, size_t y_stride);
void ora_matmul_q4_1_q8_rows(const ora_block_q4_1* w, const ora_block_q8_0* xq, float* y,
                             size_t n_rows, size_t n_out, size_t n_in, size_t y_stride);
void ora_matmul_q6_k(const ora_block_q6_k* w, const float* x, float* y, size_t n_out, size_t n_in);
void ora_matmul_q6_k_rows(const ora_block_q6_k* w, const float* x, float* y, size_t n_rows,
                          size_t n_out, size_t n_in, size_t y_stride);

/* Per-block int32 dot sums of one weight row against one Q8_0 activation row: the integer
 * phase of matmul_*_q8 (src/kernels/ref/quant.cpp:47-50, 59-65, 166-175), exposed so the
 * HIP table's test hook can be compared block by block. type is ORA_Q8_0/Q4_0/Q4_1; for
 * Q4_1 sumx (the activation's integer sum per block) is written too when non-NULL. */
void ora_block_sums(int type, const void* w_row, const ora_block_q8_0* xq, size_t n_blocks,
                    int32_t* sumi, int32_t* sumx);

/* ---- Forward pass restated from src/model/llama.cpp:315-639 (single thread) ---------- */

typedef struct {
  const void* data;  /* host pointer into the mapped GGUF */
  int type;          /* ORA_* */
  uint64_t ne0, ne1; /* n_in, n_out */
} ora_tensor;

typedef struct {
  ora_tensor attn_norm, wq, wk, wv, wo, ffn_norm, w_gate, w_up, w_down;
  ora_tensor bq, bk, bv; /* data == NULL when absent */
} ora_layer;

typedef struct {
  uint32_t n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab, head_dim, rotary_dim;
  float rope_theta, rms_eps;
  int rope_style;          /* 0 Normal (llama), 1 NeoX (qwen2) */
  int exact_activations;   /* 1: float-activation paths for quantized weights */
  ora_tensor token_embd, output_norm, output;
  const float* rope_freqs; /* NULL unless llama3 scaling */
  const ora_layer* layers;
} ora_model;

/* A per-sequence cache, laid out as src/model/kv_cache.cpp:15-18: layer l's K rows at
 * base + (2l) * max_ctx * row, V rows at base + (2l+1) * max_ctx * row (elements). f16 == 0:
 * float elements (CacheType::F32); f16 == 1: fp16 bit patterns (CacheType::F16,
 * src/model/kv_cache.h:34-43). The caches of one forward_batch call share one type. */
typedef struct {
  void* base;
  size_t max_ctx;
  size_t pos;
  int f16;
} ora_cache;

/* Scratch sized by ora_workspace_floats(model, n_tokens, ctx). */
size_t ora_workspace_floats(const ora_model* m, size_t n_tokens, size_t ctx);

/* forward_prefill (cache != NULL) or the cache-free forward (cache == NULL): tokens at
 * positions cache->pos ..; logits [n_tokens][n_vocab]. Returns 0 or a negative error. */
int ora_forward(const ora_model* m, const int32_t* tokens, size_t n_tokens, ora_cache* cache,
                float* workspace, float* logits);
/* forward_batch: tokens[i] appended to caches[i] at its own position; logits [n][n_vocab]. */
int ora_forward_batch(const ora_model* m, const int32_t* tokens, size_t n, ora_cache* const* caches,
                      float* workspace, float* logits);

/* ---- Sampler restated from src/sampling/sampler.cpp and src/sampling/rng.h ------------- */
typedef struct { uint64_t s[4]; } ora_rng;
void ora_rng_seed(ora_rng* r, uint64_t seed);
uint64_t ora_rng_next(ora_rng* r);
double ora_rng_uniform(ora_rng* r);

typedef struct {
  float temperature;
  int top_k;
  float top_p;
  float min_p;
  float repeat_penalty;
  int repeat_last_n;
} ora_sampler_config;

/* One draw. scratch_* hold n_vocab entries each. */
int32_t ora_sample(const ora_sampler_config* c, ora_rng* rng, const float* logits, int32_t n_vocab,
                   const int32_t* recent, size_t n_recent, float* scratch_logits,
                   int32_t* scratch_order, double* scratch_probs, uint8_t* scratch_touched);

/* The repetition penalty alone (sampler.cpp:73-97), in place on n logits: each distinct id in
 * [0, n) of the last min(n_recent, repeat_last_n) ids, once, when penalty != 1 and
 * repeat_last_n > 0. touched: n zeroed bytes, left zeroed. ora_sample runs it first. */
void ora_repeat_penalty(float* logits, size_t n, const int32_t* recent, size_t n_recent, float penalty,
                        int repeat_last_n, uint8_t* touched);

#ifdef __cplusplus
}
#endif
#endif
