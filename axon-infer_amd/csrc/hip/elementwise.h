// Launchers of the row-wise kernels (elementwise.hip) and the attention kernels (attention.hip).
#pragma once

#include <cstddef>
#include <cstdint>

namespace axon_hip {

struct RopeRowsArgs {
  float* q;               // [rows][q_stride], n_head heads rotated in place (or null)
  float* k;               // [rows][k_stride], n_kv heads rotated in place (or null)
  float* v;               // [rows][k_stride], biased and copied to the cache (or null)
  const float* bq;        // biases (all three or none)
  const float* bk;
  const float* bv;
  const int32_t* pos;     // per-row position, or null for pos0 + row
  int32_t pos0;
  uint32_t q_stride, k_stride;
  uint32_t n_head, n_kv, head_dim, rotary_dim;
  int neox;
  float theta;
  const float* freq_factors;  // device, rotary_dim/2 divisors, or null
  const float* table;         // device cos/sin pairs [pos][rotary_dim/2], or null
  void* cache;                // KV pool base (or null: no cache write)
  const int64_t* cache_off;   // per-row element offset of the row's sequence in the pool
  int64_t k_layer_off, v_layer_off;  // element offsets of this layer's K and V regions
  int cache_f16;              // the pool holds fp16 bit patterns (rows rounded in once)
};

int quantize_rows_launch(const float* x, uint8_t* out, uint32_t n, uint32_t n_rows, uint32_t x_stride);
int rmsnorm_launch(const float* x, const float* w, float* y, uint8_t* yq, uint32_t n, uint32_t n_rows, float eps);
int silu_mul_launch(const float* gate, const float* up, float* out, uint8_t* outq, uint32_t n, uint32_t n_rows);
int softmax_launch(float* x, uint32_t n);
int add_launch(float* x, const float* y, size_t n);
// Greedy selection (sampling.hip). repeat_penalty rescales each row's distinct recent ids in
// place; argmax_rows takes the first maximum of each row, with argmax_scratch_words words of
// scratch.
int repeat_penalty_launch(float* x, uint32_t n, uint32_t n_rows, size_t stride, const int32_t* recent,
                          const uint32_t* recent_len, size_t recent_stride, float penalty);
size_t argmax_scratch_words(uint32_t n_rows);
// The k largest values of each row (k <= kMaxTopK), descending, equal values by ascending index,
// NaN skipped; out_logit/out_id [n_rows][k], id -1 past a row's non-NaN values.
constexpr uint32_t kMaxTopK = 256;
int topk_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, uint32_t k, float* out_logit,
                     int32_t* out_id);
// Every value of each row in the same order (out_logit/out_id [n_rows][n], NaN last with id -1),
// through a workspace of 8 * n * n_rows bytes.
int sort_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, void* work, float* out_logit,
                     int32_t* out_id);
int argmax_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, uint64_t* scratch, int32_t* out);
// argmax_rows over a fixed per-device array instead of a workspace (at most kArgmaxNoAllocRows rows);
// argmax_noalloc_setup finds the array's address on the current device (once per device).
constexpr uint32_t kArgmaxNoAllocRows = 512;
int argmax_noalloc_setup();
int argmax_rows_noalloc_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, int32_t* out);
int rope_rows_launch(const RopeRowsArgs& a, uint32_t n_rows);
int embedding_launch(int type, const uint8_t* table, uint32_t n, const int32_t* ids, int64_t id0, uint32_t n_rows,
                     float* out);
// The greedy id of one logits row x from n_parts partial keys (argmax_key), into *out_id, and that
// token's row of an embedding table of table_rows rows into emb[n].
int argmax_embed_launch(const float* x, const uint64_t* part, uint32_t n_parts, int32_t* out_id, int type,
                        const uint8_t* table, uint32_t table_rows, uint32_t n, float* emb);

// Attention over per-row KV spans. Row r reads its query at q + r * q_stride and attends over
// positions 0 .. n_vis(r) - 1 of K/V rows [pos][n_kv][head_dim] starting at
// kv + k_off(r) / kv + v_off(r) (elements). With per-row arrays null the constants apply and
// n_vis(r) = n_past + r + 1 (one sequence's prefill rows).
struct AttnArgs {
  const float* q;
  float* out;
  uint32_t q_stride, out_stride;
  const void* kv;            // float or fp16 elements
  const int64_t* k_off;      // per row (or null)
  const int64_t* v_off;
  const int32_t* n_vis;
  int64_t k_off_c, v_off_c;  // added to the per-row offsets (or used alone)
  int32_t n_past;
  uint32_t n_head, n_kv, head_dim;
  uint32_t head_begin, head_end;
  float scale;
  int f16;                   // cache holds fp16 bit patterns
  float* scratch;            // global score scratch when the scores do not fit LDS (or null)
  uint32_t max_vis;          // upper bound of n_vis over the rows
  int split;                 // decode-shaped launches may take the two-kernel path (scratch sized for it)
  uint8_t* outq;             // Q8_0 blocks of each output row as well (split path only), or null
};
int attention_launch(const AttnArgs& a, uint32_t n_rows);
// Floats of global scratch attention_launch needs for these rows (0 when LDS suffices).
size_t attention_scratch_floats(const AttnArgs& a, uint32_t n_rows);

}  // namespace axon_hip
