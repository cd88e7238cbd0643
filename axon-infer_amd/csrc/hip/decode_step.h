// The persistent decode-step kernel's launch descriptor (decode_step.hip).
#pragma once

#include <cstddef>
#include <cstdint>

namespace axon_hip {

// One layer's tensors (device pointers), laid out as the caller's array of layers.
struct StepLayer {
  const uint8_t* wq;
  const uint8_t* wk;
  const uint8_t* wv;
  const uint8_t* wo;
  const uint8_t* w_gate;
  const uint8_t* w_up;
  const uint8_t* w_down;
  const float* attn_norm;
  const float* ffn_norm;
  const float* bq;  // Q/K/V biases, all or none
  const float* bk;
  const float* bv;
  int64_t k_layer_off, v_layer_off;  // cache elements from the sequence's slot to the layer's K / V rows
};

struct StepShape {
  uint32_t n_layer, d, dq, dkv, ff, n_head, n_kv, rot_half;
  uint32_t max_ctx;              // positions of the caller's cache slots (bounds pos)
  int t_qkv, t_o, t_gu, t_down;  // weight types (Q8_0, Q4_0, Q4_1), the same in every layer
  int cache_f16;                 // the KV pool holds fp16 bit patterns (keys and values rounded once)
};

struct StepCall {
  const StepLayer* layers;  // device array of shape.n_layer records
  float eps, scale;
  const float* rope_table;  // [pos][rot_half] (cos, sin)
  float* x;                 // [d] residual stream, in and out
  float* cache;             // KV pool (float elements, or fp16 ones with shape.cache_f16)
  int64_t cache_off;        // the sequence's slot
  int32_t pos;              // the row's position: attention sees pos + 1 positions
  void* work;               // workspace of step_workspace_bytes
  uint64_t epoch;           // phases run on this workspace before the call
  uint32_t* status;         // pinned host word: 0, or why the kernel gave up
  uint32_t spin_limit;      // polls of one tagged word before giving up
  uint32_t fail_waits;      // test hook: nonzero, no wait ever sees its word written
  uint64_t* stamps;         // per-phase clock stamps (step_stamp_count words), or null
};

// Why a step kernel gave up (the status word): a word it waited for outlasted the poll limit.
constexpr uint32_t kStepTimedOut = 1;

size_t step_workspace_bytes(const StepShape& s);
// Words of a stamp buffer: 4 points x 5 phases x n_layer x one slot per CU (the grid may be
// smaller: 128 workgroups for a shape that fits them).
size_t step_stamp_count(const StepShape& s);
// 0 when this GPU runs the shape as one persistent kernel, else the reason (a static string).
const char* step_unsupported(const StepShape& s);
// Phases one call runs (each tags the words it writes with its own number).
uint64_t step_phases(const StepShape& s);
int step_launch(const StepShape& s, const StepCall& c);

}  // namespace axon_hip
