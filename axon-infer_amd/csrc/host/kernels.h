#pragma once

// The kernel-table interface of trickymind1324/axon-infer (src/kernels/kernels.h:18-146),
// restated so the hip table can be built and tested without the reference checkout, with one
// more member of KernelSet: Hip.
//
// Conventions as the reference states them: row-major and contiguous, weights [n_out][n_in] in
// GGUF layout. For the hip table every tensor pointer is a device pointer (HBM). Entries are
// asynchronous and stream-ordered: a later entry sees an earlier entry's output, and the host
// synchronizes (axon_hip_synchronize) before it reads device memory itself.

#include "expected.h"

#include <cstddef>
#include <cstdint>
#include <string_view>

namespace axon {

// ggml tensor type ids (src/core/dtype.h:17-49), the subset the table handles.
enum class DType : std::uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q8_0 = 8, Q6_K = 14, BF16 = 30 };

// GGUF block structs, byte-identical to src/core/dtype.h:85-120.
inline constexpr std::uint32_t kQK8_0 = 32;
inline constexpr std::uint32_t kQK_K = 256;
struct BlockQ8_0 { std::uint16_t d; std::int8_t qs[32]; };
struct BlockQ4_0 { std::uint16_t d; std::uint8_t qs[16]; };
struct BlockQ4_1 { std::uint16_t d; std::uint16_t m; std::uint8_t qs[16]; };
struct BlockQ6_K { std::uint8_t ql[128]; std::uint8_t qh[64]; std::int8_t scales[16]; std::uint16_t d; };
static_assert(sizeof(BlockQ8_0) == 34 && sizeof(BlockQ4_0) == 18 && sizeof(BlockQ4_1) == 20 &&
              sizeof(BlockQ6_K) == 210);

}  // namespace axon

namespace axon::kernels {

enum class RopeStyle : std::uint8_t { Normal, NeoX };

struct RopeParams {
  std::size_t head_dim;
  std::size_t rotary_dim;
  float theta;
  RopeStyle style;
  const float* freq_factors;  // nullptr, or rotary_dim/2 divisors of inv_freq (Llama 3.x)
};

// kernels.h:33-128, member for member.
struct KernelTable {
  void (*matmul_f32)(const float* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_f16)(const std::uint16_t* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_bf16)(const std::uint16_t* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_f32_rows)(const float* w, const float* x, float* y, std::size_t n_rows, std::size_t n_out,
                          std::size_t n_in, std::size_t y_stride);
  void (*matmul_f16_rows)(const std::uint16_t* w, const float* x, float* y, std::size_t n_rows,
                          std::size_t n_out, std::size_t n_in, std::size_t y_stride);
  void (*matmul_bf16_rows)(const std::uint16_t* w, const float* x, float* y, std::size_t n_rows,
                           std::size_t n_out, std::size_t n_in, std::size_t y_stride);
  void (*rmsnorm)(const float* x, const float* weight, float* y, std::size_t n, float eps);
  void (*rope)(float* x, std::size_t n_heads, std::size_t pos, const RopeParams& params);
  void (*softmax)(float* x, std::size_t n);
  void (*silu_mul)(const float* gate, const float* up, float* out, std::size_t n);
  void (*embedding_row)(DType type, const void* table, std::size_t n, std::int64_t index, float* out);
  void (*attention)(const float* q, const float* k, const float* v, float* out, float* scores, std::size_t seq,
                    std::size_t n_head, std::size_t n_head_kv, std::size_t head_dim, float scale);
  void (*attention_kv)(const float* q, const float* k_cache, const float* v_cache, float* out, float* scores,
                       std::size_t n_q, std::size_t n_past, std::size_t n_head, std::size_t n_head_kv,
                       std::size_t head_dim, float scale);
  void (*attention_kv_heads)(const float* q, const float* k_cache, const float* v_cache, float* out,
                             float* scores, std::size_t n_q, std::size_t n_past, std::size_t n_head,
                             std::size_t n_head_kv, std::size_t head_dim, float scale, std::size_t head_begin,
                             std::size_t head_end);
  void (*attention_kv_heads_f16)(const float* q, const std::uint16_t* k_cache, const std::uint16_t* v_cache,
                                 float* out, float* scores, std::size_t n_q, std::size_t n_past,
                                 std::size_t n_head, std::size_t n_head_kv, std::size_t head_dim, float scale,
                                 std::size_t head_begin, std::size_t head_end);
  void (*matmul_q8_0)(const BlockQ8_0* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q4_0)(const BlockQ4_0* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q8_0_q8)(const BlockQ8_0* w, const BlockQ8_0* xq, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q4_0_q8)(const BlockQ4_0* w, const BlockQ8_0* xq, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q8_0_rows)(const BlockQ8_0* w, const float* x, float* y, std::size_t n_rows, std::size_t n_out,
                           std::size_t n_in, std::size_t y_stride);
  void (*matmul_q4_0_rows)(const BlockQ4_0* w, const float* x, float* y, std::size_t n_rows, std::size_t n_out,
                           std::size_t n_in, std::size_t y_stride);
  void (*matmul_q8_0_q8_rows)(const BlockQ8_0* w, const BlockQ8_0* xq, float* y, std::size_t n_rows,
                              std::size_t n_out, std::size_t n_in, std::size_t y_stride);
  void (*matmul_q4_0_q8_rows)(const BlockQ4_0* w, const BlockQ8_0* xq, float* y, std::size_t n_rows,
                              std::size_t n_out, std::size_t n_in, std::size_t y_stride);
  void (*quantize_row_q8_0)(const float* x, BlockQ8_0* out, std::size_t n);
  void (*matmul_q4_1)(const BlockQ4_1* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q4_1_q8)(const BlockQ4_1* w, const BlockQ8_0* xq, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q4_1_rows)(const BlockQ4_1* w, const float* x, float* y, std::size_t n_rows, std::size_t n_out,
                           std::size_t n_in, std::size_t y_stride);
  void (*matmul_q4_1_q8_rows)(const BlockQ4_1* w, const BlockQ8_0* xq, float* y, std::size_t n_rows,
                              std::size_t n_out, std::size_t n_in, std::size_t y_stride);
  void (*matmul_q6_k)(const BlockQ6_K* w, const float* x, float* y, std::size_t n_out, std::size_t n_in);
  void (*matmul_q6_k_rows)(const BlockQ6_K* w, const float* x, float* y, std::size_t n_rows, std::size_t n_out,
                           std::size_t n_in, std::size_t y_stride);
};

// kernels.h:135 plus Hip. This library builds the hip table only: Scalar and Neon are the
// reference's own tables and stay in its build.
enum class KernelSet : std::uint8_t { Auto, Scalar, Neon, Hip };

// The hip table (device pointers). Calling it on a host without a gfx950 device aborts, so
// obtain it through select(), which checks.
const KernelTable& hip_kernels();

// kernels.h:137-140: the table for a set, or Unsupported; never a silent fallback. Hip and
// Auto initialise device 0 and return the hip table when a gfx950 device answers.
Expected<const KernelTable*> select(KernelSet set);
// "hip" for the hip table, "custom" for anything else (kernels.cpp:105-112).
std::string_view name(const KernelTable& table);
// "auto", "scalar", "neon" or "hip" (kernels.cpp:114-126).
bool parse_kernel_set(std::string_view text, KernelSet& out);

}  // namespace axon::kernels
