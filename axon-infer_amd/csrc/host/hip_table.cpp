// The hip KernelTable: one thunk per entry of src/kernels/kernels.h:33-128 that forwards to the
// C ABI of libaxon_hip.so. Table entries cannot fail in the reference (preconditions are
// checks that abort, src/kernels/ref/embedding.cpp:61-62), so a non-zero status aborts here
// with the library's message, the same contract.

#include "kernels.h"

#include "axon_hip.h"

#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

namespace axon::kernels {

namespace {

void must(int rc, const char* entry) {
  if (rc != AXON_HIP_OK) {
    std::fprintf(stderr, "axon hip table: %s failed (%d): %s\n", entry, rc, axon_hip_last_error());
    std::abort();
  }
}

#define FWD(entry, ...) must(axon_hip_##entry(__VA_ARGS__), #entry)

void matmul_f32(const float* w, const float* x, float* y, std::size_t n_out, std::size_t n_in) {
  FWD(matmul_f32, w, x, y, n_out, n_in);
}
void matmul_f16(const std::uint16_t* w, const float* x, float* y, std::size_t n_out, std::size_t n_in) {
  FWD(matmul_f16, w, x, y, n_out, n_in);
}
void matmul_bf16(const std::uint16_t* w, const float* x, float* y, std::size_t n_out, std::size_t n_in) {
  FWD(matmul_bf16, w, x, y, n_out, n_in);
}
void matmul_f32_rows(const float* w, const float* x, float* y, std::size_t r, std::size_t o, std::size_t i,
                     std::size_t s) {
  FWD(matmul_f32_rows, w, x, y, r, o, i, s);
}
void matmul_f16_rows(const std::uint16_t* w, const float* x, float* y, std::size_t r, std::size_t o, std::size_t i,
                     std::size_t s) {
  FWD(matmul_f16_rows, w, x, y, r, o, i, s);
}
void matmul_bf16_rows(const std::uint16_t* w, const float* x, float* y, std::size_t r, std::size_t o,
                      std::size_t i, std::size_t s) {
  FWD(matmul_bf16_rows, w, x, y, r, o, i, s);
}
void rmsnorm(const float* x, const float* weight, float* y, std::size_t n, float eps) {
  FWD(rmsnorm, x, weight, y, n, eps);
}
void rope(float* x, std::size_t n_heads, std::size_t pos, const RopeParams& p) {
  FWD(rope, x, n_heads, pos, p.head_dim, p.rotary_dim, p.theta, p.style == RopeStyle::NeoX ? 1 : 0,
      p.freq_factors);
}
void softmax(float* x, std::size_t n) { FWD(softmax, x, n); }
void silu_mul(const float* gate, const float* up, float* out, std::size_t n) { FWD(silu_mul, gate, up, out, n); }
void embedding_row(DType type, const void* table, std::size_t n, std::int64_t index, float* out) {
  FWD(embedding_row, static_cast<int>(type), table, n, index, out);
}
void attention(const float* q, const float* k, const float* v, float* out, float* scores, std::size_t seq,
               std::size_t n_head, std::size_t n_head_kv, std::size_t head_dim, float scale) {
  FWD(attention, q, k, v, out, scores, seq, n_head, n_head_kv, head_dim, scale);
}
void attention_kv(const float* q, const float* k, const float* v, float* out, float* scores, std::size_t n_q,
                  std::size_t n_past, std::size_t n_head, std::size_t n_head_kv, std::size_t head_dim, float scale) {
  FWD(attention_kv, q, k, v, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale);
}
void attention_kv_heads(const float* q, const float* k, const float* v, float* out, float* scores, std::size_t n_q,
                        std::size_t n_past, std::size_t n_head, std::size_t n_head_kv, std::size_t head_dim,
                        float scale, std::size_t hb, std::size_t he) {
  FWD(attention_kv_heads, q, k, v, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale, hb, he);
}
void attention_kv_heads_f16(const float* q, const std::uint16_t* k, const std::uint16_t* v, float* out,
                            float* scores, std::size_t n_q, std::size_t n_past, std::size_t n_head,
                            std::size_t n_head_kv, std::size_t head_dim, float scale, std::size_t hb,
                            std::size_t he) {
  FWD(attention_kv_heads_f16, q, k, v, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale, hb, he);
}
void matmul_q8_0(const BlockQ8_0* w, const float* x, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q8_0, w, x, y, o, i);
}
void matmul_q4_0(const BlockQ4_0* w, const float* x, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q4_0, w, x, y, o, i);
}
void matmul_q8_0_q8(const BlockQ8_0* w, const BlockQ8_0* xq, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q8_0_q8, w, xq, y, o, i);
}
void matmul_q4_0_q8(const BlockQ4_0* w, const BlockQ8_0* xq, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q4_0_q8, w, xq, y, o, i);
}
void matmul_q8_0_rows(const BlockQ8_0* w, const float* x, float* y, std::size_t r, std::size_t o, std::size_t i,
                      std::size_t s) {
  FWD(matmul_q8_0_rows, w, x, y, r, o, i, s);
}
void matmul_q4_0_rows(const BlockQ4_0* w, const float* x, float* y, std::size_t r, std::size_t o, std::size_t i,
                      std::size_t s) {
  FWD(matmul_q4_0_rows, w, x, y, r, o, i, s);
}
void matmul_q8_0_q8_rows(const BlockQ8_0* w, const BlockQ8_0* xq, float* y, std::size_t r, std::size_t o,
                         std::size_t i, std::size_t s) {
  FWD(matmul_q8_0_q8_rows, w, xq, y, r, o, i, s);
}
void matmul_q4_0_q8_rows(const BlockQ4_0* w, const BlockQ8_0* xq, float* y, std::size_t r, std::size_t o,
                         std::size_t i, std::size_t s) {
  FWD(matmul_q4_0_q8_rows, w, xq, y, r, o, i, s);
}
void quantize_row_q8_0(const float* x, BlockQ8_0* out, std::size_t n) { FWD(quantize_row_q8_0, x, out, n); }
void matmul_q4_1(const BlockQ4_1* w, const float* x, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q4_1, w, x, y, o, i);
}
void matmul_q4_1_q8(const BlockQ4_1* w, const BlockQ8_0* xq, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q4_1_q8, w, xq, y, o, i);
}
void matmul_q4_1_rows(const BlockQ4_1* w, const float* x, float* y, std::size_t r, std::size_t o, std::size_t i,
                      std::size_t s) {
  FWD(matmul_q4_1_rows, w, x, y, r, o, i, s);
}
void matmul_q4_1_q8_rows(const BlockQ4_1* w, const BlockQ8_0* xq, float* y, std::size_t r, std::size_t o,
                         std::size_t i, std::size_t s) {
  FWD(matmul_q4_1_q8_rows, w, xq, y, r, o, i, s);
}
void matmul_q6_k(const BlockQ6_K* w, const float* x, float* y, std::size_t o, std::size_t i) {
  FWD(matmul_q6_k, w, x, y, o, i);
}
void matmul_q6_k_rows(const BlockQ6_K* w, const float* x, float* y, std::size_t r, std::size_t o, std::size_t i,
                      std::size_t s) {
  FWD(matmul_q6_k_rows, w, x, y, r, o, i, s);
}

#undef FWD

constexpr KernelTable kHipTable{
    .matmul_f32 = matmul_f32,
    .matmul_f16 = matmul_f16,
    .matmul_bf16 = matmul_bf16,
    .matmul_f32_rows = matmul_f32_rows,
    .matmul_f16_rows = matmul_f16_rows,
    .matmul_bf16_rows = matmul_bf16_rows,
    .rmsnorm = rmsnorm,
    .rope = rope,
    .softmax = softmax,
    .silu_mul = silu_mul,
    .embedding_row = embedding_row,
    .attention = attention,
    .attention_kv = attention_kv,
    .attention_kv_heads = attention_kv_heads,
    .attention_kv_heads_f16 = attention_kv_heads_f16,
    .matmul_q8_0 = matmul_q8_0,
    .matmul_q4_0 = matmul_q4_0,
    .matmul_q8_0_q8 = matmul_q8_0_q8,
    .matmul_q4_0_q8 = matmul_q4_0_q8,
    .matmul_q8_0_rows = matmul_q8_0_rows,
    .matmul_q4_0_rows = matmul_q4_0_rows,
    .matmul_q8_0_q8_rows = matmul_q8_0_q8_rows,
    .matmul_q4_0_q8_rows = matmul_q4_0_q8_rows,
    .quantize_row_q8_0 = quantize_row_q8_0,
    .matmul_q4_1 = matmul_q4_1,
    .matmul_q4_1_q8 = matmul_q4_1_q8,
    .matmul_q4_1_rows = matmul_q4_1_rows,
    .matmul_q4_1_q8_rows = matmul_q4_1_q8_rows,
    .matmul_q6_k = matmul_q6_k,
    .matmul_q6_k_rows = matmul_q6_k_rows,
};

}  // namespace

const KernelTable& hip_kernels() { return kHipTable; }

Expected<const KernelTable*> select(KernelSet set) {
  switch (set) {
  case KernelSet::Scalar:
  case KernelSet::Neon:
    return make_error(ErrorCode::Unsupported,
                      "kernels: this library provides the hip table only; the scalar and NEON tables are "
                      "the reference's own");
  case KernelSet::Auto:
  case KernelSet::Hip: {
    const int rc = axon_hip_init(0);
    if (rc != AXON_HIP_OK) {
      return make_error(ErrorCode::Unsupported, std::string("kernels: no usable gfx950 device: ") +
                                                    axon_hip_last_error());
    }
    return &kHipTable;
  }
  }
  return make_error(ErrorCode::InvalidArgument, "kernels: unknown kernel set");
}

std::string_view name(const KernelTable& table) { return &table == &kHipTable ? "hip" : "custom"; }

bool parse_kernel_set(std::string_view text, KernelSet& out) {
  if (text == "auto") {
    out = KernelSet::Auto;
  } else if (text == "scalar") {
    out = KernelSet::Scalar;
  } else if (text == "neon") {
    out = KernelSet::Neon;
  } else if (text == "hip") {
    out = KernelSet::Hip;
  } else {
    return false;
  }
  return true;
}

}  // namespace axon::kernels
