// Float-activation matmuls of the hip table: F32 / F16 / BF16 weights
// (trickymind1324/axon-infer src/kernels/ref/matmul.cpp:12-68) and Q8_0 / Q4_0 / Q4_1 weights
// against float activations (src/kernels/ref/quant.cpp:15-40, 147-159), single-row and rows.
//
// None of the benchmark configurations reaches these entries (they serve float weight files and
// the exact-activations option), so each output is one lane walking its weight row left to
// right in float, which reproduces the scalar table's sum bit for bit, including the
// interleaved low/high nibble order of the Q4 formats.
#include "common.h"
#include "matmul_float.h"

namespace axon_hip {

namespace {

template <int T>
__device__ float row_dot(const uint8_t* w, const float* x, uint32_t n_in) {
  float acc = 0.0f;
  if constexpr (T == F32) {
    const float* r = reinterpret_cast<const float*>(w);
    for (uint32_t i = 0; i < n_in; ++i) acc += r[i] * x[i];
  } else if constexpr (T == F16) {
    const uint16_t* r = reinterpret_cast<const uint16_t*>(w);
    for (uint32_t i = 0; i < n_in; ++i) acc += half_bits_to_float(r[i]) * x[i];
  } else if constexpr (T == BF16) {
    const uint16_t* r = reinterpret_cast<const uint16_t*>(w);
    for (uint32_t i = 0; i < n_in; ++i) acc += bf16_bits_to_float(r[i]) * x[i];
  } else if constexpr (T == Q8_0) {
    for (uint32_t b = 0; b < n_in / kQK; ++b) {
      const uint8_t* blk = w + b * kBytesQ8_0;
      const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
      const float* xb = x + b * kQK;
      for (int i = 0; i < kQK; ++i) acc += static_cast<float>(static_cast<int8_t>(blk[2 + i])) * d * xb[i];
    }
  } else if constexpr (T == Q4_0) {
    for (uint32_t b = 0; b < n_in / kQK; ++b) {
      const uint8_t* blk = w + b * kBytesQ4_0;
      const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
      const float* xb = x + b * kQK;
      for (int i = 0; i < 16; ++i) {
        const uint8_t q = blk[2 + i];
        acc += static_cast<float>(static_cast<int>(q & 0x0f) - 8) * d * xb[i];
        acc += static_cast<float>(static_cast<int>(q >> 4) - 8) * d * xb[i + 16];
      }
    }
  } else {
    for (uint32_t b = 0; b < n_in / kQK; ++b) {
      const uint8_t* blk = w + b * kBytesQ4_1;
      const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
      const float m = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk + 2));
      const float* xb = x + b * kQK;
      for (int i = 0; i < 16; ++i) {
        const uint8_t q = blk[4 + i];
        acc += (static_cast<float>(q & 0x0f) * d + m) * xb[i];
        acc += (static_cast<float>(q >> 4) * d + m) * xb[i + 16];
      }
    }
  }
  return acc;
}

template <int T>
__global__ __launch_bounds__(256) void matmul_float_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                           float* __restrict__ y, uint32_t n_rows, uint32_t n_out,
                                                           uint32_t n_in, uint32_t y_stride, size_t row_bytes) {
  const uint32_t o = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t r = blockIdx.y;
  if (o >= n_out || r >= n_rows) return;
  y[static_cast<size_t>(r) * y_stride + o] = row_dot<T>(w + o * row_bytes, x + static_cast<size_t>(r) * n_in, n_in);
}

}  // namespace

int matmul_float_launch(int type, const void* w, const float* x, float* y, uint32_t n_rows, uint32_t n_out,
                        uint32_t n_in, uint32_t y_stride) {
  if (n_rows == 0 || n_out == 0) return kOk;
  size_t row_bytes = 0;
  switch (type) {
  case F32: row_bytes = 4ull * n_in; break;
  case F16: case BF16: row_bytes = 2ull * n_in; break;
  case Q8_0: row_bytes = n_in / kQK * kBytesQ8_0; break;
  case Q4_0: row_bytes = n_in / kQK * kBytesQ4_0; break;
  case Q4_1: row_bytes = n_in / kQK * kBytesQ4_1; break;
  default: return fail(kUnsupported, "matmul: weight type %d", type);
  }
  if ((type == Q8_0 || type == Q4_0 || type == Q4_1) && n_in % kQK != 0)
    return fail(kInvalidArgument, "quantized matmul: n_in %u is not a multiple of 32", n_in);
  const dim3 grid(static_cast<uint32_t>(ceil_div(n_out, 256)), n_rows);
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  switch (type) {
  case F32: hipLaunchKernelGGL(matmul_float_kernel<F32>, grid, dim3(256), 0, stream(), wb, x, y, n_rows, n_out, n_in, y_stride, row_bytes); break;
  case F16: hipLaunchKernelGGL(matmul_float_kernel<F16>, grid, dim3(256), 0, stream(), wb, x, y, n_rows, n_out, n_in, y_stride, row_bytes); break;
  case BF16: hipLaunchKernelGGL(matmul_float_kernel<BF16>, grid, dim3(256), 0, stream(), wb, x, y, n_rows, n_out, n_in, y_stride, row_bytes); break;
  case Q8_0: hipLaunchKernelGGL(matmul_float_kernel<Q8_0>, grid, dim3(256), 0, stream(), wb, x, y, n_rows, n_out, n_in, y_stride, row_bytes); break;
  case Q4_0: hipLaunchKernelGGL(matmul_float_kernel<Q4_0>, grid, dim3(256), 0, stream(), wb, x, y, n_rows, n_out, n_in, y_stride, row_bytes); break;
  default: hipLaunchKernelGGL(matmul_float_kernel<Q4_1>, grid, dim3(256), 0, stream(), wb, x, y, n_rows, n_out, n_in, y_stride, row_bytes); break;
  }
  return check_launch("matmul_float");
}

}  // namespace axon_hip
