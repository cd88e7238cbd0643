// Greedy token selection on the device, as the reference's sampler takes it at temperature zero
// (trickymind1324/axon-infer src/sampling/sampler.cpp:67-102): the repetition penalty over each
// row's recent tokens, then the index of the first maximum (std::ranges::max_element). Only the
// chosen ids cross to the host instead of [rows][n_vocab] floats.
//
// Penalty (sampler.cpp:73-97): one workgroup per row; each distinct in-range id of the row's
// window is rescaled once, by the thread holding its first occurrence, so no two threads write
// one logit. The window is short (repeat_last_n, 64 by default), so the quadratic first-occurrence
// scan costs less than a launch.
//
// Argmax, two launches: kParts workgroups per row each reduce a contiguous slice to one key, then one
// wave per row reduces the keys. A key orders (value, index) as max_element does: a larger
// value wins, and between equal values the smaller index. Values map to an unsigned order that
// matches float comparison for every non-NaN value (negative zero and zero compare equal, as
// they do with `<`). NaN follows max_element's scan with `<`: a NaN never replaces the running
// maximum and is skipped, except that a NaN in the first element is never replaced, so such a
// row selects index 0.
#include "common.h"
#include "elementwise.h"

namespace axon_hip {

namespace {

constexpr uint32_t kParts = 64;
constexpr uint32_t kThreads = 256;

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0;  // -0 == +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(~i);
}

__device__ __forceinline__ uint64_t max_key_wave(uint64_t k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(k, off, 64);
    k = o > k ? o : k;
  }
  return k;
}

__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float* __restrict__ x, uint32_t n,
                                                                  size_t stride, uint64_t* __restrict__ part) {
  __shared__ uint64_t red[kThreads / 64];
  const uint32_t r = blockIdx.y;
  const uint32_t chunk = (n + kParts - 1) / kParts;
  const uint32_t j0 = blockIdx.x * chunk;
  const uint32_t j1 = min(n, j0 + chunk);
  const float* row = x + static_cast<size_t>(r) * stride;
  uint64_t best = 0;
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kThreads) {
    const float v = row[j];
    if (v == v) {  // NaN never compares greater under max_element's `<`
      const uint64_t k = argmax_key(v, j);
      best = k > best ? k : best;
    }
  }
  best = max_key_wave(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t k = red[0];
    for (uint32_t w = 1; w < kThreads / 64; ++w) k = red[w] > k ? red[w] : k;
    part[static_cast<size_t>(r) * kParts + blockIdx.x] = k;
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ x, size_t stride,
                                                          const uint64_t* __restrict__ part, int32_t* __restrict__ out) {
  const uint32_t r = blockIdx.x;
  const uint64_t k = max_key_wave(part[static_cast<size_t>(r) * kParts + threadIdx.x]);
  if (threadIdx.x == 0) {
    const float first = x[static_cast<size_t>(r) * stride];
    // A NaN first element, or no key at all (every value NaN): index 0.
    out[r] = (first != first || k == 0) ? 0 : static_cast<int32_t>(~static_cast<uint32_t>(k & 0xffffffffu));
  }
}

__global__ __launch_bounds__(256) void repeat_penalty_kernel(float* __restrict__ x, uint32_t n, size_t stride,
                                                             const int32_t* __restrict__ recent,
                                                             const uint32_t* __restrict__ recent_len,
                                                             size_t recent_stride, float penalty) {
  const uint32_t r = blockIdx.x;
  const int32_t* ids = recent + static_cast<size_t>(r) * recent_stride;
  const uint32_t m = static_cast<uint32_t>(min(static_cast<size_t>(recent_len[r]), recent_stride));
  float* row = x + static_cast<size_t>(r) * stride;
  for (uint32_t i = threadIdx.x; i < m; i += blockDim.x) {
    const int32_t id = ids[i];
    if (id < 0 || static_cast<uint32_t>(id) >= n) continue;
    bool first = true;
    for (uint32_t j = 0; j < i && first; ++j) first = ids[j] != id;
    if (!first) continue;
    const float v = row[id];
    row[id] = v > 0.0f ? v / penalty : v * penalty;  // correctly rounded division, as on the host
  }
}

}  // namespace

int repeat_penalty_launch(float* x, uint32_t n, uint32_t n_rows, size_t stride, const int32_t* recent,
                          const uint32_t* recent_len, size_t recent_stride, float penalty) {
  if (n_rows == 0 || recent_stride == 0) return kOk;
  hipLaunchKernelGGL(repeat_penalty_kernel, dim3(n_rows), dim3(256), 0, stream(), x, n, stride, recent, recent_len,
                     recent_stride, penalty);
  return check_launch("repeat_penalty");
}

size_t argmax_scratch_words(uint32_t n_rows) { return static_cast<size_t>(n_rows) * kParts; }

int argmax_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, uint64_t* scratch, int32_t* out) {
  if (n_rows == 0) return kOk;
  if (n == 0) return fail(kInvalidArgument, "argmax: empty rows");
  if (n_rows > 65535) return fail(kInvalidArgument, "argmax: %u rows exceed one launch's 65535", n_rows);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(kParts, n_rows), dim3(kThreads), 0, stream(), x, n, stride, scratch);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(n_rows), dim3(64), 0, stream(), x, stride, scratch, out);
  return check_launch("argmax");
}

}  // namespace axon_hip
