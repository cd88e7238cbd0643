// Grouped-query attention over KV-cache spans, one workgroup per (query row, kv head): the
// table's attention / attention_kv / attention_kv_heads(_f16) entries and the ragged batched
// entry that serves every sequence of a continuous batch in one launch per layer.
//
// Follows trickymind1324/axon-infer src/kernels/ref/attention.cpp:27-59 (and 77-113 for the
// fp16 cache) with softmax from src/kernels/ref/softmax.cpp:10-25:
//   scores[j] = scale * dot(q, k_j), the dot left to right in float, j <= pos;
//   softmax: max, e_j = exp(s_j - max) in float, sum in double, p_j = e_j * float(1 / sum);
//   o[d] = sum over j in ascending order of p_j * v_j[d], in float.
// The score dots run one position per lane (each lane walks d in order), the value mix one
// (head, d) pair per lane (each lane walks j in order), so both float reductions keep the
// scalar table's order. The exponential is evaluated in double and rounded once, and the double
// sum is reduced as a tree; both differ from the scalar table only in rare last-bit cases.
//
// The workgroup's query heads share one kv head, so every K and V row is read from HBM once
// per query row. Scores live in LDS when they fit, otherwise in a global scratch.
#include "common.h"
#include "elementwise.h"

namespace axon_hip {

namespace {

constexpr int kThreads = 256;
constexpr size_t kLdsScores = 48 * 1024;

template <bool F16>
__device__ __forceinline__ float kv_at(const void* base, size_t i) {
  if constexpr (F16) {
    return half_bits_to_float(reinterpret_cast<const uint16_t*>(base)[i]);
  } else {
    return reinterpret_cast<const float*>(base)[i];
  }
}

template <bool F16, bool GLOBAL>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t r = blockIdx.x;
  const uint32_t g = blockIdx.y;
  const uint32_t tid = threadIdx.x;
  const uint32_t hd = a.head_dim;
  const uint32_t group = a.n_head / a.n_kv;
  const uint32_t h_lo = max(g * group, a.head_begin);
  const uint32_t h_hi = min(g * group + group, a.head_end);
  if (h_lo >= h_hi) return;
  const uint32_t nh = h_hi - h_lo;

  const int64_t k_off = (a.k_off != nullptr ? a.k_off[r] : 0) + a.k_off_c;
  const int64_t v_off = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * hd;

  float* qs = lds;                                   // [nh][hd]
  __shared__ double red_d[kThreads / 64];
  __shared__ float red_f[kThreads / 64];
  float* sc = GLOBAL ? a.scratch + (static_cast<size_t>(r) * gridDim.y + g) * group * a.max_vis : lds + group * hd;
  const uint32_t pitch = GLOBAL ? a.max_vis : n_vis;

  // 16-byte loads of K rows when every row of this span is 16-byte aligned.
  const bool vec4 = !F16 && hd == 64 &&
                    (reinterpret_cast<uintptr_t>(reinterpret_cast<const float*>(a.kv) + k_off) & 15u) == 0 &&
                    (kv_row & 3u) == 0;
  const float* q = a.q + static_cast<size_t>(r) * a.q_stride + static_cast<size_t>(h_lo) * hd;
  for (uint32_t i = tid; i < nh * hd; i += kThreads) qs[i] = q[i];
  __syncthreads();

  // Scores: one position per lane, each dot in d order.
  for (uint32_t j = tid; j < n_vis; j += kThreads) {
    const size_t krow = k_off + j * kv_row + static_cast<size_t>(g) * hd;
    if (vec4) {
      float kr[64];
      const float4* kp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kv) + krow);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float4 t = kp[i];
        kr[4 * i] = t.x;
        kr[4 * i + 1] = t.y;
        kr[4 * i + 2] = t.z;
        kr[4 * i + 3] = t.w;
      }
      for (uint32_t h = 0; h < nh; ++h) {
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < 64; ++d) acc += qs[h * 64 + d] * kr[d];
        sc[h * pitch + j] = a.scale * acc;
      }
    } else {
      for (uint32_t h = 0; h < nh; ++h) {
        float acc = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) acc += qs[h * hd + d] * kv_at<F16>(a.kv, krow + d);
        sc[h * pitch + j] = a.scale * acc;
      }
    }
  }
  __syncthreads();

  // Softmax per head.
  for (uint32_t h = 0; h < nh; ++h) {
    float* s = sc + h * pitch;
    float m = -INFINITY;
    for (uint32_t j = tid; j < n_vis; j += kThreads) m = fmaxf(m, s[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red_f[tid >> 6] = m;
    __syncthreads();
    m = red_f[0];
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red_f[w]);
    double sum = 0.0;
    for (uint32_t j = tid; j < n_vis; j += kThreads) {
      const float e = exp_rounded(s[j] - m);
      s[j] = e;
      sum += static_cast<double>(e);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if ((tid & 63) == 0) red_d[tid >> 6] = sum;
    __syncthreads();
    sum = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) sum += red_d[w];
    const float inv = static_cast<float>(1.0 / sum);
    for (uint32_t j = tid; j < n_vis; j += kThreads) s[j] *= inv;
    __syncthreads();
  }

  // Value mix: one (head, d) per lane, positions in ascending order.
  float* out = a.out + static_cast<size_t>(r) * a.out_stride + static_cast<size_t>(h_lo) * hd;
  for (uint32_t t = tid; t < nh * hd; t += kThreads) {
    const uint32_t h = t / hd;
    const uint32_t d = t - h * hd;
    const float* p = sc + h * pitch;
    const size_t vbase = v_off + static_cast<size_t>(g) * hd + d;
    float acc = 0.0f;
    uint32_t j = 0;
    for (; j + 4 <= n_vis; j += 4) {
      const float v0 = kv_at<F16>(a.kv, vbase + (j + 0) * kv_row);
      const float v1 = kv_at<F16>(a.kv, vbase + (j + 1) * kv_row);
      const float v2 = kv_at<F16>(a.kv, vbase + (j + 2) * kv_row);
      const float v3 = kv_at<F16>(a.kv, vbase + (j + 3) * kv_row);
      acc += p[j] * v0;
      acc += p[j + 1] * v1;
      acc += p[j + 2] * v2;
      acc += p[j + 3] * v3;
    }
    for (; j < n_vis; ++j) acc += p[j] * kv_at<F16>(a.kv, vbase + j * kv_row);
    out[t] = acc;
  }
}

bool scores_fit_lds(const AttnArgs& a) {
  const uint32_t group = a.n_head / a.n_kv;
  return static_cast<size_t>(group) * (a.head_dim + a.max_vis) * 4 <= kLdsScores;
}

}  // namespace

size_t attention_scratch_floats(const AttnArgs& a, uint32_t n_rows) {
  if (scores_fit_lds(a)) return 0;
  return static_cast<size_t>(n_rows) * a.n_head * a.max_vis;
}

int attention_launch(const AttnArgs& a, uint32_t n_rows) {
  if (n_rows == 0) return kOk;
  if (a.n_kv == 0 || a.n_head % a.n_kv != 0)
    return fail(kInvalidArgument, "attention: %u heads over %u kv heads", a.n_head, a.n_kv);
  if (a.head_begin > a.head_end || a.head_end > a.n_head)
    return fail(kInvalidArgument, "attention: heads [%u, %u) of %u", a.head_begin, a.head_end, a.n_head);
  if (a.head_begin == a.head_end) return kOk;
  const uint32_t group = a.n_head / a.n_kv;
  const dim3 grid(n_rows, a.n_kv);
  const bool lds_ok = scores_fit_lds(a);
  if (!lds_ok && a.scratch == nullptr) return fail(kInvalidArgument, "attention: %u positions need a score scratch", a.max_vis);
  const size_t lds = lds_ok ? static_cast<size_t>(group) * (a.head_dim + a.max_vis) * 4
                            : static_cast<size_t>(group) * a.head_dim * 4;
  if (a.f16) {
    if (lds_ok) hipLaunchKernelGGL((attention_kernel<true, false>), grid, dim3(kThreads), lds, stream(), a);
    else hipLaunchKernelGGL((attention_kernel<true, true>), grid, dim3(kThreads), lds, stream(), a);
  } else {
    if (lds_ok) hipLaunchKernelGGL((attention_kernel<false, false>), grid, dim3(kThreads), lds, stream(), a);
    else hipLaunchKernelGGL((attention_kernel<false, true>), grid, dim3(kThreads), lds, stream(), a);
  }
  return check_launch("attention");
}

}  // namespace axon_hip
