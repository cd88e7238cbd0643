// Row-wise kernels of the hip table: Q8_0 activation quantization (alone, fused behind
// RMSNorm, fused behind SiLU * up), RMSNorm, RoPE (with the Qwen2 bias and the KV-cache write
// fused in), softmax, residual add and embedding rows. Each follows one scalar-table function of
// trickymind1324/axon-infer; the citation sits above each kernel.
#include "common.h"
#include "elementwise.h"

namespace axon_hip {

namespace {

// Double-precision sum over the workgroup (256 threads), result broadcast to all threads.
__device__ __forceinline__ double block_sum_double(double v, double* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const uint32_t wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  double s = 0.0;
  for (uint32_t w = 0; w < blockDim.x / 64; ++w) s += red[w];
  __syncthreads();
  return s;
}

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const uint32_t wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (uint32_t w = 1; w < blockDim.x / 64; ++w) m = fmaxf(m, red[w]);
  __syncthreads();
  return m;
}

// quantize_row_q8_0 over rows: one half-wave per block. Grid: (ceil(blocks/8), rows).
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                            uint32_t n, uint32_t x_stride) {
  const uint32_t nb = n / kQK;
  const uint32_t b = blockIdx.x * 8 + (threadIdx.x >> 5);
  const uint32_t lane = threadIdx.x & 31;
  const uint32_t row = blockIdx.y;
  if (b >= nb) return;  // whole half-waves leave together
  const float v = x[static_cast<size_t>(row) * x_stride + b * kQK + lane];
  quantize_block_lanes(v, lane, out + (static_cast<size_t>(row) * nb + b) * kBytesQ8_0);
}

// rmsnorm (src/kernels/ref/rmsnorm.cpp:10-21): inv = float(1 / sqrt(sum(x^2)/n + eps)) with
// the sum in double, then y = x * inv * w. The double sum is reduced as a tree: it differs from
// the scalar table's left-to-right double sum only in its last bits, which survive the
// rounding to float only when the two sums straddle a float rounding boundary. Optionally
// writes y, the Q8_0 blocks of y, or both. One workgroup per row.
// Rows of up to 256 * 8 elements (every model here) take rmsnorm_regs_kernel: each thread
// holds 8 consecutive elements in registers from one load to the quantized store, and the 4
// threads of a 32-element block agree on its scale through shuffles.
__global__ __launch_bounds__(256) void rmsnorm_regs_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ y, uint8_t* __restrict__ yq,
                                                           uint32_t n, float eps) {
  __shared__ double red[4];
  const size_t row = blockIdx.x;
  rmsnorm_row_256(x + row * n, w, y != nullptr ? y + row * n : nullptr,
                  yq != nullptr ? yq + row * (n / kQK) * kBytesQ8_0 : nullptr, n, eps, red);
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      float* __restrict__ y, uint8_t* __restrict__ yq,
                                                      uint32_t n, float eps) {
  __shared__ double red[4];
  const uint32_t row = blockIdx.x;
  const float* xr = x + static_cast<size_t>(row) * n;
  double ss = 0.0;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    const double v = static_cast<double>(xr[i]);
    ss += v * v;
  }
  ss = block_sum_double(ss, red);
  const float inv = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(n) + static_cast<double>(eps)));
  if (yq == nullptr) {
    float* yr = y + static_cast<size_t>(row) * n;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) yr[i] = xr[i] * inv * w[i];
    return;
  }
  // One half-wave per Q8_0 block of the normalised row; each half-wave first loads all of its
  // blocks' inputs (up to eight at a time) so the loads are in flight together.
  const uint32_t nb = n / kQK;
  const uint32_t lane = threadIdx.x & 31;
  const uint32_t halves = blockDim.x / 32;
  uint8_t* qr = yq + static_cast<size_t>(row) * nb * kBytesQ8_0;
  for (uint32_t b0 = threadIdx.x >> 5; b0 < nb; b0 += 8 * halves) {
    float xv[8], wv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t b = b0 + k * halves;
      if (b < nb) {
        xv[k] = xr[b * kQK + lane];
        wv[k] = w[b * kQK + lane];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t b = b0 + k * halves;
      if (b < nb) {
        const float v = xv[k] * inv * wv[k];
        if (y != nullptr) y[static_cast<size_t>(row) * n + b * kQK + lane] = v;
        quantize_block_lanes(v, lane, qr + b * kBytesQ8_0);
      }
    }
  }
}

// silu_mul (src/kernels/ref/silu.cpp:8-13): out = g / (1 + exp(-g)) * up. With `outq` the
// product is also quantized to Q8_0 blocks (the down projection's input).
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                       float* out, uint8_t* __restrict__ outq, uint32_t n,
                                                       uint32_t n_rows) {
  const size_t total = static_cast<size_t>(n) * n_rows;
  if (outq == nullptr) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
      const float g = gate[i];
      out[i] = g / (1.0f + exp_libm(-g)) * up[i];
    }
    return;
  }
  const uint32_t nb = n / kQK;
  const size_t blocks = static_cast<size_t>(nb) * n_rows;
  const uint32_t lane = threadIdx.x & 31;
  for (size_t blk = static_cast<size_t>(blockIdx.x) * (blockDim.x / 32) + (threadIdx.x >> 5); blk < blocks;
       blk += static_cast<size_t>(gridDim.x) * (blockDim.x / 32)) {
    const size_t i = blk * kQK + lane;
    const float g = gate[i];
    const float v = g / (1.0f + exp_libm(-g)) * up[i];
    if (out != nullptr) out[i] = v;
    quantize_block_lanes(v, lane, outq + blk * kBytesQ8_0);
  }
}

// softmax (src/kernels/ref/softmax.cpp:10-25) of one row, in place: max, exp(x - max) in
// float, sum in double, scale by float(1 / sum).
__global__ __launch_bounds__(256) void softmax_kernel(float* x, uint32_t n) {
  __shared__ double red[4];
  __shared__ float redf[4];
  float m = -INFINITY;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
  m = block_max(m, redf);
  double s = 0.0;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float e = exp_libm(x[i] - m);
    x[i] = e;
    s += static_cast<double>(e);
  }
  s = block_sum_double(s, red);
  const float inv = static_cast<float>(1.0 / s);
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) x[i] *= inv;
}

// x += y over n floats (the residual add of src/model/llama.cpp:122-126).
__global__ __launch_bounds__(256) void add_kernel(float* x, const float* __restrict__ y, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    x[i] = x[i] + y[i];
  }
}

// rope (src/kernels/ref/rope.cpp:13-37) on rows of heads. The rotation of pair (a, b) by the
// angle pos * inv_freq_i is x0 * c - x1 * s, x0 * s + x1 * c in float. The cos/sin come from a
// table [pos][rotary_dim / 2] (float pairs) built on the host with the same double-precision
// libm calls as the scalar table, or, without a table, are evaluated here in double.
//
// Per row r: the q row (n_head heads) and the k row (n_kv heads) are rotated at pos[r]. With
// biases, b is added first (src/model/llama.cpp:507-511). With a cache, the rotated k row and
// the (biased) v row are written to the cache at the row's position.
__global__ __launch_bounds__(256) void rope_rows_kernel(RopeRowsArgs a) {
  const uint32_t r = blockIdx.x;
  const uint32_t half = a.rotary_dim / 2;
  const int32_t pos = a.pos != nullptr ? a.pos[r] : a.pos0 + static_cast<int32_t>(r);
  float* q = a.q != nullptr ? a.q + static_cast<size_t>(r) * a.q_stride : nullptr;
  float* k = a.k != nullptr ? a.k + static_cast<size_t>(r) * a.k_stride : nullptr;
  const float* v = a.v != nullptr ? a.v + static_cast<size_t>(r) * a.k_stride : nullptr;
  // The row's cache slots: float elements, or fp16 bit patterns rounded in once.
  float* kc = nullptr;
  float* vc = nullptr;
  uint16_t* kc16 = nullptr;
  uint16_t* vc16 = nullptr;
  if (a.cache != nullptr) {
    const int64_t base = a.cache_off != nullptr ? a.cache_off[r] : 0;
    const size_t row = static_cast<size_t>(a.n_kv) * a.head_dim;
    const size_t k_at = base + a.k_layer_off + static_cast<size_t>(pos) * row;
    const size_t v_at = base + a.v_layer_off + static_cast<size_t>(pos) * row;
    if (a.cache_f16) {
      kc16 = static_cast<uint16_t*>(a.cache) + k_at;
      vc16 = static_cast<uint16_t*>(a.cache) + v_at;
    } else {
      kc = static_cast<float*>(a.cache) + k_at;
      vc = static_cast<float*>(a.cache) + v_at;
    }
  }
  const uint32_t nq = a.q != nullptr ? a.n_head * a.head_dim : 0;
  const uint32_t nk = a.k != nullptr ? a.n_kv * a.head_dim : 0;
  // Pass 1: biases (in place on q and k; v is biased on its way to the cache or in place).
  if (a.bq != nullptr) {
    for (uint32_t i = threadIdx.x; i < nq; i += blockDim.x) q[i] = q[i] + a.bq[i];
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x) k[i] = k[i] + a.bk[i];
  }
  if (v != nullptr) {
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x) {
      const float vv = a.bv != nullptr ? v[i] + a.bv[i] : v[i];
      if (vc != nullptr) vc[i] = vv;
      else if (vc16 != nullptr) vc16[i] = static_cast<uint16_t>(float_to_half_bits(vv));
      else const_cast<float*>(v)[i] = vv;
    }
  }
  __syncthreads();
  // Pass 2: rotate pairs. Element t enumerates (head, i) over q heads then k heads.
  const uint32_t pairs_q = a.q != nullptr ? a.n_head * half : 0;
  const uint32_t pairs = pairs_q + (a.k != nullptr ? a.n_kv * half : 0);
  for (uint32_t t = threadIdx.x; t < pairs; t += blockDim.x) {
    const bool is_q = t < pairs_q;
    const uint32_t u = is_q ? t : t - pairs_q;
    const uint32_t h = u / half;
    const uint32_t i = u - h * half;
    float c, s;
    if (a.table != nullptr) {
      const float2 cs = reinterpret_cast<const float2*>(a.table)[static_cast<size_t>(pos) * half + i];
      c = cs.x;
      s = cs.y;
    } else {
      double inv_freq = pow(static_cast<double>(a.theta), -static_cast<double>(2 * i) / static_cast<double>(a.rotary_dim));
      if (a.freq_factors != nullptr) inv_freq /= static_cast<double>(a.freq_factors[i]);
      const double angle = static_cast<double>(pos) * inv_freq;
      c = static_cast<float>(cos(angle));
      s = static_cast<float>(sin(angle));
    }
    const uint32_t ia = a.neox ? i : 2 * i;
    const uint32_t ib = a.neox ? i + half : 2 * i + 1;
    float* head = (is_q ? q : k) + h * a.head_dim;
    const float x0 = head[ia];
    const float x1 = head[ib];
    head[ia] = x0 * c - x1 * s;
    head[ib] = x0 * s + x1 * c;
  }
  if (kc != nullptr || kc16 != nullptr) {
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x) {
      if (kc != nullptr) kc[i] = k[i];
      else kc16[i] = static_cast<uint16_t>(float_to_half_bits(k[i]));
    }
  }
}

// embedding_row (src/kernels/ref/embedding.cpp:12-64): element i of row `row` of an n-wide
// table, dequantized exactly as dtype.cpp:274-336 does (types checked by the launchers).
__device__ __forceinline__ float embed_value(int type, const uint8_t* __restrict__ table, uint32_t n, int64_t row,
                                             uint32_t i) {
  switch (type) {
  case F32:
    return reinterpret_cast<const float*>(table)[row * n + i];
  case F16:
    return half_bits_to_float(reinterpret_cast<const uint16_t*>(table)[row * n + i]);
  case BF16:
    return bf16_bits_to_float(reinterpret_cast<const uint16_t*>(table)[row * n + i]);
  case Q8_0: {
    const uint8_t* blk = table + (row * (n / kQK) + i / kQK) * kBytesQ8_0;
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
    return static_cast<float>(static_cast<int8_t>(blk[2 + i % kQK])) * d;
  }
  case Q4_0: {
    const uint8_t* blk = table + (row * (n / kQK) + i / kQK) * kBytesQ4_0;
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
    const uint32_t e = i % kQK;
    const int nib = e < 16 ? (blk[2 + e] & 0x0f) : (blk[2 + e - 16] >> 4);
    return static_cast<float>(nib - 8) * d;
  }
  case Q4_1: {
    const uint8_t* blk = table + (row * (n / kQK) + i / kQK) * kBytesQ4_1;
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
    const float m = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk + 2));
    const uint32_t e = i % kQK;
    const int nib = e < 16 ? (blk[4 + e] & 0x0f) : (blk[4 + e - 16] >> 4);
    return static_cast<float>(nib) * d + m;
  }
  case Q6_K: {
    const uint8_t* blk = table + (row * (n / kQKK) + i / kQKK) * kBytesQ6_K;
    const uint32_t e = i % kQKK;
    const uint32_t nh = e / 128;       // which 128-half
    const uint32_t w = e % 128;
    const uint32_t quarter = w / 32;   // 0: q1, 1: q2, 2: q3, 3: q4
    const uint32_t l = w % 32;
    const uint8_t* ql = blk + nh * 64;
    const uint8_t* qh = blk + 128 + nh * 32;
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + nh * 8);
    const uint32_t qlb = ql[l + (quarter & 1) * 32];
    const uint32_t lowbits = (quarter < 2) ? (qlb & 0x0f) : (qlb >> 4);
    const uint32_t hibits = (qh[l] >> (2 * quarter)) & 3u;
    const int q = static_cast<int>(lowbits | (hibits << 4)) - 32;
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
    return d * static_cast<float>(sc[l / 16 + 2 * quarter]) * static_cast<float>(q);
  }
  default:
    return 0.0f;
  }
}

// embedding_row for a list of token ids: row ids[r] of the table into out[r][n].
__global__ __launch_bounds__(256) void embedding_kernel(int type, const uint8_t* __restrict__ table, uint32_t n,
                                                        const int32_t* __restrict__ ids, int64_t id0,
                                                        float* __restrict__ out) {
  const uint32_t r = blockIdx.y;
  const int64_t row = ids != nullptr ? ids[r] : id0;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[static_cast<size_t>(r) * n + i] = embed_value(type, table, n, row, i);
}

// The greedy choice of one logits row from its n_parts partial keys (argmax_final_kernel's rule:
// the largest key, index 0 when the row's first value is NaN or no key exists), then that
// token's embedding row: every workgroup reduces the keys (a few KB) and embeds its 256
// elements; workgroup 0 writes the id.
__global__ __launch_bounds__(256) void argmax_embed_kernel(const float* __restrict__ x,
                                                           const uint64_t* __restrict__ part, uint32_t n_parts,
                                                           int32_t* __restrict__ out_id, int type,
                                                           const uint8_t* __restrict__ table, uint32_t table_rows,
                                                           uint32_t n, float* __restrict__ emb) {
  __shared__ uint64_t red[4];
  uint64_t k = 0;
  for (uint32_t j = threadIdx.x; j < n_parts; j += 256) k = part[j] > k ? part[j] : k;
  k = max_key_wave(k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  k = red[0];
  for (int w = 1; w < 4; ++w) k = red[w] > k ? red[w] : k;
  const float first = x[0];
  const int32_t id = (first != first || k == 0) ? 0 : static_cast<int32_t>(~static_cast<uint32_t>(k & 0xffffffffu));
  if (blockIdx.x == 0 && threadIdx.x == 0) *out_id = id;
  // The keys index a row of at most table_rows values; the clamp only keeps a caller's mismatch
  // inside the table.
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) emb[i] = embed_value(type, table, n, min(static_cast<uint32_t>(id), table_rows - 1), i);
}

}  // namespace

int quantize_rows_launch(const float* x, uint8_t* out, uint32_t n, uint32_t n_rows, uint32_t x_stride) {
  if (n % kQK != 0) return fail(kInvalidArgument, "quantize_row_q8_0: n %u is not a multiple of 32", n);
  if (n == 0 || n_rows == 0) return kOk;
  const dim3 grid(static_cast<uint32_t>(ceil_div(n / kQK, 8)), n_rows);
  hipLaunchKernelGGL(quantize_rows_kernel, grid, dim3(256), 0, stream(), x, out, n, x_stride);
  return check_launch("quantize_rows");
}

int rmsnorm_launch(const float* x, const float* w, float* y, uint8_t* yq, uint32_t n, uint32_t n_rows, float eps) {
  if (n == 0 || n_rows == 0) return kOk;
  if (yq != nullptr && n % kQK != 0) return fail(kInvalidArgument, "rmsnorm+quantize: n %u is not a multiple of 32", n);
  const bool regs = n % kQK == 0 && n <= 256 * 8 &&
                    ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                      reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  if (regs) {
    hipLaunchKernelGGL(rmsnorm_regs_kernel, dim3(n_rows), dim3(256), 0, stream(), x, w, y, yq, n, eps);
  } else {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_rows), dim3(256), 0, stream(), x, w, y, yq, n, eps);
  }
  return check_launch("rmsnorm");
}

int silu_mul_launch(const float* gate, const float* up, float* out, uint8_t* outq, uint32_t n, uint32_t n_rows) {
  if (n == 0 || n_rows == 0) return kOk;
  if (outq != nullptr && n % kQK != 0) return fail(kInvalidArgument, "silu_mul+quantize: n %u is not a multiple of 32", n);
  const size_t total = static_cast<size_t>(n) * n_rows;
  const uint32_t grid = static_cast<uint32_t>(std::min<size_t>(ceil_div(total, 256), 4096));
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid), dim3(256), 0, stream(), gate, up, out, outq, n, n_rows);
  return check_launch("silu_mul");
}

int softmax_launch(float* x, uint32_t n) {
  if (n == 0) return kOk;
  hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(256), 0, stream(), x, n);
  return check_launch("softmax");
}

int add_launch(float* x, const float* y, size_t n) {
  if (n == 0) return kOk;
  const uint32_t grid = static_cast<uint32_t>(std::min<size_t>(ceil_div(n, 256), 4096));
  hipLaunchKernelGGL(add_kernel, dim3(grid), dim3(256), 0, stream(), x, y, n);
  return check_launch("add_rows");
}

int rope_rows_launch(const RopeRowsArgs& a, uint32_t n_rows) {
  if (n_rows == 0) return kOk;
  if (a.rotary_dim % 2 != 0 || a.rotary_dim > a.head_dim)
    return fail(kInvalidArgument, "rope: rotary_dim %u with head_dim %u", a.rotary_dim, a.head_dim);
  hipLaunchKernelGGL(rope_rows_kernel, dim3(n_rows), dim3(256), 0, stream(), a);
  return check_launch("rope_rows");
}

namespace {
int embedding_check(int type, uint32_t n) {
  switch (type) {
  case F32: case F16: case BF16: break;
  case Q8_0: case Q4_0: case Q4_1:
    if (n % kQK != 0) return fail(kInvalidArgument, "embedding_row: n %u is not a multiple of 32", n);
    break;
  case Q6_K:
    if (n % kQKK != 0) return fail(kInvalidArgument, "embedding_row: n %u is not a multiple of 256", n);
    break;
  default:
    return fail(kUnsupported, "embedding_row: unsupported dtype %d", type);
  }
  return kOk;
}
}  // namespace

int embedding_launch(int type, const uint8_t* table, uint32_t n, const int32_t* ids, int64_t id0, uint32_t n_rows,
                     float* out) {
  if (n == 0 || n_rows == 0) return kOk;
  if (const int rc = embedding_check(type, n); rc != kOk) return rc;
  const dim3 grid(static_cast<uint32_t>(ceil_div(n, 256)), n_rows);
  hipLaunchKernelGGL(embedding_kernel, grid, dim3(256), 0, stream(), type, table, n, ids, id0, out);
  return check_launch("embedding");
}

int argmax_embed_launch(const float* x, const uint64_t* part, uint32_t n_parts, int32_t* out_id, int type,
                        const uint8_t* table, uint32_t table_rows, uint32_t n, float* emb) {
  if (n == 0 || n_parts == 0 || table_rows == 0)
    return fail(kInvalidArgument, "argmax_embed: %u keys, %u table rows of %u", n_parts, table_rows, n);
  if (const int rc = embedding_check(type, n); rc != kOk) return rc;
  hipLaunchKernelGGL(argmax_embed_kernel, dim3(static_cast<uint32_t>(ceil_div(n, 256))), dim3(256), 0, stream(), x,
                     part, n_parts, out_id, type, table, table_rows, n, emb);
  return check_launch("argmax_embed");
}

}  // namespace axon_hip
