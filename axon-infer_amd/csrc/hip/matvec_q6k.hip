// Q6_K weights against float activations: the output and embedding matrices' path, following
// trickymind1324/axon-infer src/kernels/ref/quant.cpp:183-194 with the super-block decoding of
// src/core/dtype.cpp:312-336 (ggml's Q6_K: ql[128], qh[64], int8 scales[16], fp16 d).
//
// The scalar table dequantizes (d * scale) * q and accumulates all n_in products in one float
// chain. This is a float path with a 1e-5 relative budget, so the kernel regroups the sum:
// per 16-element scale group it accumulates q' * x with q' = q - 32 exact in float, then adds
// (d * scale) * group_sum. The error stays at the level of one float summation of the row.
//
// A workgroup stages `rows` weight rows (1680 bytes each at n_in = 2048) into LDS with 16-byte
// coalesced loads and the activation rows as floats; each wave then walks whole rows, one ql
// dword (8 weights) per lane and step, and reduces across the wave at the end of a row.
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float byte_f(uint32_t w, int e) {
  return static_cast<float>(static_cast<int>((w >> (8 * e)) & 0xffu) - 32);
}

template <int MM>
__global__ __launch_bounds__(kThreads) void matvec_q6k_kernel(MatvecArgs args, uint32_t n_in, uint32_t x_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = tid >> 6;
  const uint32_t nsb = args.nb;
  const uint32_t R = args.rows;
  const MatvecSeg seg = args.seg[0];
  const uint32_t r0 = blockIdx.x * R;
  const uint32_t nr = min(R, seg.n_out - r0);
  const uint32_t row_bytes = nsb * kBytesQ6_K;
  const float* x = reinterpret_cast<const float*>(args.xq);

  float* xs = reinterpret_cast<float*>(smem);  // [MM][n_in]
  uint8_t* tile = smem + args.lds_tile;
  if (((reinterpret_cast<uintptr_t>(x) | (x_stride * 4u)) & 15u) == 0) {
    for (uint32_t m = 0; m < MM; ++m) {
      for (uint32_t i = tid; i < n_in / 4; i += kThreads) {
        reinterpret_cast<float4*>(xs + m * n_in)[i] = reinterpret_cast<const float4*>(x + m * x_stride)[i];
      }
    }
  } else {
    for (uint32_t m = 0; m < MM; ++m) {
      for (uint32_t i = tid; i < n_in; i += kThreads) xs[m * n_in + i] = x[m * x_stride + i];
    }
  }
  stage_bytes(seg.w + static_cast<size_t>(r0) * row_bytes, tile, nr * row_bytes, tid, kThreads);
  __syncthreads();

  const uint32_t units = nsb * 32;
  for (uint32_t r = wave; r < nr; r += kThreads / 64) {
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
    for (uint32_t u = lane; u < units; u += 64) {
      const uint32_t sb = u >> 5;
      const uint32_t i = u & 31;
      const uint32_t base = r * row_bytes + sb * kBytesQ6_K;
      uint32_t q[1], h[1];
      const uint32_t half = i >> 4;
      const uint32_t j0 = 4 * (i & 15);
      const bool upper = j0 >= 32;
      const uint32_t l = upper ? j0 - 32 : j0;
      lds_read_unaligned<1>(tile, base + 4 * i, q);
      lds_read_unaligned<1>(tile, base + 128 + half * 32 + l, h);
      const int8_t* sc = reinterpret_cast<const int8_t*>(tile + base + 192 + half * 8 + l / 16);
      const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(tile + base + 208));
      const float da = d * static_cast<float>(sc[upper ? 2 : 0]);
      const float db = d * static_cast<float>(sc[upper ? 6 : 4]);
      const uint32_t lo = q[0] & 0x0f0f0f0fu;
      const uint32_t hi = (q[0] >> 4) & 0x0f0f0f0fu;
      const uint32_t qa = lo | (upper ? (h[0] & 0x0c0c0c0cu) << 2 : (h[0] & 0x03030303u) << 4);
      const uint32_t qb = hi | (upper ? (h[0] & 0xc0c0c0c0u) >> 2 : (h[0] & 0x30303030u));
      const uint32_t ya = sb * 256 + half * 128 + l + (upper ? 32 : 0);
      const uint32_t yb = ya + 64;
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        const float4 xa = *reinterpret_cast<const float4*>(xs + m * n_in + ya);
        const float4 xb = *reinterpret_cast<const float4*>(xs + m * n_in + yb);
        float sa = byte_f(qa, 0) * xa.x;
        sa = fmaf(byte_f(qa, 1), xa.y, sa);
        sa = fmaf(byte_f(qa, 2), xa.z, sa);
        sa = fmaf(byte_f(qa, 3), xa.w, sa);
        float sbv = byte_f(qb, 0) * xb.x;
        sbv = fmaf(byte_f(qb, 1), xb.y, sbv);
        sbv = fmaf(byte_f(qb, 2), xb.z, sbv);
        sbv = fmaf(byte_f(qb, 3), xb.w, sbv);
        acc[m] = fmaf(da, sa, acc[m]);
        acc[m] = fmaf(db, sbv, acc[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float v = acc[m];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) seg.y[static_cast<size_t>(m) * seg.y_stride + r0 + r] = v;
    }
  }
}

}  // namespace

int matvec_q6k_launch(MatvecArgs& a, uint32_t n_in) {
  const uint32_t n_out = a.seg[0].n_out;
  if (a.m == 0 || n_out == 0) return kOk;
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k: n_in %u is not a multiple of 256", n_in);
  const size_t row_bytes = static_cast<size_t>(a.nb) * kBytesQ6_K;
  uint32_t rows = static_cast<uint32_t>(std::max<size_t>(4, 16384 / row_bytes));
  rows = std::min<uint32_t>(rows, std::max<uint32_t>(1, n_out / 1024));
  rows = std::max<uint32_t>(rows, 1);
  const MatvecArgs base = a;
  const float* x = reinterpret_cast<const float*>(a.xq);
  uint32_t done = 0;
  while (done < base.m) {
    uint32_t mm = std::min<uint32_t>(4, base.m - done);
    while (mm > 1 && static_cast<size_t>(mm) * n_in * 4 + rows * row_bytes + 32 > 65536) mm /= 2;
    while (rows > 1 && static_cast<size_t>(mm) * n_in * 4 + rows * row_bytes + 32 > 65536) rows /= 2;
    const size_t xbytes = (static_cast<size_t>(mm) * n_in * 4 + 15) & ~size_t(15);
    const size_t lds = xbytes + rows * row_bytes + 32;
    if (lds > 65536) return fail(kUnsupported, "matmul_q6_k: n_in %u too large for one LDS tile", n_in);
    MatvecArgs g = base;
    g.m = mm;
    g.rows = rows;
    g.lds_tile = static_cast<uint32_t>(xbytes);
    g.xq = reinterpret_cast<const uint8_t*>(x + static_cast<size_t>(done) * n_in);
    g.seg[0].y = base.seg[0].y + static_cast<size_t>(done) * base.seg[0].y_stride;
    const dim3 grid(static_cast<uint32_t>(ceil_div(n_out, rows)));
    switch (mm) {
    case 4: hipLaunchKernelGGL(matvec_q6k_kernel<4>, grid, dim3(kThreads), lds, stream(), g, n_in, n_in); break;
    case 3: hipLaunchKernelGGL(matvec_q6k_kernel<3>, grid, dim3(kThreads), lds, stream(), g, n_in, n_in); break;
    case 2: hipLaunchKernelGGL(matvec_q6k_kernel<2>, grid, dim3(kThreads), lds, stream(), g, n_in, n_in); break;
    default: hipLaunchKernelGGL(matvec_q6k_kernel<1>, grid, dim3(kThreads), lds, stream(), g, n_in, n_in); break;
    }
    const int rc = check_launch("matvec_q6k");
    if (rc != kOk) return rc;
    done += mm;
  }
  return kOk;
}

}  // namespace axon_hip
