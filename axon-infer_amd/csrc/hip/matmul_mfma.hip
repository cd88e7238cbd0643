// Quantized weights (Q8_0, Q4_0, Q4_1) against 16 or more Q8_0 activation rows on the int8
// matrix cores: the batched-decode and prefill path of trickymind1324/axon-infer
// src/kernels/ref/quant.cpp:95-139 and 211-232 (the `_q8_rows` entries).
//
// One v_mfma_i32_16x16x32_i8 consumes exactly one 32-element block of 16 activation rows
// against one block of 16 weight rows, so its int32 results are the per-block sums sumi of the
// scalar table, exactly. Each lane then folds its four results into float accumulators with
// the scalar table's expression, block after block in order:
//
//   acc += float(sumi) * d_w * d_x                      (Q8_0, Q4_0: sumi includes the -8 offset)
//   acc += float(sumi) * d_w * d_x + m_w * d_x * float(sumx)          (Q4_1)
//
// so every output is bit-identical to the scalar table's. Q4 nibbles enter the MFMA as
// unsigned values 0..15; the Q4_0 offset is applied as -8 * sum(qx) in int32.
//
// Workgroup tile: 64 activation rows x 64 weight rows (four waves, 16 weight rows each, four
// 16-row activation tiles per wave), K staged through LDS 16 blocks at a time.
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr int kThreads = 256;
constexpr int kTileM = 64;  // activation rows per workgroup
constexpr int kTileN = 64;  // weight rows per workgroup

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

template <int T>
constexpr int block_bytes() {
  return T == Q8_0 ? kBytesQ8_0 : T == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
}

template <int T>
__global__ __launch_bounds__(kThreads) void mfma_q8_kernel(MatvecArgs args, uint32_t kc) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int bs = block_bytes<T>();
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = tid >> 6;
  const uint32_t nb = args.nb;
  const MatvecSeg seg = args.seg[0];
  const uint32_t n0 = blockIdx.x * kTileN;
  const uint32_t m0 = blockIdx.y * kTileM;
  const uint32_t nn = min(static_cast<uint32_t>(kTileN), seg.n_out - n0);
  const uint32_t mm = min(static_cast<uint32_t>(kTileM), args.m - m0);
  const size_t w_pitch = static_cast<size_t>(nb) * bs;
  const size_t x_pitch = static_cast<size_t>(nb) * kBytesQ8_0;

  // LDS: weight chunk [64][kc*bs], activation chunk [64][kc*34], then per (act row, block)
  // the float scale and the int sum of the quants.
  const uint32_t wrow = kc * bs;
  const uint32_t xrow = kc * kBytesQ8_0;
  uint8_t* wt = smem;
  uint8_t* xt = smem + ((kTileN * wrow + 16 + 15) & ~15u);
  float* xd = reinterpret_cast<float*>(xt + ((kTileM * xrow + 16 + 15) & ~15u));
  int32_t* xs = reinterpret_cast<int32_t*>(xd + kTileM * kc);

  const uint32_t col = lane & 15;     // weight row within the wave's 16 / D column
  const uint32_t kq = lane >> 4;      // which 8 of the block's 32 elements this lane feeds
  const uint32_t wr = wave * 16 + col;
  const int n_mt = static_cast<int>((mm + 15) / 16);

  float acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;

  for (uint32_t b0 = 0; b0 < nb; b0 += kc) {
    const uint32_t cb = min(kc, nb - b0);
    stage_rows(seg.w + static_cast<size_t>(n0) * w_pitch + static_cast<size_t>(b0) * bs, w_pitch, wt, wrow, nn,
               cb * bs, tid, kThreads);
    stage_rows(args.xq + static_cast<size_t>(m0) * x_pitch + static_cast<size_t>(b0) * kBytesQ8_0, x_pitch, xt,
               xrow, mm, cb * kBytesQ8_0, tid, kThreads);
    __syncthreads();
    for (uint32_t i = tid; i < mm * cb; i += kThreads) {
      const uint32_t r = i / cb;
      const uint32_t b = i - r * cb;
      const ActBlock a = unpack_q8_0_lds(xt, r * xrow + b * kBytesQ8_0);
      xd[r * kc + b] = a.d;
      xs[r * kc + b] = a.sum;
    }
    __syncthreads();

    for (uint32_t b = 0; b < cb; ++b) {
      // B operand: weight row wr, elements 8*kq .. 8*kq+7 of block b.
      int64_t bw;
      float dw, mw = 0.0f;
      {
        const uint32_t off = wr * wrow + b * bs;
        if constexpr (T == Q8_0) {
          uint32_t h[1];
          lds_read_unaligned<1>(wt, off, h);
          dw = half_bits_to_float(h[0] & 0xffffu);
          uint32_t q[2];
          lds_read_unaligned<2>(wt, off + 2 + 8 * kq, q);
          bw = static_cast<int64_t>((static_cast<uint64_t>(q[1]) << 32) | q[0]);
        } else {
          constexpr uint32_t qoff = T == Q4_0 ? 2 : 4;
          uint32_t h[1];
          lds_read_unaligned<1>(wt, off, h);
          dw = half_bits_to_float(h[0] & 0xffffu);
          if constexpr (T == Q4_1) mw = half_bits_to_float(h[0] >> 16);
          uint32_t q[2];
          lds_read_unaligned<2>(wt, off + qoff + 8 * (kq & 1), q);
          const uint32_t sh = (kq >> 1) * 4;  // low nibbles for elements 0..15, high for 16..31
          const uint32_t lo = (q[0] >> sh) & 0x0f0f0f0fu;
          const uint32_t hi = (q[1] >> sh) & 0x0f0f0f0fu;
          bw = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t < n_mt) {
          // A operand: activation row 16t + col, elements 8*kq .. 8*kq+7 of block b.
          const uint32_t ar = 16 * t + col;
          uint32_t q[2];
          lds_read_unaligned<2>(xt, ar * xrow + b * kBytesQ8_0 + 2 + 8 * kq, q);
          const int64_t ax = static_cast<int64_t>((static_cast<uint64_t>(q[1]) << 32) | q[0]);
          i32x4 d = {0, 0, 0, 0};
          d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, d, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t r = 16 * t + 4 * kq + v;  // activation row of D[v]
            const float dx = xd[r * kc + b];
            if constexpr (T == Q4_0) {
              const int32_t sumi = d[v] - 8 * xs[r * kc + b];
              acc[t][v] += static_cast<float>(sumi) * dw * dx;
            } else if constexpr (T == Q8_0) {
              acc[t][v] += static_cast<float>(d[v]) * dw * dx;
            } else {
              acc[t][v] += static_cast<float>(d[v]) * dw * dx + mw * dx * static_cast<float>(xs[r * kc + b]);
            }
          }
        }
      }
    }
    __syncthreads();
  }

  if (wr < nn) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t r = 16 * t + 4 * kq + v;
        if (r < mm) {
          float* y = seg.y + static_cast<size_t>(m0 + r) * seg.y_stride + n0 + wr;
          *y = args.accumulate ? *y + acc[t][v] : acc[t][v];
        }
      }
    }
  }
}

}  // namespace

int matmul_q8_mfma_launch(int type, MatvecArgs& a) {
  const uint32_t n_out = a.seg[0].n_out;
  if (a.m == 0 || n_out == 0 || a.nb == 0) return kOk;
  const int bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  uint32_t kc = 16;
  auto lds_of = [&](uint32_t k) {
    const size_t w = (kTileN * static_cast<size_t>(k) * bs + 16 + 15) & ~size_t(15);
    const size_t x = (kTileM * static_cast<size_t>(k) * kBytesQ8_0 + 16 + 15) & ~size_t(15);
    return w + x + kTileM * static_cast<size_t>(k) * 8;
  };
  while (kc > 1 && lds_of(kc) > 65536) kc /= 2;
  const size_t lds = lds_of(kc);
  const dim3 grid(static_cast<uint32_t>(ceil_div(n_out, kTileN)), static_cast<uint32_t>(ceil_div(a.m, kTileM)));
  switch (type) {
  case Q8_0: launch(mfma_q8_kernel<Q8_0>, grid, dim3(kThreads), lds, a, kc); break;
  case Q4_0: launch(mfma_q8_kernel<Q4_0>, grid, dim3(kThreads), lds, a, kc); break;
  case Q4_1: launch(mfma_q8_kernel<Q4_1>, grid, dim3(kThreads), lds, a, kc); break;
  default: return fail(kUnsupported, "matmul rows: weight type %d has no Q8_0-activation path", type);
  }
  return check_launch("mfma_q8");
}

}  // namespace axon_hip
