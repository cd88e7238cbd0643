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

// ---- Few activation rows (batched decode): 5..64 rows -------------------------------------
// The same MFMA sums and the same per-output expression, block after block in order, with the
// work spread for latency rather than reuse: each wave owns one 16 weight rows x 16 activation
// rows tile, a workgroup's four waves sit WN x WM over the weight and activation rows (4 x 1 up
// to 16 rows, 2 x 2 up to 32, 1 x 4 up to 64), every segment of the call (q|k|v, gate|up) is one
// grid, and the next K chunk is loaded into registers while the current one computes. Chunk
// loads are raw buffer loads sized to the segment's and the activations' bytes: a load past
// either returns zero and touches nothing (the last rows and the last partial chunk).
constexpr uint32_t kRowsChunk = 16;  // blocks per K chunk

template <int T>
__host__ __device__ constexpr uint32_t rows_wpitch() { return kRowsChunk * block_bytes<T>() + 4; }
__host__ __device__ constexpr uint32_t rows_xpitch() { return kRowsChunk * kBytesQ8_0 + 4; }

template <int T, int WN, int WM>
__host__ __device__ constexpr size_t rows_lds() {
  return static_cast<size_t>(16 * WN) * rows_wpitch<T>() + static_cast<size_t>(16 * WM) * rows_xpitch() +
         static_cast<size_t>(kRowsChunk) * 16 * WM * 8 + static_cast<size_t>(kRowsChunk) * 16 * WN * 8;
}

template <int T, int WN, int WM>
__global__ __launch_bounds__(kThreads) void mfma_rows_kernel(MatvecArgs args) {
  static_assert(WN * WM == kThreads / 64, "four waves");
  constexpr int bs = block_bytes<T>();
  constexpr uint32_t TN = 16 * WN, TM = 16 * WM, KC = kRowsChunk;
  constexpr uint32_t WPITCH = rows_wpitch<T>(), XPITCH = rows_xpitch();
  constexpr uint32_t WU = KC * bs / 4, XU = KC * kBytesQ8_0 / 4;  // dwords per row chunk
  constexpr uint32_t NW = (TN * WU + kThreads - 1) / kThreads;
  constexpr uint32_t NX = (TM * XU + kThreads - 1) / kThreads;
  static_assert((KC * bs) % 4 == 0 && (KC * kBytesQ8_0) % 4 == 0, "dword chunks");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* wt = smem;                                         // [TN][WPITCH] weight bytes
  uint8_t* xt = wt + TN * WPITCH;                             // [TM][XPITCH] activation bytes
  float* xd = reinterpret_cast<float*>(xt + TM * XPITCH);     // [KC][TM] activation scales
  int32_t* xs = reinterpret_cast<int32_t*>(xd + KC * TM);     // [KC][TM] activation quant sums
  float* wd = reinterpret_cast<float*>(xs + KC * TM);         // [KC][TN] weight scales
  float* wmn = wd + KC * TN;                                  // [KC][TN] weight minimums (Q4_1)

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = tid >> 6;
  const uint32_t wn = wave % WN, wm = wave / WN;
  int s = 0;
  if (args.n_seg > 1 && blockIdx.x >= args.seg[1].wg_begin) s = 1;
  if (args.n_seg > 2 && blockIdx.x >= args.seg[2].wg_begin) s = 2;
  const MatvecSeg seg = args.seg[s];
  const uint32_t n0 = (blockIdx.x - seg.wg_begin) * TN;
  const uint32_t m0 = blockIdx.y * TM;
  const uint32_t nn = min(TN, seg.n_out - n0);
  const uint32_t mm = min(TM, args.m - m0);
  const uint32_t nb = args.nb;
  const uint32_t w_pitch = nb * bs, x_pitch = nb * kBytesQ8_0;
  const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(seg.w) + static_cast<size_t>(n0) * w_pitch, 0, static_cast<int>(nn * w_pitch),
      static_cast<int>(kRawBufferWord3));
  const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(args.xq) + static_cast<size_t>(m0) * x_pitch, 0, static_cast<int>(mm * x_pitch),
      static_cast<int>(kRawBufferWord3));

  uint32_t rw[NW], rx[NX];
  auto load = [&](uint32_t b0) {
#pragma unroll
    for (uint32_t k = 0; k < NW; ++k) {
      const uint32_t j = tid + k * kThreads;
      const uint32_t r = j / WU, c = j - r * WU;
      rw[k] = j < TN * WU ? __builtin_amdgcn_raw_buffer_load_b32(wsrc, r * w_pitch + b0 * bs + 4 * c, 0, 0) : 0u;
    }
#pragma unroll
    for (uint32_t k = 0; k < NX; ++k) {
      const uint32_t j = tid + k * kThreads;
      const uint32_t r = j / XU, c = j - r * XU;
      rx[k] = j < TM * XU ? __builtin_amdgcn_raw_buffer_load_b32(xsrc, r * x_pitch + b0 * kBytesQ8_0 + 4 * c, 0, 0)
                          : 0u;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (uint32_t k = 0; k < NW; ++k) {
      const uint32_t j = tid + k * kThreads;
      const uint32_t r = j / WU, c = j - r * WU;
      if (j < TN * WU) *reinterpret_cast<uint32_t*>(wt + r * WPITCH + 4 * c) = rw[k];
    }
#pragma unroll
    for (uint32_t k = 0; k < NX; ++k) {
      const uint32_t j = tid + k * kThreads;
      const uint32_t r = j / XU, c = j - r * XU;
      if (j < TM * XU) *reinterpret_cast<uint32_t*>(xt + r * XPITCH + 4 * c) = rx[k];
    }
  };

  const uint32_t col = lane & 15;  // weight row (B) / activation row (A) within the wave's 16
  const uint32_t kq = lane >> 4;   // which 8 of a block's 32 elements this lane feeds
  const uint32_t wr = wn * 16 + col;
  const uint32_t ar = wm * 16 + col;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};

  load(0);
  for (uint32_t b0 = 0; b0 < nb; b0 += KC) {
    const uint32_t cb = min(KC, nb - b0);
    store();
    __syncthreads();
    for (uint32_t i = tid; i < TM * KC; i += kThreads) {
      const uint32_t r = i / KC, b = i - r * KC;
      if (b < cb) {
        const ActBlock a = unpack_q8_0_lds(xt, r * XPITCH + b * kBytesQ8_0);
        xd[b * TM + r] = a.d;
        xs[b * TM + r] = a.sum;
      }
    }
    for (uint32_t i = tid; i < TN * KC; i += kThreads) {
      const uint32_t r = i / KC, b = i - r * KC;
      if (b < cb) {
        const uint32_t h = *reinterpret_cast<const uint16_t*>(wt + r * WPITCH + b * bs);
        wd[b * TN + r] = half_bits_to_float(h);
        if constexpr (T == Q4_1) {
          wmn[b * TN + r] = half_bits_to_float(*reinterpret_cast<const uint16_t*>(wt + r * WPITCH + b * bs + 2));
        }
      }
    }
    __syncthreads();
    if (b0 + KC < nb) load(b0 + KC);  // in flight while this chunk computes

    for (uint32_t b = 0; b < cb; ++b) {
      // B operand: weight row wr, elements 8*kq .. 8*kq+7 of block b.
      int64_t bw;
      {
        const uint32_t off = wr * WPITCH + b * bs;
        uint32_t q[2];
        if constexpr (T == Q8_0) {
          lds_read_unaligned<2>(wt, off + 2 + 8 * kq, q);
          bw = static_cast<int64_t>((static_cast<uint64_t>(q[1]) << 32) | q[0]);
        } else {
          constexpr uint32_t qoff = T == Q4_0 ? 2 : 4;
          lds_read_unaligned<2>(wt, off + qoff + 8 * (kq & 1), q);
          const uint32_t sh = (kq >> 1) * 4;  // low nibbles for elements 0..15, high for 16..31
          const uint32_t lo = (q[0] >> sh) & 0x0f0f0f0fu;
          const uint32_t hi = (q[1] >> sh) & 0x0f0f0f0fu;
          bw = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
        }
      }
      const float dw = wd[b * TN + wr];
      // A operand: activation row ar, elements 8*kq .. 8*kq+7 of block b.
      uint32_t qa[2];
      lds_read_unaligned<2>(xt, ar * XPITCH + b * kBytesQ8_0 + 2 + 8 * kq, qa);
      const int64_t ax = static_cast<int64_t>((static_cast<uint64_t>(qa[1]) << 32) | qa[0]);
      i32x4 d = {0, 0, 0, 0};
      d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, d, 0, 0, 0);
      const float4 dx4 = *reinterpret_cast<const float4*>(xd + b * TM + wm * 16 + 4 * kq);
      const int4 xs4 = *reinterpret_cast<const int4*>(xs + b * TM + wm * 16 + 4 * kq);
      const float dxv[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
      const int32_t xsv[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float dx = dxv[v];
        if constexpr (T == Q4_0) {
          const int32_t sumi = d[v] - 8 * xsv[v];
          acc[v] += static_cast<float>(sumi) * dw * dx;
        } else if constexpr (T == Q8_0) {
          acc[v] += static_cast<float>(d[v]) * dw * dx;
        } else {
          const float mw = wmn[b * TN + wr];
          acc[v] += static_cast<float>(d[v]) * dw * dx + mw * dx * static_cast<float>(xsv[v]);
        }
      }
    }
    __syncthreads();
  }

  if (wr < nn) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t r = wm * 16 + 4 * kq + v;
      if (r < mm) {
        float* y = seg.y + static_cast<size_t>(m0 + r) * seg.y_stride + n0 + wr;
        *y = args.accumulate ? *y + acc[v] : acc[v];
      }
    }
  }
}

template <int WN, int WM>
int rows_launch(int type, MatvecArgs& a) {
  constexpr uint32_t TN = 16 * WN, TM = 16 * WM;
  uint32_t wg = 0;
  for (int s = 0; s < a.n_seg; ++s) {
    a.seg[s].wg_begin = wg;
    wg += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, TN));
  }
  const dim3 grid(wg, static_cast<uint32_t>(ceil_div(a.m, TM)));
  switch (type) {
  case Q8_0: launch(mfma_rows_kernel<Q8_0, WN, WM>, grid, dim3(kThreads), rows_lds<Q8_0, WN, WM>(), a); break;
  case Q4_0: launch(mfma_rows_kernel<Q4_0, WN, WM>, grid, dim3(kThreads), rows_lds<Q4_0, WN, WM>(), a); break;
  case Q4_1: launch(mfma_rows_kernel<Q4_1, WN, WM>, grid, dim3(kThreads), rows_lds<Q4_1, WN, WM>(), a); break;
  default: return fail(kUnsupported, "matmul rows: weight type %d", type);
  }
  return check_launch("mfma_rows");
}

}  // namespace

bool matmul_q8_rows_fits(int type, const MatvecArgs& a) {
  if (a.m < 1 || a.m > kRowsMaxM || a.nb == 0) return false;
  if (type != Q8_0 && type != Q4_0 && type != Q4_1) return false;
  const uint32_t bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  // Dword loads: every weight row and activation row starts on a 4-byte boundary, and the
  // buffer ranges (rows x row bytes) fit a 32-bit record count.
  uintptr_t bases = reinterpret_cast<uintptr_t>(a.xq);
  for (int s = 0; s < a.n_seg; ++s) {
    bases |= reinterpret_cast<uintptr_t>(a.seg[s].w);
    if (static_cast<uint64_t>(a.nb) * bs * 64 >= (uint64_t(1) << 31)) return false;
  }
  return (bases & 3u) == 0 && (a.nb * bs) % 4 == 0 && (a.nb * kBytesQ8_0) % 4 == 0;
}

int matmul_q8_rows_launch(int type, MatvecArgs& a) {
  if (!matmul_q8_rows_fits(type, a)) return fail(kUnsupported, "matmul rows: shape or alignment");
  if (a.m <= 16) return rows_launch<4, 1>(type, a);
  if (a.m <= 32) return rows_launch<2, 2>(type, a);
  return rows_launch<1, 4>(type, a);
}

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
