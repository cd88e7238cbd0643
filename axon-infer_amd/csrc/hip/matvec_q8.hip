// Quantized weights (Q8_0, Q4_0, Q4_1) against Q8_0 activations for one to four activation
// rows: the batch-1 decode matvec. Follows trickymind1324/axon-infer
// src/kernels/ref/quant.cpp:44-69 (Q8_0, Q4_0) and quant.cpp:161-181 (Q4_1):
//
//   y[o] = sum over blocks b, in order, of float(sumi_b) * d_w * d_x   (Q8_0, Q4_0)
//   y[o] = sum over b of float(sumi_b) * d_w * d_x + m_w * d_x * float(sumx_b)   (Q4_1)
//
// where sumi_b is the exact int32 dot of the block's quants. The int32 dots (v_dot4_i32_i8)
// and the per-block float terms are computed in parallel across the workgroup; the float
// accumulation over blocks then runs left to right per output, exactly as the scalar table
// adds them, so every output is bit-identical to the scalar table's.
//
// Work split: a workgroup owns `rows` consecutive weight rows of one segment. Waves 1-3 copy
// the weight tile HBM -> LDS with coalesced 16-byte loads while wave 0 copies the activation
// blocks; the (row, block) pairs are then spread over all 256 lanes; finally one lane per
// (activation row, weight row) sums its row's block terms in order. Up to three weights that
// share one input (q, k and v) run as one launch: each segment owns a range of workgroups.
#include "common.h"
#include "matmul_float.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr int kThreads = 256;

template <int T>
struct Fmt;
template <>
struct Fmt<Q8_0> {
  static constexpr int bytes = kBytesQ8_0;
};
template <>
struct Fmt<Q4_0> {
  static constexpr int bytes = kBytesQ4_0;
};
template <>
struct Fmt<Q4_1> {
  static constexpr int bytes = kBytesQ4_1;
};

// The exact int32 dot of one weight block (at LDS byte offset `off`) with one activation
// block, with the Q4_0 offset applied, plus the block's weight scale (and Q4_1 minimum).
template <int T>
__device__ __forceinline__ int32_t block_sumi(const uint8_t* tile, uint32_t off, const ActBlock& a, float& dw,
                                              float& mw) {
  if constexpr (T == Q8_0) {
    uint32_t w[9];
    lds_read_unaligned<9>(tile, off, w);
    int32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = static_cast<int32_t>(__builtin_amdgcn_alignbit(w[i + 1], w[i], 16));
    dw = half_bits_to_float(w[0] & 0xffffu);
    mw = 0.0f;
    return dot32(q, a.qs);
  } else {
    // Q4_0 {d, qs[16]} and Q4_1 {d, m, qs[16]}: element i < 16 is the low nibble of qs[i],
    // element i + 16 the high nibble. Nibbles enter the signed dot as 0..15.
    constexpr uint32_t head = T == Q4_0 ? 2 : 4;
    uint32_t w[4];
    lds_read_unaligned<4>(tile, off + head, w);
    uint32_t h[1];
    lds_read_unaligned<1>(tile, off, h);
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = __builtin_amdgcn_sdot4(static_cast<int32_t>(w[i] & 0x0f0f0f0fu), a.qs[i], s, false);
      s = __builtin_amdgcn_sdot4(static_cast<int32_t>((w[i] >> 4) & 0x0f0f0f0fu), a.qs[4 + i], s, false);
    }
    dw = half_bits_to_float(h[0] & 0xffffu);
    if constexpr (T == Q4_0) {
      mw = 0.0f;
      // sum (nib - 8) * qx = sum nib * qx - 8 * sum qx, exactly, in int32.
      return s - 8 * a.sum;
    } else {
      mw = half_bits_to_float(h[0] >> 16);
      return s;
    }
  }
}

// The float term one weight block contributes against one activation block, in the scalar
// table's evaluation order.
template <int T>
__device__ __forceinline__ float block_term(const uint8_t* tile, uint32_t off, const ActBlock& a) {
  float dw, mw;
  const int32_t sumi = block_sumi<T>(tile, off, a, dw, mw);
  if constexpr (T == Q4_1) {
    return static_cast<float>(sumi) * dw * a.d + mw * a.d * static_cast<float>(a.sum);
  } else {
    return static_cast<float>(sumi) * dw * a.d;
  }
}

// Test hook: the per-block sums of one weight row against one activation row, through the same
// staging and block_sumi code the matvec runs. One workgroup, blocks strided over its lanes.
template <int T>
__global__ __launch_bounds__(kThreads) void block_sums_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xq,
                                                             uint32_t nb, int32_t* __restrict__ sumi,
                                                             int32_t* __restrict__ sumx) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int bs = Fmt<T>::bytes;
  uint8_t* wt = smem;
  uint8_t* xt = smem + ((nb * bs + 16 + 15) & ~15u);
  stage_bytes(w, wt, nb * bs, threadIdx.x, kThreads);
  stage_bytes(xq, xt, nb * kBytesQ8_0, threadIdx.x, kThreads);
  __syncthreads();
  for (uint32_t b = threadIdx.x; b < nb; b += kThreads) {
    const ActBlock a = unpack_q8_0_lds(xt, b * kBytesQ8_0);
    float dw, mw;
    sumi[b] = block_sumi<T>(wt, b * bs, a, dw, mw);
    if (sumx != nullptr) sumx[b] = a.sum;
  }
}

template <int T>
__global__ __launch_bounds__(kThreads) void matvec_q8_kernel(MatvecArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int bs = Fmt<T>::bytes;
  const uint32_t tid = threadIdx.x;
  const uint32_t nb = args.nb;
  const uint32_t M = args.m;
  const uint32_t R = args.rows;

  // Which segment and which of its rows this workgroup owns.
  uint32_t wg = blockIdx.x;
  int s = 0;
  if (args.n_seg > 1 && wg >= args.seg[1].wg_begin) s = 1;
  if (args.n_seg > 2 && wg >= args.seg[2].wg_begin) s = 2;
  const MatvecSeg seg = args.seg[s];
  const uint32_t r0 = (wg - seg.wg_begin) * R;
  const uint32_t nr = min(R, seg.n_out - r0);
  const uint32_t row_bytes = nb * bs;

  // LDS: act[M][nb] | tile[R * row_bytes] (+16 pad) | raw xq, later the term matrix.
  ActBlock* act = reinterpret_cast<ActBlock*>(smem);
  uint8_t* tile = smem + args.lds_tile;
  uint8_t* scratch = smem + args.lds_scratch;
  float* terms = reinterpret_cast<float*>(scratch);
  const uint32_t tpitch = nb + 1;  // odd pitch: the chain lanes read distinct banks

  // The activation blocks and the weight tile are copied side by side, by waves split in
  // proportion to their bytes, so both streams are in flight at once.
  const uint32_t xbytes = M * nb * kBytesQ8_0;
  const uint32_t tbytes = nr * row_bytes;
  const uint32_t xwaves = min(3u, max(1u, (4 * xbytes + (xbytes + tbytes) / 2) / (xbytes + tbytes)));
  const uint32_t xthreads = 64 * xwaves;
  if (tid < xthreads) {
    stage_bytes(args.xq, scratch, xbytes, tid, xthreads);
  } else {
    stage_bytes(seg.w + static_cast<size_t>(r0) * row_bytes, tile, tbytes, tid - xthreads, kThreads - xthreads);
  }
  __syncthreads();
  for (uint32_t i = tid; i < M * nb; i += kThreads) act[i] = unpack_q8_0_lds(scratch, i * kBytesQ8_0);
  __syncthreads();

  const uint32_t pairs = nr * nb;
  for (uint32_t p = tid; p < pairs; p += kThreads) {
    const uint32_t r = p / nb;
    const uint32_t b = p - r * nb;
    for (uint32_t m = 0; m < M; ++m) {
      terms[(m * R + r) * tpitch + b] = block_term<T>(tile, p * bs, act[m * nb + b]);
    }
  }
  __syncthreads();

  if (tid < M * nr) {
    const uint32_t m = tid / nr;
    const uint32_t r = tid - m * nr;
    const float* t = terms + (m * R + r) * tpitch;
    float acc = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) acc += t[b];
    float* y = seg.y + static_cast<size_t>(m) * seg.y_stride + r0 + r;
    *y = args.accumulate ? *y + acc : acc;
  }
}

}  // namespace

int block_sums_launch(int type, const void* w_row, const void* xq, uint32_t n_blocks, int32_t* sumi, int32_t* sumx) {
  if (n_blocks == 0) return kOk;
  const int bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  const size_t lds = ((static_cast<size_t>(n_blocks) * bs + 31) & ~size_t(15)) + n_blocks * kBytesQ8_0 + 16;
  if (lds > 65536) return fail(kInvalidArgument, "block_sums: %u blocks exceed one LDS tile", n_blocks);
  const uint8_t* w = static_cast<const uint8_t*>(w_row);
  const uint8_t* x = static_cast<const uint8_t*>(xq);
  switch (type) {
  case Q8_0: launch(block_sums_kernel<Q8_0>, dim3(1), dim3(kThreads), lds, w, x, n_blocks, sumi, sumx); break;
  case Q4_0: launch(block_sums_kernel<Q4_0>, dim3(1), dim3(kThreads), lds, w, x, n_blocks, sumi, sumx); break;
  case Q4_1: launch(block_sums_kernel<Q4_1>, dim3(1), dim3(kThreads), lds, w, x, n_blocks, sumi, sumx); break;
  default: return fail(kUnsupported, "block_sums: weight type %d", type);
  }
  return check_launch("block_sums");
}

namespace {

size_t matvec_lds_bytes(int bs, uint32_t m, uint32_t nb, uint32_t rows, size_t* act_out, size_t* tile_out) {
  const size_t row_bytes = static_cast<size_t>(nb) * bs;
  const size_t act = (static_cast<size_t>(m) * nb * sizeof(ActBlock) + 15) & ~size_t(15);
  const size_t tile = (rows * row_bytes + 16 + 15) & ~size_t(15);
  const size_t raw = static_cast<size_t>(m) * nb * kBytesQ8_0 + 16;
  const size_t terms = static_cast<size_t>(m) * rows * (nb + 1) * 4;
  if (act_out != nullptr) *act_out = act;
  if (tile_out != nullptr) *tile_out = tile;
  return act + tile + std::max(raw, terms);
}

}  // namespace

uint32_t matvec_q8_max_rows(int type, uint32_t nb) {
  const int bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  for (uint32_t m = 4; m > 1; --m) {
    if (matvec_lds_bytes(bs, m, nb, 1, nullptr, nullptr) <= 65536) return m;
  }
  return 1;
}

int matvec_q8_launch(int type, MatvecArgs& a) {
  if (a.m == 0 || a.nb == 0) return kOk;
  const int bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  const size_t row_bytes = static_cast<size_t>(a.nb) * bs;
  uint32_t total_out = 0;
  for (int s = 0; s < a.n_seg; ++s) total_out += a.seg[s].n_out;
  // Rows per workgroup: a tile of up to 16 KB, but at least ~512 workgroups when the matrix
  // has the rows for it, and at most 64 rows so every (activation, weight) row gets a lane.
  uint32_t rows = static_cast<uint32_t>(std::max<size_t>(1, 16384 / row_bytes));
  rows = std::min<uint32_t>(rows, std::max<uint32_t>(1, total_out / 512));
  rows = std::min<uint32_t>(rows, 256 / a.m);
  for (;;) {
    size_t act = 0, tile = 0;
    const size_t lds = matvec_lds_bytes(bs, a.m, a.nb, rows, &act, &tile);
    if (lds <= 65536 || rows == 1) {
      if (lds > 65536) return fail(kUnsupported, "matvec: %u blocks per row over %u rows exceed LDS", a.nb, a.m);
      a.rows = rows;
      a.lds_tile = static_cast<uint32_t>(act);
      a.lds_scratch = static_cast<uint32_t>(act + tile);
      uint32_t wg = 0;
      for (int s = 0; s < a.n_seg; ++s) {
        a.seg[s].wg_begin = wg;
        wg += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, rows));
      }
      if (wg == 0) return kOk;
      switch (type) {
      case Q8_0:
        launch(matvec_q8_kernel<Q8_0>, dim3(wg), dim3(kThreads), lds, a);
        break;
      case Q4_0:
        launch(matvec_q8_kernel<Q4_0>, dim3(wg), dim3(kThreads), lds, a);
        break;
      case Q4_1:
        launch(matvec_q8_kernel<Q4_1>, dim3(wg), dim3(kThreads), lds, a);
        break;
      default:
        return fail(kUnsupported, "matvec: weight type %d has no Q8_0-activation path", type);
      }
      return check_launch("matvec_q8");
    }
    rows = std::max<uint32_t>(1, rows / 2);
  }
}

}  // namespace axon_hip
