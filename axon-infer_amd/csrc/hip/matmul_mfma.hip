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

// ---- Few activation rows (batched decode): 3..64 rows -------------------------------------
// The same MFMA sums and the same per-output expression, block after block in order, with the
// work spread for latency: a workgroup owns 16 (or 8) weight rows x 16 activation rows, every
// segment of the call (q|k|v, gate|up) is one grid, and 17..64 rows take several row tiles
// along the grid's second axis. Per K chunk the four waves split its blocks, run each block's
// MFMA once and write its terms float(sumi) * d_w * d_x into LDS; then each thread adds one
// output's terms in block order (terms, then chains).
// K goes in chunks of KC blocks (32, or 64 where the grid is one round of workgroups). Each
// thread loads whole (row, block) items of the next
// chunk into registers (from the 4-byte boundary at or below the block, enough dwords to cover
// it) while the current chunk computes, then expands them once into 32 aligned int8 values and
// the scales in LDS: Q8_0 quants as they are, Q4_0 nibbles as q - 8 ((b + 0x78) ^ 0x80 per
// byte, so the MFMA sum is sumi itself), Q4_1 nibbles as q. The loads are raw buffer loads
// sized to the segment's and the activations' bytes: a load past either returns zero and
// touches nothing (the last rows, the last blocks, the last partial chunk).
constexpr uint32_t kRowsChunk = 32;                 // blocks per K chunk
constexpr uint32_t kRowsTN = 16;                    // weight rows per workgroup

template <int T>
__host__ __device__ constexpr uint32_t item_dwords() {
  return (block_bytes<T>() + 2 + 3) / 4;  // a 2-byte aligned block from its 4-byte boundary
}

// LDS: expanded weights [16][KC * 8 + 4], expanded activations [TM][KC * 8 + 4] (dwords), then
// per (row, block) scales: wd, wm [16][KC], xd, xs [KC][TM] (KC blocks per chunk); the launcher
// adds the terms buffer.
template <int TM, uint32_t TN = kRowsTN, uint32_t KC = kRowsChunk>
__host__ __device__ constexpr size_t rows_lds() {
  return (static_cast<size_t>(TN + TM) * (KC * 8 + 4) + static_cast<size_t>(TN + TM) * KC * 2) * 4;
}

// TN: weight rows per workgroup, 16 or 8. With 8 (a narrow matrix, so twice the workgroups),
// lanes of weight column col read row col % 8 into the 16-wide MFMA and only columns below 8
// are stored.
template <int T, int TM, uint32_t TN = kRowsTN, bool ROPE = false, uint32_t KCH = kRowsChunk>
__global__ __launch_bounds__(kThreads) void mfma_rows_kernel(MatvecArgs args, RowsRope rp) {
  static_assert(TN == 16 || TN == 8, "16 or 8 weight rows");
  constexpr int bs = block_bytes<T>();
  constexpr uint32_t KC = KCH, P = KCH * 8 + 4;
  static_assert(TM == 16, "one tile of 16 activation rows");
  constexpr uint32_t WI = TN * KC / kThreads;           // weight items per thread per chunk
  constexpr uint32_t XI = TM * KC / kThreads;           // activation items per thread per chunk
  constexpr uint32_t WD = item_dwords<T>(), XD = item_dwords<Q8_0>();
  static_assert(TN * KC % kThreads == 0 && TM * KC % kThreads == 0, "whole items per thread");

  extern __shared__ __attribute__((aligned(16))) uint32_t lds_rows[];
  uint32_t* wa = lds_rows;                               // [TN][P]
  uint32_t* xa = wa + TN * P;                            // [TM][P]
  float* wd = reinterpret_cast<float*>(xa + TM * P);     // [TN][KC]
  float* wmn = wd + TN * KC;                             // [TN][KC] (Q4_1)
  float* xd = wmn + TN * KC;                             // [TM][KC]
  int32_t* xs = reinterpret_cast<int32_t*>(xd + TM * KC);  // [TM][KC] (Q4_1)

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = tid >> 6;
  int s = 0;
  if (args.n_seg > 1 && blockIdx.x >= args.seg[1].wg_begin) s = 1;
  if (args.n_seg > 2 && blockIdx.x >= args.seg[2].wg_begin) s = 2;
  const MatvecSeg seg = args.seg[s];
  const uint32_t n0 = (blockIdx.x - seg.wg_begin) * TN;
  const uint32_t m0 = blockIdx.y * TM;
  const uint32_t nn = min(TN, seg.n_out - n0);
  const uint32_t mm = min(static_cast<uint32_t>(TM), args.m - m0);
  const uint32_t nb = args.nb;
  const uint32_t n_chunks = (nb + KC - 1) / KC;
  const uint32_t w_pitch = nb * bs, x_pitch = nb * kBytesQ8_0;
  const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(seg.w) + static_cast<size_t>(n0) * w_pitch, 0, static_cast<int>(nn * w_pitch),
      static_cast<int>(kRawBufferWord3));
  const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(args.xq) + static_cast<size_t>(m0) * x_pitch, 0, static_cast<int>(mm * x_pitch),
      static_cast<int>(kRawBufferWord3));

  // Item i of a chunk: block i % KC of row i / KC (blocks fastest: consecutive threads read
  // consecutive blocks of a row). The bases are 4-byte aligned (the launcher checks), so a
  // block's byte offset and its 4-byte boundary differ by 0 or 2.
  struct Raw {
    uint32_t w[WI][WD];
    uint32_t x[XI][XD];
  };
  auto load = [&](uint32_t c, Raw& r) {
    const uint32_t b0 = c * KC;
#pragma unroll
    for (uint32_t k = 0; k < WI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t off = row * w_pitch + (b0 + b) * bs;
#pragma unroll
      for (uint32_t d = 0; d < WD; ++d)
        r.w[k][d] = __builtin_amdgcn_raw_buffer_load_b32(wsrc, (off & ~3u) + 4 * d, 0, 0);
    }
#pragma unroll
    for (uint32_t k = 0; k < XI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t off = row * x_pitch + (b0 + b) * kBytesQ8_0;
#pragma unroll
      for (uint32_t d = 0; d < XD; ++d)
        r.x[k][d] = __builtin_amdgcn_raw_buffer_load_b32(xsrc, (off & ~3u) + 4 * d, 0, 0);
    }
  };
  auto expand = [&](uint32_t c, const Raw& r) {
    const uint32_t b0 = c * KC;
#pragma unroll
    for (uint32_t k = 0; k < WI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t sh = (((b0 + b) * bs) & 3u) * 8;  // the row start is 4-byte aligned
      // v: the block from its first byte (the fp16 scale(s), then the quants); its last dword
      // holds only the block's last bytes, from the last loaded dword.
      uint32_t v[WD];
#pragma unroll
      for (uint32_t d = 0; d < WD; ++d) v[d] = __builtin_amdgcn_alignbit(d + 1 < WD ? r.w[k][d + 1] : 0u, r.w[k][d], sh);
      uint32_t q[8];
      if constexpr (T == Q8_0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbit(v[j + 1], v[j], 16);
      } else {
        constexpr uint32_t first = T == Q4_0 ? 0 : 1;  // the dword where the nibbles start
        constexpr uint32_t bsh = T == Q4_0 ? 16 : 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t n4 = bsh ? __builtin_amdgcn_alignbit(v[first + j + 1], v[first + j], bsh) : v[first + j];
          q[j] = n4 & 0x0f0f0f0fu;             // elements 4j .. 4j+3: low nibbles
          q[j + 4] = (n4 >> 4) & 0x0f0f0f0fu;  // elements 16+4j ..: high nibbles
          if constexpr (T == Q4_0) {
            // q - 8 as int8 per byte: a byte is at most 0x87 after the add, so no carry
            // crosses bytes, and flipping bit 7 subtracts 128.
            q[j] = (q[j] + 0x78787878u) ^ 0x80808080u;
            q[j + 4] = (q[j + 4] + 0x78787878u) ^ 0x80808080u;
          }
        }
      }
      uint4* dst = reinterpret_cast<uint4*>(wa + row * P + b * 8);
      dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
      dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
      wd[row * KC + b] = half_bits_to_float(v[0] & 0xffffu);
      if constexpr (T == Q4_1) wmn[row * KC + b] = half_bits_to_float(v[0] >> 16);
    }
#pragma unroll
    for (uint32_t k = 0; k < XI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t sh = (((b0 + b) * kBytesQ8_0) & 3u) * 8;
      uint32_t v[XD];
#pragma unroll
      for (uint32_t d = 0; d < XD; ++d) v[d] = __builtin_amdgcn_alignbit(d + 1 < XD ? r.x[k][d + 1] : 0u, r.x[k][d], sh);
      uint32_t q[8];
      int32_t sum = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        q[j] = __builtin_amdgcn_alignbit(v[j + 1], v[j], 16);
        if constexpr (T == Q4_1) sum = __builtin_amdgcn_sdot4(static_cast<int32_t>(q[j]), 0x01010101, sum, false);
      }
      uint4* dst = reinterpret_cast<uint4*>(xa + row * P + b * 8);
      dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
      dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
      // The terms read a lane's four rows of a block at once: block-major.
      const uint32_t xi = b * TM + row;
      xd[xi] = half_bits_to_float(v[0] & 0xffffu);
      if constexpr (T == Q4_1) xs[xi] = sum;
    }
  };

  const uint32_t col = lane & 15;  // weight row (B) within the tile's 16
  const uint32_t wrow = col % TN;  // the LDS row it reads (col itself when TN = 16)
  const uint32_t kq = lane >> 4;   // which 8 of a block's 32 elements this lane feeds

  // The output (activation row r, weight column c of the tile) with value x: stored or added,
  // or (ROPE) biased, rotated and written to q or the cache. Every lane calls it (the RoPE
  // partner comes from lane ^ 1, the column next to it).
  auto finish = [&](uint32_t c, uint32_t r, float x) {
    if constexpr (ROPE) {
      // Segments q, k, v: the bias, then the rotation of each pair (2i, 2i + 1) of a head as
      // rope_rows_kernel forms it (x0 * c - x1 * s, x0 * s + x1 * c); n0 is a multiple of TN,
      // so output n's partner n ^ 1 is column c ^ 1, held by lane ^ 1.
      const uint32_t n = n0 + c;
      if (rp.bias[s] != nullptr && c < nn) x = x + rp.bias[s][n];
      const float other = __shfl_xor(x, 1, 64);
      if (c < nn && r < mm) {
        const int32_t pos = rp.pos[m0 + r];
        if (s < 2) {
          const uint32_t i = (n % rp.head_dim) / 2;
          if (i < rp.rot_half) {
            const float2 cs = reinterpret_cast<const float2*>(rp.table)[static_cast<size_t>(pos) * rp.rot_half + i];
            const float x0 = (c & 1) ? other : x;
            const float x1 = (c & 1) ? x : other;
            x = (c & 1) ? x0 * cs.y + x1 * cs.x : x0 * cs.x - x1 * cs.y;
          }
        }
        if (s == 0) {
          seg.y[static_cast<size_t>(m0 + r) * seg.y_stride + n] = x;
        } else {
          const size_t at = rp.cache_off[m0 + r] + (s == 1 ? rp.k_layer_off : rp.v_layer_off) +
                            static_cast<size_t>(pos) * rp.kv_row + n;
          if (rp.cache_f16) static_cast<uint16_t*>(rp.cache)[at] = static_cast<uint16_t>(float_to_half_bits(x));
          else static_cast<float*>(rp.cache)[at] = x;
        }
      }
    } else {
      if (c < nn && r < mm) {
        float* y = seg.y + static_cast<size_t>(m0 + r) * seg.y_stride + n0 + c;
        *y = args.accumulate ? *y + x : x;
      }
    }
  };

  // Terms, then chains. Per chunk, wave w runs the MFMAs of its quarter of the blocks (each
  // once, all four results of a lane used) and forms their terms float(sumi) * d_w * d_x
  // (+ m_w * d_x * float(sumx), Q4_1) into LDS ([row][column][block]); after a barrier thread t
  // adds the chunk's terms of output (row t / 16, column t % 16) in block order. The terms and
  // the adds are the scalar table's operations in its order, so the bits are its bits.
  constexpr uint32_t TP = KC + 4;              // floats per (row, column) of terms
  constexpr uint32_t BW = KC / 4;              // blocks per wave per chunk
  float* terms = reinterpret_cast<float*>(xs + TM * KC);  // [16][16][TP]
  const uint32_t crow = tid >> 4, ccol = tid & 15;        // this thread's chain
  float acc = 0.0f;
  auto chunk = [&](uint32_t c, Raw& r) {
    const uint32_t cb = min(KC, nb - c * KC);
    expand(c, r);
    __syncthreads();
    if (c + 2 < n_chunks) load(c + 2, r);
    const uint32_t b0 = wave * BW;
    i32x4 d[BW];
#pragma unroll
    for (uint32_t i = 0; i < BW; ++i) {
      const uint2 wq = *reinterpret_cast<const uint2*>(wa + wrow * P + (b0 + i) * 8 + 2 * kq);
      const uint2 xq = *reinterpret_cast<const uint2*>(xa + col * P + (b0 + i) * 8 + 2 * kq);
      const int64_t bw = static_cast<int64_t>((static_cast<uint64_t>(wq.y) << 32) | wq.x);
      const int64_t ax = static_cast<int64_t>((static_cast<uint64_t>(xq.y) << 32) | xq.x);
      i32x4 z = {0, 0, 0, 0};
      d[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
    }
    // Blocks past cb hold stale bytes; their terms are never added.
    float t[4][BW];
#pragma unroll
    for (uint32_t i = 0; i < BW; ++i) {
      const uint32_t b = b0 + i;
      const float dw = wd[wrow * KC + b];
      const float4 dx4 = *reinterpret_cast<const float4*>(xd + b * TM + 4 * kq);  // rows 4kq..4kq+3
      const float dx[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
      if constexpr (T == Q4_1) {
        const float mw = wmn[wrow * KC + b];
        const int4 sx4 = *reinterpret_cast<const int4*>(xs + b * TM + 4 * kq);
        const int32_t sx[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
        for (uint32_t v = 0; v < 4; ++v)
          t[v][i] = static_cast<float>(d[i][v]) * dw * dx[v] + mw * dx[v] * static_cast<float>(sx[v]);
      } else {
        // Q4_0: sumi carries the -8 offset already (the weights entered as q - 8).
#pragma unroll
        for (uint32_t v = 0; v < 4; ++v) t[v][i] = static_cast<float>(d[i][v]) * dw * dx[v];
      }
    }
#pragma unroll
    for (uint32_t v = 0; v < 4; ++v) {
      float4* dst = reinterpret_cast<float4*>(terms + ((4 * kq + v) * 16 + col) * TP + b0);
#pragma unroll
      for (uint32_t i = 0; i < BW; i += 4) dst[i / 4] = make_float4(t[v][i], t[v][i + 1], t[v][i + 2], t[v][i + 3]);
    }
    __syncthreads();
    const float* tp = terms + (crow * 16 + ccol) * TP;
    if (cb == KC) {
#pragma unroll
      for (uint32_t b = 0; b < KC; b += 4) {
        const float4 q4 = *reinterpret_cast<const float4*>(tp + b);
        acc += q4.x;
        acc += q4.y;
        acc += q4.z;
        acc += q4.w;
      }
    } else {
      for (uint32_t b = 0; b < cb; ++b) acc += tp[b];
    }
    // The next chunk's expand writes only the operand and scale regions, and its barrier
    // orders these reads before the next terms are written.
  };
  Raw ra, rb;
  load(0, ra);
  if (n_chunks > 1) load(1, rb);
  for (uint32_t c = 0; c < n_chunks; c += 2) {
    chunk(c, ra);
    if (c + 1 < n_chunks) chunk(c + 1, rb);
  }
  finish(ccol, crow, acc);

}

// ---- Many activation rows (prefill, mixed passes): 65 rows and more ------------------------
// A workgroup owns TN weight rows x 64 activation rows; wave w owns activation rows
// 16w..16w+15 against all TN weight rows, so each MFMA runs once and the wave that ran it folds
// its four results: per block a lane folds TN/16 x 4 outputs, with one float4 of activation
// scales and TN/16 weight scales from LDS. The K chunks (kTileChunk blocks) load into registers
// while the previous chunk computes and expand into aligned int8 in LDS as in mfma_rows_kernel;
// the scales sit block-major ([block][row], padded) so a lane's four activation scales are one
// 16-byte read. Every segment of the call is one grid. The per-output order is the scalar
// table's: block after block, acc += float(sumi) * d_w * d_x (+ m_w * d_x * float(sumx), Q4_1).
constexpr uint32_t kTileChunk = 16;
constexpr uint32_t kTilePitch = kTileChunk * 8 + 4;  // dwords per expanded row
constexpr uint32_t kTileRows = 64;

template <uint32_t TN>
__host__ __device__ constexpr uint32_t tile_wp() { return TN + 4; }  // scale pitch, weights
template <uint32_t TM = kTileRows>
__host__ __device__ constexpr uint32_t tile_xp() { return TM + 4; }  // scale pitch, activations

template <int T, uint32_t TN, uint32_t TM = kTileRows>
__host__ __device__ constexpr size_t tile_lds() {
  const size_t scales = static_cast<size_t>(kTileChunk) * (tile_wp<TN>() + tile_xp<TM>()) * (T == Q4_1 ? 2 : 1);
  return (static_cast<size_t>(TN + TM) * kTilePitch + scales) * 4;
}

template <int T, uint32_t TN, bool SWIGLU = false, uint32_t TM = kTileRows>
__global__ __launch_bounds__(kThreads) void mfma_tile_kernel(MatvecArgs args) {
  constexpr int bs = block_bytes<T>();
  constexpr uint32_t KC = kTileChunk, P = kTilePitch;
  constexpr uint32_t WP = tile_wp<TN>(), XP = tile_xp<TM>();
  constexpr uint32_t NT = TN / 16;                      // weight sub-tiles of the tile
  // The four waves split the tile's (activation tile, weight sub-tile) pairs: with MT
  // activation tiles of 16 rows, wave w takes activation tile w % MT and NTW weight sub-tiles
  // from (w / MT) * NTW on (all NT when the tile has 64 activation rows).
  constexpr uint32_t MT = TM / 16;
  constexpr uint32_t NTW = NT * MT / 4;
  static_assert(TM == 16 || TM == 32 || TM == 64, "16, 32 or 64 activation rows");
  static_assert(NTW >= 1 && NTW * 4 == NT * MT, "whole sub-tiles per wave");
  constexpr uint32_t WI = TN * KC / kThreads;           // weight items per thread per chunk
  constexpr uint32_t XI = TM * KC / kThreads;           // activation items per thread per chunk
  constexpr uint32_t WD = item_dwords<T>(), XD = item_dwords<Q8_0>();
  static_assert(TN * KC % kThreads == 0 && TM * KC % kThreads == 0, "whole items per thread");

  extern __shared__ __attribute__((aligned(16))) uint32_t lds_tile[];
  uint32_t* wa = lds_tile;                               // [TN][P]
  uint32_t* xa = wa + TN * P;                            // [TM][P]
  float* wd = reinterpret_cast<float*>(xa + TM * P);     // [KC][WP]
  float* xd = wd + KC * WP;                              // [KC][XP]
  float* wmn = xd + KC * XP;                             // [KC][WP] (Q4_1)
  int32_t* xs = reinterpret_cast<int32_t*>(wmn + KC * WP);  // [KC][XP] (Q4_1)

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = tid >> 6;
  static_assert(!SWIGLU || TN == 64, "the SwiGLU tile pairs 32 gate rows with 32 up rows");
  int s = 0;
  if (!SWIGLU && args.n_seg > 1 && blockIdx.x >= args.seg[1].wg_begin) s = 1;
  if (!SWIGLU && args.n_seg > 2 && blockIdx.x >= args.seg[2].wg_begin) s = 2;
  const MatvecSeg seg = args.seg[s];
  // SwiGLU: tile rows 0..31 are gate rows n0.., rows 32..63 the up rows of the same outputs.
  const uint32_t n0 = SWIGLU ? blockIdx.x * 32 : (blockIdx.x - seg.wg_begin) * TN;
  const uint32_t m0 = blockIdx.y * TM;
  const uint32_t nn = SWIGLU ? 64 : min(TN, seg.n_out - n0);
  const uint32_t mm = min(TM, args.m - m0);
  const uint32_t nb = args.nb;
  const uint32_t n_chunks = (nb + KC - 1) / KC;
  const uint32_t w_pitch = nb * bs, x_pitch = nb * kBytesQ8_0;
  const uint32_t w_rows = SWIGLU ? 32 : nn;  // rows behind each weight resource
  const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(seg.w) + static_cast<size_t>(n0) * w_pitch, 0, static_cast<int>(w_rows * w_pitch),
      static_cast<int>(kRawBufferWord3));
  const __amdgpu_buffer_rsrc_t usrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(SWIGLU ? args.seg[1].w : seg.w) + static_cast<size_t>(n0) * w_pitch, 0,
      static_cast<int>(w_rows * w_pitch), static_cast<int>(kRawBufferWord3));
  const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(args.xq) + static_cast<size_t>(m0) * x_pitch, 0, static_cast<int>(mm * x_pitch),
      static_cast<int>(kRawBufferWord3));

  struct Raw {
    uint32_t w[WI][WD];
    uint32_t x[XI][XD];
  };
  // Item i of a chunk: block i % KC of row i / KC (consecutive threads, consecutive blocks).
  auto load = [&](uint32_t c, Raw& r) {
    const uint32_t b0 = c * KC;
#pragma unroll
    for (uint32_t k = 0; k < WI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      // SwiGLU: items k < WI / 2 are rows 0..31 (gate), the rest rows 32..63 (up); the choice
      // of resource is uniform per k.
      const bool upper = SWIGLU && k >= WI / 2;
      const uint32_t off = (SWIGLU ? row & 31u : row) * w_pitch + (b0 + b) * bs;
#pragma unroll
      for (uint32_t d = 0; d < WD; ++d)
        r.w[k][d] = __builtin_amdgcn_raw_buffer_load_b32(upper ? usrc : wsrc, (off & ~3u) + 4 * d, 0, 0);
    }
#pragma unroll
    for (uint32_t k = 0; k < XI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t off = row * x_pitch + (b0 + b) * kBytesQ8_0;
#pragma unroll
      for (uint32_t d = 0; d < XD; ++d)
        r.x[k][d] = __builtin_amdgcn_raw_buffer_load_b32(xsrc, (off & ~3u) + 4 * d, 0, 0);
    }
  };
  auto expand = [&](uint32_t c, const Raw& r) {
    const uint32_t b0 = c * KC;
#pragma unroll
    for (uint32_t k = 0; k < WI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t sh = (((b0 + b) * bs) & 3u) * 8;
      uint32_t v[WD];
#pragma unroll
      for (uint32_t d = 0; d < WD; ++d) v[d] = __builtin_amdgcn_alignbit(d + 1 < WD ? r.w[k][d + 1] : 0u, r.w[k][d], sh);
      uint32_t q[8];
      if constexpr (T == Q8_0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbit(v[j + 1], v[j], 16);
      } else {
        constexpr uint32_t first = T == Q4_0 ? 0 : 1;
        constexpr uint32_t bsh = T == Q4_0 ? 16 : 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t n4 = bsh ? __builtin_amdgcn_alignbit(v[first + j + 1], v[first + j], bsh) : v[first + j];
          q[j] = n4 & 0x0f0f0f0fu;
          q[j + 4] = (n4 >> 4) & 0x0f0f0f0fu;
          if constexpr (T == Q4_0) {  // q - 8 per byte (no carry crosses bytes)
            q[j] = (q[j] + 0x78787878u) ^ 0x80808080u;
            q[j + 4] = (q[j + 4] + 0x78787878u) ^ 0x80808080u;
          }
        }
      }
      uint4* dst = reinterpret_cast<uint4*>(wa + row * P + b * 8);
      dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
      dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
      wd[b * WP + row] = half_bits_to_float(v[0] & 0xffffu);
      if constexpr (T == Q4_1) wmn[b * WP + row] = half_bits_to_float(v[0] >> 16);
    }
#pragma unroll
    for (uint32_t k = 0; k < XI; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t row = i / KC, b = i - row * KC;
      const uint32_t sh = (((b0 + b) * kBytesQ8_0) & 3u) * 8;
      uint32_t v[XD];
#pragma unroll
      for (uint32_t d = 0; d < XD; ++d) v[d] = __builtin_amdgcn_alignbit(d + 1 < XD ? r.x[k][d + 1] : 0u, r.x[k][d], sh);
      uint32_t q[8];
      int32_t sum = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        q[j] = __builtin_amdgcn_alignbit(v[j + 1], v[j], 16);
        if constexpr (T == Q4_1) sum = __builtin_amdgcn_sdot4(static_cast<int32_t>(q[j]), 0x01010101, sum, false);
      }
      uint4* dst = reinterpret_cast<uint4*>(xa + row * P + b * 8);
      dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
      dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
      xd[b * XP + row] = half_bits_to_float(v[0] & 0xffffu);
      if constexpr (T == Q4_1) xs[b * XP + row] = sum;
    }
  };

  const uint32_t col = lane & 15;  // weight row within a 16-row sub-tile; A row within the wave's 16
  const uint32_t kq = lane >> 4;   // which 8 of a block's 32 elements this lane feeds
  const uint32_t arow = 16 * (wave % MT) + col;     // the A operand row (activation row in the tile)
  const uint32_t orow = 16 * (wave % MT) + 4 * kq;  // the lane's output rows: orow .. orow + 3
  const uint32_t j0 = (wave / MT) * NTW;           // the wave's first weight sub-tile
  float acc[NTW][4];
#pragma unroll
  for (uint32_t j = 0; j < NTW; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[j][v] = 0.0f;

  constexpr uint32_t kBatch = 4;  // blocks whose MFMAs are issued before their folds
  static_assert(KC % kBatch == 0, "whole batches");
  auto block_sums = [&](uint32_t b, i32x4 (&d)[NTW]) {
    const uint2 xq = *reinterpret_cast<const uint2*>(xa + arow * P + b * 8 + 2 * kq);
    const int64_t ax = static_cast<int64_t>((static_cast<uint64_t>(xq.y) << 32) | xq.x);
#pragma unroll
    for (uint32_t j = 0; j < NTW; ++j) {
      const uint2 wq = *reinterpret_cast<const uint2*>(wa + (16 * (j0 + j) + col) * P + b * 8 + 2 * kq);
      const int64_t bw = static_cast<int64_t>((static_cast<uint64_t>(wq.y) << 32) | wq.x);
      i32x4 z = {0, 0, 0, 0};
      d[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax, bw, z, 0, 0, 0);
    }
  };
  auto block_fold = [&](uint32_t b, const i32x4 (&d)[NTW]) {
    const float4 dx = *reinterpret_cast<const float4*>(xd + b * XP + orow);
    const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
    int4 sx = make_int4(0, 0, 0, 0);
    if constexpr (T == Q4_1) sx = *reinterpret_cast<const int4*>(xs + b * XP + orow);
    const int32_t sxv[4] = {sx.x, sx.y, sx.z, sx.w};
#pragma unroll
    for (uint32_t j = 0; j < NTW; ++j) {
      const float dw = wd[b * WP + 16 * (j0 + j) + col];
      float mw = 0.0f;
      if constexpr (T == Q4_1) mw = wmn[b * WP + 16 * (j0 + j) + col];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if constexpr (T == Q4_1) {
          acc[j][v] += static_cast<float>(d[j][v]) * dw * dxv[v] + mw * dxv[v] * static_cast<float>(sxv[v]);
        } else {
          acc[j][v] += static_cast<float>(d[j][v]) * dw * dxv[v];
        }
      }
    }
  };

  Raw r;
  load(0, r);
  for (uint32_t c = 0; c < n_chunks; ++c) {
    const uint32_t cb = min(KC, nb - c * KC);
    expand(c, r);
    __syncthreads();
    if (c + 1 < n_chunks) load(c + 1, r);
    if (cb == KC) {
      for (uint32_t b0 = 0; b0 < KC; b0 += kBatch) {
        i32x4 d[kBatch][NTW];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) block_sums(b0 + k, d[k]);
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) block_fold(b0 + k, d[k]);
      }
    } else {
      for (uint32_t b = 0; b < cb; ++b) {
        i32x4 d[NTW];
        block_sums(b, d);
        block_fold(b, d);
      }
    }
    __syncthreads();
  }

  if constexpr (SWIGLU) {
    // Output n0 + col (sub-tiles 0 and 2) and n0 + 16 + col (1 and 3): silu(gate) * up as
    // silu_mul_kernel forms it, then each row's 32 outputs as one Q8_0 block, quantized as
    // quantize_block_lanes does (the 16 lanes of a kq group hold the block, row rr of the tile).
    const size_t row_blocks = seg.n_out / kQK;
    auto swiglu_row = [&](uint32_t rr, float g0, float g1, float u0, float u1) {
      const float y0 = g0 / (1.0f + exp_libm(-g0)) * u0;
      const float y1 = g1 / (1.0f + exp_libm(-g1)) * u1;
      float amax = fmaxf(fabsf(y0), fabsf(y1));
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
      if (rr < mm) {
        if (seg.y != nullptr) {
          float* y = seg.y + static_cast<size_t>(m0 + rr) * seg.y_stride + n0 + col;
          y[0] = y0;
          y[16] = y1;
        }
        const float dq = amax / 127.0f;
        const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
        uint8_t* blk = args.outq + (static_cast<size_t>(m0 + rr) * row_blocks + n0 / kQK) * kBytesQ8_0;
        blk[2 + col] = static_cast<uint8_t>(static_cast<int32_t>(roundf(y0 * id)) & 0xff);
        blk[2 + 16 + col] = static_cast<uint8_t>(static_cast<int32_t>(roundf(y1 * id)) & 0xff);
        if (col == 0) *reinterpret_cast<uint16_t*>(blk) = static_cast<uint16_t>(float_to_half_bits(dq));
      }
    };
    if constexpr (TM == kTileRows) {
#pragma unroll
      for (int v = 0; v < 4; ++v) swiglu_row(orow + v, acc[0][v], acc[1][v], acc[2][v], acc[3][v]);
    } else {
      // Fewer activation rows: a row's gate and up sub-tiles sit on different waves. They meet
      // in LDS ([sub-tile][row][16] floats; the chunk loop's last barrier freed it), and wave w
      // then takes rows w * TM / 4 .., four per pass (one per 16-lane group).
      float* st = reinterpret_cast<float*>(lds_tile);
#pragma unroll
      for (uint32_t j = 0; j < NTW; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) st[((j0 + j) * TM + orow + v) * 16 + col] = acc[j][v];
      __syncthreads();
#pragma unroll
      for (uint32_t p = 0; p < TM / 16; ++p) {
        const uint32_t rr = wave * (TM / 4) + 4 * p + kq;
        swiglu_row(rr, st[rr * 16 + col], st[(TM + rr) * 16 + col], st[(2 * TM + rr) * 16 + col],
                   st[(3 * TM + rr) * 16 + col]);
      }
    }
    return;
  }
#pragma unroll
  for (uint32_t j = 0; j < NTW; ++j) {
    if (16 * (j0 + j) + col < nn) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t rr = orow + v;
        if (rr < mm) {
          float* y = seg.y + static_cast<size_t>(m0 + rr) * seg.y_stride + n0 + 16 * (j0 + j) + col;
          *y = args.accumulate ? *y + acc[j][v] : acc[j][v];
        }
      }
    }
  }
}

template <uint32_t TN, uint32_t TM = kTileRows>
int tile_launch(int type, MatvecArgs& a) {
  uint32_t wg = 0;
  for (int s = 0; s < a.n_seg; ++s) {
    a.seg[s].wg_begin = wg;
    wg += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, TN));
  }
  const dim3 grid(wg, static_cast<uint32_t>(ceil_div(a.m, TM)));
  // Dynamic LDS above 64 KB is granted per kernel, once.
  static const bool granted = [] {
    bool ok = true;
    auto grant = [&](auto kernel, size_t lds) {
      if (lds > 65536)
        ok = ok && hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds)) == hipSuccess;
    };
    grant(mfma_tile_kernel<Q8_0, TN, false, TM>, tile_lds<Q8_0, TN, TM>());
    grant(mfma_tile_kernel<Q4_0, TN, false, TM>, tile_lds<Q4_0, TN, TM>());
    grant(mfma_tile_kernel<Q4_1, TN, false, TM>, tile_lds<Q4_1, TN, TM>());
    return ok;
  }();
  if (!granted) return fail(kUnsupported, "matmul tile: the LDS grant was refused");
  switch (type) {
  case Q8_0: launch(mfma_tile_kernel<Q8_0, TN, false, TM>, grid, dim3(kThreads), tile_lds<Q8_0, TN, TM>(), a); break;
  case Q4_0: launch(mfma_tile_kernel<Q4_0, TN, false, TM>, grid, dim3(kThreads), tile_lds<Q4_0, TN, TM>(), a); break;
  case Q4_1: launch(mfma_tile_kernel<Q4_1, TN, false, TM>, grid, dim3(kThreads), tile_lds<Q4_1, TN, TM>(), a); break;
  default: return fail(kUnsupported, "matmul tile: weight type %d", type);
  }
  return check_launch("mfma_tile");
}

template <int TM, uint32_t TN = kRowsTN, bool ROPE = false, uint32_t KCH = kRowsChunk>
int rows_launch(int type, MatvecArgs& a, const RowsRope& rp = RowsRope{}) {
  uint32_t wg = 0;
  for (int s = 0; s < a.n_seg; ++s) {
    a.seg[s].wg_begin = wg;
    wg += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, TN));
  }
  const dim3 grid(wg, static_cast<uint32_t>(ceil_div(a.m, TM)));
  // The terms buffer ([16][16][KCH + 4] floats) after the operands and scales.
  constexpr size_t lds = rows_lds<TM, TN, KCH>() + 16 * 16 * (KCH + 4) * 4;
  static_assert(lds <= 163840, "within one CU's LDS");
  static const bool granted = [] {
    bool ok = true;
    auto grant = [&](auto kernel) {
      if (lds > 65536)
        ok = ok && hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds)) == hipSuccess;
    };
    grant(mfma_rows_kernel<Q8_0, TM, TN, ROPE, KCH>);
    grant(mfma_rows_kernel<Q4_0, TM, TN, ROPE, KCH>);
    grant(mfma_rows_kernel<Q4_1, TM, TN, ROPE, KCH>);
    return ok;
  }();
  if (!granted) return fail(kUnsupported, "matmul rows: the LDS grant was refused");
  switch (type) {
  case Q8_0: launch(mfma_rows_kernel<Q8_0, TM, TN, ROPE, KCH>, grid, dim3(kThreads), lds, a, rp); break;
  case Q4_0: launch(mfma_rows_kernel<Q4_0, TM, TN, ROPE, KCH>, grid, dim3(kThreads), lds, a, rp); break;
  case Q4_1: launch(mfma_rows_kernel<Q4_1, TM, TN, ROPE, KCH>, grid, dim3(kThreads), lds, a, rp); break;
  default: return fail(kUnsupported, "matmul rows: weight type %d", type);
  }
  return check_launch(ROPE ? "mfma_rows (rope)" : "mfma_rows");
}

// Weight rows per workgroup: 8 when that grid is still one round of workgroups (at most 256),
// else 16 when that one is (so the 64-block chunks apply: q|k|v of C4 at 16 rows 7.2 -> 5.8 us),
// else 8 while 16 would leave CUs without a workgroup, else 16.
bool rows_narrow(const MatvecArgs& a) {
  uint32_t wg8 = 0, wg16 = 0;
  for (int s = 0; s < a.n_seg; ++s) {
    wg8 += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, 8));
    wg16 += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, kRowsTN));
  }
  const uint64_t tiles = ceil_div(a.m, 16u);
  if (wg8 * tiles <= 256) return true;
  if (wg16 * tiles <= 256) return false;
  return wg16 * tiles < 256;
}

// Chunks of 64 blocks where the grid is one round of workgroups (their LDS then holds one per
// CU) and the row is whole 64-block chunks: C4 down at 16 / 32 rows 15.3 / 18.8 -> 14.8 / 17.1 us,
// wo 5.5 / 6.3 -> 5.1 / 5.7. Otherwise 32 (q|k|v of C4, C5's matrices, 64 rows: slower at 64).
template <uint32_t TN, bool ROPE>
int rows_launch_chunked(int type, MatvecArgs& a, const RowsRope& rp = RowsRope{}) {
  uint32_t wg = 0;
  for (int s = 0; s < a.n_seg; ++s) wg += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, TN));
  if (static_cast<uint64_t>(wg) * ceil_div(a.m, 16u) <= 256 && a.nb % 64 == 0)
    return rows_launch<16, TN, ROPE, 64>(type, a, rp);
  return rows_launch<16, TN, ROPE, kRowsChunk>(type, a, rp);
}

}  // namespace

bool matmul_q8_rows_fits(int type, const MatvecArgs& a, bool many_rows) {
  if (a.m < 1 || (!many_rows && a.m > kRowsMaxM) || a.nb == 0) return false;
  if (type != Q8_0 && type != Q4_0 && type != Q4_1) return false;
  const uint32_t bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  // Dword loads: every weight row and activation row starts on a 4-byte boundary, and the
  // buffer ranges (rows x row bytes) fit a 32-bit record count.
  uintptr_t bases = reinterpret_cast<uintptr_t>(a.xq);
  for (int s = 0; s < a.n_seg; ++s) {
    bases |= reinterpret_cast<uintptr_t>(a.seg[s].w);
    if (static_cast<uint64_t>(a.nb) * bs * 64 >= (uint64_t(1) << 31)) return false;
  }
  if (static_cast<uint64_t>(a.nb) * kBytesQ8_0 * 64 >= (uint64_t(1) << 31)) return false;
  return (bases & 3u) == 0 && (a.nb * bs) % 4 == 0 && (a.nb * kBytesQ8_0) % 4 == 0;
}

constexpr uint32_t kDecodeTileWg = 256;  // workgroups a decode matrix needs for the tile kernel

// From 128 tiles of 64 weight rows (33..64 rows, Q4_0): 8192 x 2048 24.4 -> 15.8 us, 9728 x 896
// 20.7 -> 10.3, 16384 x 2048 46.0 -> 20.7; at 48 tiles and fewer the rows kernel stays ahead.
bool matmul_q8_tile_fills(const MatvecArgs& a) {
  if (a.m < 33 || a.m > kRowsMaxM) return false;
  uint32_t wg64 = 0;
  for (int s = 0; s < a.n_seg; ++s) wg64 += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, 64));
  return wg64 >= 128;
}

template <uint32_t TM>
int swiglu_launch(int type, MatvecArgs& a) {
  const dim3 grid(static_cast<uint32_t>(a.seg[0].n_out / 32), static_cast<uint32_t>(ceil_div(a.m, TM)));
  static const bool granted = [] {
    bool ok = true;
    auto grant = [&](auto kernel, size_t lds) {
      if (lds > 65536)
        ok = ok && hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds)) == hipSuccess;
    };
    grant(mfma_tile_kernel<Q8_0, 64, true, TM>, tile_lds<Q8_0, 64, TM>());
    grant(mfma_tile_kernel<Q4_0, 64, true, TM>, tile_lds<Q4_0, 64, TM>());
    grant(mfma_tile_kernel<Q4_1, 64, true, TM>, tile_lds<Q4_1, 64, TM>());
    return ok;
  }();
  if (!granted) return fail(kUnsupported, "matmul swiglu: the LDS grant was refused");
  switch (type) {
  case Q8_0: launch(mfma_tile_kernel<Q8_0, 64, true, TM>, grid, dim3(kThreads), tile_lds<Q8_0, 64, TM>(), a); break;
  case Q4_0: launch(mfma_tile_kernel<Q4_0, 64, true, TM>, grid, dim3(kThreads), tile_lds<Q4_0, 64, TM>(), a); break;
  case Q4_1: launch(mfma_tile_kernel<Q4_1, 64, true, TM>, grid, dim3(kThreads), tile_lds<Q4_1, 64, TM>(), a); break;
  default: return fail(kUnsupported, "matmul swiglu: weight type %d", type);
  }
  return check_launch("mfma_tile (swiglu)");
}

int matmul_q8_swiglu_launch(int type, MatvecArgs& a) {
  MatvecArgs probe = a;
  probe.n_seg = 2;
  if (a.n_seg != 2 || a.outq == nullptr || a.seg[0].n_out != a.seg[1].n_out || a.seg[0].n_out % kQK != 0 ||
      !matmul_q8_rows_fits(type, probe, true))
    return fail(kUnsupported, "matmul swiglu: shape or alignment");
  // Decode-sized calls (up to kRowsMaxM rows) take the fused tile when it has at least 128
  // workgroups (one per 32 outputs: FFNs of 4096 and up); with fewer the caller runs the matmul
  // and silu_mul apart. C5's 4864-wide FFN (152 workgroups) gained 2-4 % against the rows
  // kernel and silu_mul.
  if (a.m <= kRowsMaxM && a.seg[0].n_out / 32 < 128)
    return fail(kUnsupported, "matmul swiglu: %u outputs give too few workgroups for %u rows", a.seg[0].n_out, a.m);
  if (a.m <= 16) return swiglu_launch<16>(type, a);
  if (a.m <= 32) return swiglu_launch<32>(type, a);
  return swiglu_launch<kTileRows>(type, a);
}

int matmul_q8_tile_launch(int type, MatvecArgs& a) {
  if (!matmul_q8_rows_fits(type, a, true)) return fail(kUnsupported, "matmul tile: shape or alignment");
  // 64-row weight tiles when they give the chip a few workgroups per CU, else 32-row tiles.
  uint32_t wg64 = 0;
  for (int s = 0; s < a.n_seg; ++s) wg64 += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, 64));
  const uint64_t tiles64 = static_cast<uint64_t>(wg64) * ceil_div(a.m, kTileRows);
  if (tiles64 >= 768) return tile_launch<64>(type, a);
  return tile_launch<32>(type, a);
}

int matmul_q8_rows_launch(int type, MatvecArgs& a) {
  if (!matmul_q8_rows_fits(type, a)) return fail(kUnsupported, "matmul rows: shape or alignment");
  // A matrix wide enough for kDecodeTileWg workgroups of 64 weight rows (16 activation rows) or
  // 32 (32 activation rows) takes the tile kernel: each workgroup reads and expands the
  // activations once for all its weight rows, where the rows kernel's 16-row workgroups read
  // them two or four times as often (gate|up of C4 at 32 rows: 27.3 -> 14.2 us).
  uint32_t wg64 = 0, wg32 = 0;
  for (int s = 0; s < a.n_seg; ++s) {
    wg64 += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, 64));
    wg32 += static_cast<uint32_t>(ceil_div(a.seg[s].n_out, 32));
  }
  if (a.m <= 16) {
    if (wg64 >= kDecodeTileWg) return tile_launch<64, 16>(type, a);
  } else if (a.m <= 32) {
    if (wg32 >= kDecodeTileWg) return tile_launch<32, 32>(type, a);
  }
  // Up to 32 rows go in tiles of 16 activation rows (two tiles along the grid's second axis
  // above 16): a workgroup of 32 rows would run twice the folds and read twice the activations
  // for the same weight rows (C4 down at 32 rows 26.9 -> 21.0 us).
  return rows_narrow(a) ? rows_launch_chunked<8, false>(type, a) : rows_launch_chunked<kRowsTN, false>(type, a);
}

int matmul_q8_rows_rope_launch(int type, MatvecArgs& a, const RowsRope& rp) {
  if (a.n_seg != 3 || !matmul_q8_rows_fits(type, a)) return fail(kUnsupported, "matmul rows (rope): shape or alignment");
  return rows_narrow(a) ? rows_launch_chunked<8, true>(type, a, rp) : rows_launch_chunked<kRowsTN, true>(type, a, rp);
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
