// Q6_K weights against float activations: the output and embedding matrices' path, following
// trickymind1324/axon-infer src/kernels/ref/quant.cpp:183-194 with the super-block decoding of
// src/core/dtype.cpp:312-336 (ggml's Q6_K: ql[128], qh[64], int8 scales[16], fp16 d).
//
// The scalar table dequantizes each weight as (d * scale) * q and adds value * x to one float
// accumulator per output, element after element. That dequantized value is exact in binary32
// (an 11-bit half scale times a 7-bit int8 scale times a 5-bit |q| fits 24 bits), so it is
// computed here as fma(d * scale, q + 32, -32 * d * scale) (one rounding of an exact value);
// the product with x and the add then follow the scalar table's order. Every output is
// bit-identical to the scalar table's.
//
// One lane owns one output row and walks it in element order with its super-block in
// registers. Two ways to get the super-blocks there:
//  * q6k_stream_kernel (rows a multiple of 4 bytes, i.e. an even super-block count: every
//    model shape): a wave's 64 rows move one super-block column at a time through the wave's
//    own LDS tile, copied row by row by LDS-DMA buffer loads (contiguous 212-byte runs); each
//    lane then reads its own window. The next column's copies are in flight while the lanes
//    work on the current one. The column's activations travel the same way and are read as
//    LDS broadcasts.
//  * matvec_q6k_kernel (any 2-byte-aligned rows): each lane fetches its own super-blocks with
//    per-lane loads, double-buffered in registers.
//
// The planar copy made at upload (q6k_repack_kernel) is what the model streams. Over it, several
// activation rows run q6k_planar_kernel (one lane per output row, up to 8 rows per lane). One
// activation row splits the products from the sums instead, since a lane that decodes and
// chains by itself runs ~14 ns an element: q6k_planar_chain_kernel (a short matrix: every
// thread forms products into LDS, then one lane per row adds them) and q6k_planar_ring_kernel
// (products streamed to the chains through two LDS slots, 64 rows per workgroup). The sums keep
// the scalar table's order in every kernel.
#include <atomic>
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr uint32_t kQ6MaxRows = 8;  // activation rows per workgroup of the planar kernel
constexpr uint32_t kChainMaxOut = 2048;  // one activation row up to this many outputs: the chain kernel

constexpr int kThreads = 256;  // rows per workgroup
constexpr int kWin = 53;       // dwords covering one super-block plus its 2-byte misalignment

// The super-block at sb (2-byte aligned) as 53 dwords starting at sb rounded down to 4 bytes.
// Dwords 1..51 are loaded whole; the first and last come from 2-byte loads (h[0..3]) so no
// access leaves the super-block, and are assembled where they are used.
struct SuperBlock {
  uint32_t w[kWin];
  uint32_t h[4];
};

__device__ __forceinline__ void q6k_fetch(const uint8_t* sb, SuperBlock& s) {
  const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb) & 2u);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(sb - sh);
#pragma unroll
  for (int k = 1; k < kWin - 1; ++k) s.w[k] = __builtin_nontemporal_load(base + k);
  s.h[0] = *reinterpret_cast<const uint16_t*>(sb);
  s.h[1] = *reinterpret_cast<const uint16_t*>(sb + 2);
  s.h[2] = *reinterpret_cast<const uint16_t*>(sb + 206);
  s.h[3] = *reinterpret_cast<const uint16_t*>(sb + 208);
}

template <int MM>
__device__ __forceinline__ void q6k_superblock(SuperBlock& s, uint32_t sh, const float* xs, uint32_t n_in,
                                               uint32_t e_base, float (&acc)[MM]) {
  uint32_t (&w)[kWin] = s.w;
  w[0] = sh ? (s.h[0] << 16) : (s.h[0] | (s.h[1] << 16));
  w[kWin - 1] = sh ? (s.h[2] | (s.h[3] << 16)) : s.h[3];
  const uint32_t bits = 8 * sh;
  // dword at byte offset o (a multiple of 4) of the super-block
  auto dw = [&](int o) { return __builtin_amdgcn_alignbit(w[o / 4 + 1], w[o / 4], bits); };
  const float d = half_bits_to_float(sh ? (w[kWin - 1] >> 16) : (w[kWin - 1] & 0xffffu));
  uint32_t sc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sc[i] = dw(192 + 4 * i);
#pragma unroll
  for (int n = 0; n < 2; ++n) {
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int si = n * 8 + qi * 2 + half;
        const float scale = static_cast<float>(static_cast<int8_t>((sc[si >> 2] >> (8 * (si & 3))) & 0xffu));
        const float ds = d * scale;       // exact
        const float neg32 = -32.0f * ds;  // exact
#pragma unroll
        for (int l4 = 0; l4 < 4; ++l4) {
          const int l = 16 * half + 4 * l4;
          const uint32_t lw = dw(64 * n + 32 * (qi & 1) + l);
          const uint32_t hw = dw(128 + 32 * n + l);
          const uint32_t q = ((lw >> (4 * (qi >> 1))) & 0x0f0f0f0fu) | (((hw >> (2 * qi)) & 0x03030303u) << 4);
          const uint32_t e0 = e_base + 128 * n + 32 * qi + l;
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            const float4 x4 = *reinterpret_cast<const float4*>(xs + m * n_in + e0);
            const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = fmaf(ds, static_cast<float>((q >> (8 * e)) & 0xffu), neg32);  // (d*scale)*(q-32)
              acc[m] += v * xv[e];
            }
          }
        }
      }
    }
  }
}

template <int MM>
__global__ __launch_bounds__(kThreads) void matvec_q6k_kernel(MatvecArgs args, uint32_t n_in) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [MM][n_in]
  const uint32_t tid = threadIdx.x;
  const uint32_t nsb = args.nb;
  const MatvecSeg seg = args.seg[0];
  const float* x = reinterpret_cast<const float*>(args.xq);
  for (uint32_t i = tid; i < MM * n_in; i += kThreads) xs[i] = x[i];
  __syncthreads();
  const uint32_t row = blockIdx.x * kThreads + tid;
  if (row >= seg.n_out) return;
  const uint8_t* rp = seg.w + static_cast<size_t>(row) * nsb * kBytesQ6_K;
  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
  // Two super-blocks per trip so the double buffer swaps roles without register copies. Every
  // fetch is unconditional (the index is clamped to the last super-block) so the compiler can
  // count the loads in flight and wait only for the buffer about to be used.
  SuperBlock a, b;
  const uint32_t last = nsb - 1;
  auto sb_at = [&](uint32_t c) { return rp + static_cast<size_t>(min(c, last)) * kBytesQ6_K; };
  auto sh_at = [&](uint32_t c) { return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb_at(c)) & 2u); };
  q6k_fetch(sb_at(0), a);
  for (uint32_t c = 0; c < nsb; c += 2) {
    q6k_fetch(sb_at(c + 1), b);
    q6k_superblock<MM>(a, sh_at(c), xs, n_in, c * kQKK, acc);
    q6k_fetch(sb_at(c + 2), a);
    if (c + 1 < nsb) q6k_superblock<MM>(b, sh_at(c + 1), xs, n_in, (c + 1) * kQKK, acc);
  }
#pragma unroll
  for (int m = 0; m < MM; ++m) seg.y[static_cast<size_t>(m) * seg.y_stride + row] = acc[m];
}


// One super-block window (53 dwords, whole) of this lane's row in element order: the same
// arithmetic as q6k_superblock, with the super-block's activations at x[m * 256 + e] (LDS).
template <int MM>
__device__ __forceinline__ void q6k_window(const uint32_t (&w)[kWin], uint32_t sh, const float* x,
                                           float (&acc)[MM]) {
  const uint32_t bits = 8 * sh;
  auto dw = [&](int o) { return __builtin_amdgcn_alignbit(w[o / 4 + 1], w[o / 4], bits); };
  const float d = half_bits_to_float(sh ? (w[kWin - 1] >> 16) : (w[kWin - 1] & 0xffffu));
  uint32_t sc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sc[i] = dw(192 + 4 * i);
#pragma unroll
  for (int n = 0; n < 2; ++n) {
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int si = n * 8 + qi * 2 + half;
        const float scale = static_cast<float>(static_cast<int8_t>((sc[si >> 2] >> (8 * (si & 3))) & 0xffu));
        const float ds = d * scale;       // exact
        const float neg32 = -32.0f * ds;  // exact
#pragma unroll
        for (int l4 = 0; l4 < 4; ++l4) {
          const int l = 16 * half + 4 * l4;
          const uint32_t lw = dw(64 * n + 32 * (qi & 1) + l);
          const uint32_t hw = dw(128 + 32 * n + l);
          const uint32_t q = ((lw >> (4 * (qi >> 1))) & 0x0f0f0f0fu) | (((hw >> (2 * qi)) & 0x03030303u) << 4);
          const uint32_t e0 = 128 * n + 32 * qi + l;
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            const float4 x4 = *reinterpret_cast<const float4*>(x + m * kQKK + e0);
            const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = fmaf(ds, static_cast<float>((q >> (8 * e)) & 0xffu), neg32);  // (d*scale)*(q-32)
              acc[m] += v * xv[e];
            }
          }
        }
      }
    }
  }
}

// Rows of an even super-block count: the window of super-block c starts at byte
// 210c - 2 (c odd) or 210c (c even), a multiple of 4, and its 212 bytes stay inside the row.
//
// One wave per workgroup, one output row per lane. Per super-block column the wave copies its
// rows' windows straight from HBM into its LDS tile [64][53] with LDS-DMA buffer loads (load
// k: lanes 0..52 move row k's 53 dwords, 212 contiguous bytes), and the column's activations
// into a double-buffered LDS chunk the same way. Each lane reads its window into registers, the
// wave issues the next column's copies into the same tile, and the lanes work on the window
// while those copies are in flight. Every LDS access stays inside the wave, so waits on the
// wave's own counters order them; no workgroup barrier is needed.
constexpr int kStreamRows = 64;


__device__ __forceinline__ void wait_all() {
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
}

template <int MM>
__global__ __launch_bounds__(kStreamRows) void q6k_stream_kernel(MatvecArgs args, uint32_t n_in) {
  extern __shared__ __attribute__((aligned(16))) uint32_t tile[];  // [64 rows][kWin], then x [2][MM][256]
  float* xc = reinterpret_cast<float*>(tile + kStreamRows * kWin);
  const uint32_t lane = threadIdx.x;
  const uint32_t nsb = args.nb;
  const uint32_t row_bytes = nsb * kBytesQ6_K;
  const MatvecSeg seg = args.seg[0];
  const uint32_t row0 = blockIdx.x * kStreamRows;
  const uint32_t rows = min(static_cast<uint32_t>(kStreamRows), seg.n_out - row0);
  const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(seg.w) + static_cast<size_t>(row0) * row_bytes, 0, static_cast<int>(rows * row_bytes),
      static_cast<int>(kRawBufferWord3));
  const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(args.xq), 0, static_cast<int>(MM * n_in * 4), static_cast<int>(kRawBufferWord3));
  const uint32_t voff = 4 * lane;
  auto window_start = [](uint32_t c) { return c * kBytesQ6_K - 2 * (c & 1); };
  // Copies of column c: rows below `rows` only (uniform), lanes below 53 for the windows.
  // Rows past the last one re-copy the last row (uniform clamp, no branch per row).
  const uint32_t last_off = (rows - 1) * row_bytes;
  auto copy_column = [&](uint32_t c) {
    uint32_t soff = window_start(c);
    if (lane < kWin) {
#pragma unroll
      for (int k = 0; k < kStreamRows; ++k) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wsrc, as_lds(tile + k * kWin), 4, voff,
                                                 min(soff, last_off + window_start(c)), 0, 0);
        soff += row_bytes;
      }
    }
    float* xb = xc + (c & 1) * MM * kQKK;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
#pragma unroll
      for (int p = 0; p < kQKK / 64; ++p) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xsrc, as_lds(xb + m * kQKK + 64 * p), 4, voff,
            4 * (m * n_in + c * kQKK + 64 * p), 0, 0);
      }
    }
  };
  copy_column(0);
  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
  for (uint32_t c = 0; c < nsb; ++c) {
    wait_all();  // column c is in LDS; the previous column's activation reads are done
    uint32_t w[kWin];
#pragma unroll
    for (int j = 0; j < kWin; ++j) w[j] = tile[lane * kWin + j];
    wait_all();  // every lane holds its window: the tile may be refilled
    if (c + 1 < nsb) copy_column(c + 1);
    q6k_window<MM>(w, 2 * (c & 1), xc + (c & 1) * MM * kQKK, acc);
  }
  if (lane < rows) {
#pragma unroll
    for (int m = 0; m < MM; ++m) seg.y[static_cast<size_t>(m) * seg.y_stride + row0 + lane] = acc[m];
  }
}

// ---- The planar layout (one-time repack at upload) --------------------------------------
// Super-block column c of an [n_out][nsb] matrix becomes a region of q6k_planar_column_bytes:
// 13 slices [n_out][16 bytes], slice s holding bytes 16s..16s+15 of each row's super-block
// (ql 0..127, qh 128..191, scales 192..207), then the d plane [n_out] of halves, padded to 16
// bytes. A lane's loads of its row are aligned 16-byte loads, and lane i of a wave reads the
// 16 bytes after lane i-1's: one load instruction moves 1 KB of one slice, contiguous.

__global__ __launch_bounds__(256) void q6k_repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         uint32_t n_out, uint32_t nsb, size_t col_bytes) {
  const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<size_t>(n_out) * nsb) return;
  const uint32_t row = static_cast<uint32_t>(i % n_out);
  const uint32_t c = static_cast<uint32_t>(i / n_out);
  const uint16_t* sb = reinterpret_cast<const uint16_t*>(src + (static_cast<size_t>(row) * nsb + c) * kBytesQ6_K);
  uint8_t* col = dst + static_cast<size_t>(c) * col_bytes;
#pragma unroll
  for (int s = 0; s < 13; ++s) {
    uint32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = sb[8 * s + 2 * k] | (static_cast<uint32_t>(sb[8 * s + 2 * k + 1]) << 16);
    *reinterpret_cast<uint4*>(col + static_cast<size_t>(s) * 16 * n_out + 16 * static_cast<size_t>(row)) =
        make_uint4(v[0], v[1], v[2], v[3]);
  }
  reinterpret_cast<uint16_t*>(col + static_cast<size_t>(208) * n_out)[row] = sb[104];
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct PlanarBlock {
  u32x4 q[13];
  uint32_t d;
};

__device__ __forceinline__ void planar_fetch(const uint8_t* col, uint32_t n_out, uint32_t row, PlanarBlock& b) {
#pragma unroll
  for (int s = 0; s < 13; ++s)
    b.q[s] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(col + static_cast<size_t>(s) * 16 * n_out) + row);
  b.d = reinterpret_cast<const uint16_t*>(col + static_cast<size_t>(208) * n_out)[row];
}

// The activations of a column, read through the constant address space: every lane of a wave
// reads the same values, so they arrive by scalar loads as instruction operands (the kernel
// never writes them).
using cfloat = const __attribute__((address_space(4))) float;

// The row's super-block in element order, as q6k_window: value (d*scale)*(q-32), then
// acc += value * x, element after element. Activation row m of the column at x + xoff[m].
template <int MM>
__device__ __forceinline__ void planar_superblock(const PlanarBlock& b, cfloat* x, const uint32_t (&xoff)[MM],
                                                  float (&acc)[MM]) {
  auto dw = [&](int o) {
    return b.q[o / 16][(o / 4) & 3];
  };
  const float d = half_value(b.d);
  uint32_t sc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sc[i] = dw(192 + 4 * i);
  // 64 steps of 4 elements (step s: elements 4s .. 4s+3, in order). Each step's activations
  // (4 per row) are loaded kAhead steps ahead into a ring of register sets; the empty asm keeps
  // the compiler from hoisting more loads above it, which would run the scalar registers out.
  constexpr int kAhead = MM >= 4 ? 1 : 8 / MM;
  float xr[kAhead + 1][MM][4];
  auto xload = [&](int st, float (&xv)[MM][4]) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      cfloat* xm = x + xoff[m] + 4 * st;
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[m][e] = xm[e];
    }
  };
  auto step = [&](int st, const float (&xv)[MM][4]) {
    const int n = st / 32, qi = (st / 8) % 4, half = (st / 4) % 2, l4 = st % 4;
    const int si = n * 8 + qi * 2 + half;
    const float scale = static_cast<float>(static_cast<int8_t>((sc[si >> 2] >> (8 * (si & 3))) & 0xffu));
    const float ds = d * scale;       // exact
    const float neg32 = -32.0f * ds;  // exact
    const int l = 16 * half + 4 * l4;
    const uint32_t lw = dw(64 * n + 32 * (qi & 1) + l);
    const uint32_t hw = dw(128 + 32 * n + l);
    const uint32_t q = ((lw >> (4 * (qi >> 1))) & 0x0f0f0f0fu) | (((hw >> (2 * qi)) & 0x03030303u) << 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = fmaf(ds, static_cast<float>((q >> (8 * e)) & 0xffu), neg32);  // (d*scale)*(q-32)
#pragma unroll
      for (int m = 0; m < MM; ++m) acc[m] += v * xv[m][e];
    }
  };
  if constexpr (kAhead == 1) {
    xload(0, xr[0]);
#pragma unroll
    for (int st = 0; st < 64; st += 2) {
      xload(st + 1, xr[1]);
      asm volatile("" ::: "memory");
      step(st, xr[0]);
      if (st + 2 < 64) xload(st + 2, xr[0]);
      asm volatile("" ::: "memory");
      step(st + 1, xr[1]);
    }
  } else {
#pragma unroll
    for (int st = 0; st < kAhead; ++st) xload(st, xr[st]);
#pragma unroll
    for (int st = 0; st < 64; ++st) {
      if (st + kAhead < 64) xload(st + kAhead, xr[(st + kAhead) % (kAhead + 1)]);
      asm volatile("" ::: "memory");
      step(st, xr[st % (kAhead + 1)]);
    }
  }
}

// One lane per output row, TH rows per workgroup (TH = 64 spreads a short matrix over more
// CUs); workgroup (blockIdx.x, blockIdx.y) takes activation rows [MM * blockIdx.x, +MM) against
// output rows [TH * blockIdx.y, +TH), so the workgroups that share a weight slice are launched
// one after another. The chunk's activation rows are read by scalar loads (rows past m_total
// read the chunk's last row; their outputs are not stored); the row's super-blocks are
// double-buffered in registers, two per trip so the buffers swap roles without copies, every
// fetch unconditional (clamped to the last column). Read as LDS broadcasts, the activations
// cost the LDS a full 1 KB per wave and read for 4 elements of one row; as scalar operands
// they cost nothing there (32 rows of 128256 x 2048: 571 -> 503 us; 4 rows 101 -> 81 us).
template <int MM, int TH>
__global__ __launch_bounds__(TH) void q6k_planar_kernel(MatvecArgs args, uint32_t n_in, size_t col_bytes,
                                                        uint32_t m_total) {
  const uint32_t tid = threadIdx.x;
  const uint32_t nsb = args.nb;
  const MatvecSeg seg = args.seg[0];
  const uint32_t m0 = blockIdx.x * MM;
  const uint32_t mm = min(static_cast<uint32_t>(MM), m_total - m0);
  // Rows past m_total read the chunk's last row (their outputs are not stored).
  cfloat* xs = (cfloat*)(reinterpret_cast<const float*>(args.xq) + static_cast<size_t>(m0) * n_in);
  uint32_t xoff[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) xoff[m] = min(static_cast<uint32_t>(m), mm - 1) * n_in;
  // The activations were just written, possibly through another XCD's L2: one round of vector
  // loads brings them into this one's, so the scalar loads that follow hit it.
  {
    const float4* xv = reinterpret_cast<const float4*>(args.xq) + static_cast<size_t>(m0) * n_in / 4;
    for (uint32_t i = tid; i < mm * n_in / 4; i += TH) {
      const float4 t = xv[i];
      asm volatile("" ::"v"(t.x));
    }
    __syncthreads();
  }
  const uint32_t row_id = blockIdx.y * TH + tid;
  // With greedy keys to form, every lane stays to the end (the reduction needs them all): a lane
  // past the last row reads the last row and neither stores nor offers a key.
  if (row_id >= seg.n_out && (MM != 1 || args.argmax_part == nullptr)) return;
  const bool live = row_id < seg.n_out;
  const uint32_t row = live ? row_id : seg.n_out - 1;
  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
  const uint32_t last = nsb - 1;
  auto col_at = [&](uint32_t c) { return seg.w + static_cast<size_t>(min(c, last)) * col_bytes; };
  PlanarBlock a, b;
  planar_fetch(col_at(0), seg.n_out, row, a);
  for (uint32_t c = 0; c < nsb; c += 2) {
    planar_fetch(col_at(c + 1), seg.n_out, row, b);
    planar_superblock<MM>(a, xs + c * kQKK, xoff, acc);
    planar_fetch(col_at(c + 2), seg.n_out, row, a);
    if (c + 1 < nsb) planar_superblock<MM>(b, xs + (c + 1) * kQKK, xoff, acc);
  }
#pragma unroll
  for (int m = 0; m < MM; ++m)
    if (live && m < static_cast<int>(mm)) seg.y[static_cast<size_t>(m0 + m) * seg.y_stride + row] = acc[m];
  if constexpr (MM == 1) {
    if (args.argmax_part != nullptr) {
      // argmax_partial_kernel's key over this workgroup's outputs (NaN never a key).
      __shared__ uint64_t red[TH / 64];
      uint64_t key = live && acc[0] == acc[0] ? argmax_key(acc[0], row) : 0;
      key = max_key_wave(key);
      if (TH > 64) {
        if ((tid & 63) == 0) red[tid >> 6] = key;
        __syncthreads();
        if (tid == 0)
          for (uint32_t w = 1; w < TH / 64; ++w) key = red[w] > key ? red[w] : key;
      }
      if (tid == 0) args.argmax_part[blockIdx.y] = key;
    }
  }
}

// One activation row against a short matrix: R output rows per workgroup, the products apart
// from the sums. The threads take units of (super-block, quarter, row) and write the quarter's
// 64 products v * x in element order into LDS ([super-block][row][256 + 4 pad] floats); then lane
// r of the first wave adds row r's products in order, four per 16-byte read. The floats are those
// of q6k_planar_kernel (each product rounded, then added in element order); the chain no longer
// waits for the decoding and the multiplies, which with one lane per row set its pace, and a short
// matrix spreads over R-row workgroups instead of 64-row ones.
constexpr uint32_t kChainPitch = kQKK + 4;  // floats per (super-block, row) of products

// Quarter Qr of a super-block is its elements 64 Qr .. 64 Qr + 63 (planar_superblock's steps
// 16 Qr .. 16 Qr + 15). It reads 6 of the 13 slices of its row (the low bits of its half, 4;
// the high bits, 2), word Qr of the scales slice, and d; the rest stays zero.
template <int Qr>
__device__ __forceinline__ void quarter_fetch(const uint8_t* col, uint32_t n_out, uint32_t row, PlanarBlock& b) {
  constexpr int n = Qr / 2;
  b.d = reinterpret_cast<const uint16_t*>(col + static_cast<size_t>(208) * n_out)[row];
#pragma unroll
  for (int s = 0; s < 12; ++s) {
    if ((s >= 4 * n && s < 4 * n + 4) || s == 8 + 2 * n || s == 9 + 2 * n)
      b.q[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(col + static_cast<size_t>(s) * 16 * n_out) + row);
    else
      b.q[s] = u32x4{0, 0, 0, 0};
  }
  // Of the scales the quarter reads one word, its four 16-element scales (a wider load would
  // leave registers that the compiler reuses while the load is still landing).
  b.q[12] = u32x4{0, 0, 0, 0};
  b.q[12][Qr] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(col + static_cast<size_t>(12) * 16 * n_out) +
                                           4 * static_cast<size_t>(row) + Qr);
}

// Products v * x of the quarter's steps S0 .. S0 + NS - 1 (4 elements each), v = (d*scale)*(q-32)
// as planar_superblock forms it; xs holds those steps' activations, pv receives the products.
template <int Qr, int S0 = 0, int NS = 16>
__device__ __forceinline__ void quarter_products(const PlanarBlock& b, const float4* xs, float4* pv) {
  auto dw = [&](int o) { return b.q[o / 16][(o / 4) & 3]; };
  const float d = half_value(b.d);
#pragma unroll
  for (int st = 16 * Qr + S0; st < 16 * Qr + S0 + NS; ++st) {
    const int n = st / 32, qi = (st / 8) % 4, half = (st / 4) % 2, l4 = st % 4;
    const int si = n * 8 + qi * 2 + half;
    const float scale = static_cast<float>(static_cast<int8_t>((dw(192 + 4 * (si >> 2)) >> (8 * (si & 3))) & 0xffu));
    const float ds = d * scale;
    const float neg32 = -32.0f * ds;
    const int l = 16 * half + 4 * l4;
    const uint32_t lw = dw(64 * n + 32 * (qi & 1) + l);
    const uint32_t hw = dw(128 + 32 * n + l);
    const uint32_t q = ((lw >> (4 * (qi >> 1))) & 0x0f0f0f0fu) | (((hw >> (2 * qi)) & 0x03030303u) << 4);
    const float4 xv = xs[st - 16 * Qr - S0];
    float4& o = pv[st - 16 * Qr - S0];
    o.x = fmaf(ds, static_cast<float>(q & 0xffu), neg32) * xv.x;
    o.y = fmaf(ds, static_cast<float>((q >> 8) & 0xffu), neg32) * xv.y;
    o.z = fmaf(ds, static_cast<float>((q >> 16) & 0xffu), neg32) * xv.z;
    o.w = fmaf(ds, static_cast<float>(q >> 24), neg32) * xv.w;
  }
}

// One unit of the chain kernel: the quarter's products of one row into dst[16 Qr ..].
template <int Qr>
__device__ __forceinline__ void chain_quarter(const uint8_t* col, uint32_t n_out, uint32_t row, const float4* xc,
                                              float4* dst) {
  PlanarBlock b;
  quarter_fetch<Qr>(col, n_out, row, b);
  // Every activation load is issued before the first step (the scheduling barrier keeps the
  // compiler from sinking them between the steps, where each would wait out its own latency).
  float4 xs[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) xs[i] = xc[16 * Qr + i];
  __builtin_amdgcn_sched_barrier(0);
  float4 pv[16];
  quarter_products<Qr>(b, xs, pv);
#pragma unroll
  for (int i = 0; i < 16; ++i) dst[16 * Qr + i] = pv[i];
}

template <int R>
__global__ __launch_bounds__(256) void q6k_planar_chain_kernel(MatvecArgs args, uint32_t n_in, size_t col_bytes) {
  extern __shared__ __attribute__((aligned(16))) float prods[];
  const uint32_t nsb = args.nb;
  const MatvecSeg seg = args.seg[0];
  const uint32_t r0 = blockIdx.x * R;
  const float* x = reinterpret_cast<const float*>(args.xq);
  // Wave w takes quarter w of every unit (the quarter's code is chosen per wave, not per lane);
  // its lanes take (super-block, row) pairs cr = c * R + r, 64 at a time.
  const uint32_t qr = threadIdx.x / 64;
  for (uint32_t cr = threadIdx.x % 64; cr < R * nsb; cr += 64) {
    const uint32_t r = cr % R, c = cr / R;
    const uint32_t row = min(r0 + r, seg.n_out - 1);  // rows past n_out repeat the last (not stored)
    const uint8_t* col = seg.w + static_cast<size_t>(c) * col_bytes;
    const float4* xc = reinterpret_cast<const float4*>(x + static_cast<size_t>(c) * kQKK);
    float4* dst = reinterpret_cast<float4*>(prods + static_cast<size_t>(c * R + r) * kChainPitch);
    switch (qr) {
      case 0: chain_quarter<0>(col, seg.n_out, row, xc, dst); break;
      case 1: chain_quarter<1>(col, seg.n_out, row, xc, dst); break;
      case 2: chain_quarter<2>(col, seg.n_out, row, xc, dst); break;
      default: chain_quarter<3>(col, seg.n_out, row, xc, dst); break;
    }
  }
  __syncthreads();
  const uint32_t r = threadIdx.x;
  if (r < R && r0 + r < seg.n_out) {
    // A super-block's 256 products in 8 rounds of 32: the next round's 8 reads are issued
    // before this round's 32 adds (a scheduling barrier keeps them there), so the adds wait for
    // LDS only at the first round of each super-block; 16 reads in flight at most, which the LDS
    // wait counter can still tell apart. (Carrying reads over to the next super-block would
    // make the loop copy its registers, and the copy waits for the reads.)
    auto add8 = [](float acc, const float4 (&v)[8]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc += v[i].x;
        acc += v[i].y;
        acc += v[i].z;
        acc += v[i].w;
      }
      return acc;
    };
    float acc = 0.0f;
    for (uint32_t c = 0; c < nsb; ++c) {
      const float4* src = reinterpret_cast<const float4*>(prods + static_cast<size_t>(c * R + r) * kChainPitch);
      float4 v[2][8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[0][i] = src[i];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if (t + 1 < 8) {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[(t + 1) & 1][i] = src[8 * (t + 1) + i];
        }
        __builtin_amdgcn_sched_barrier(0);
        acc = add8(acc, v[t & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    seg.y[r0 + r] = acc;
  }
}

// One activation row against any number of output rows: 64 rows per workgroup, the products
// streamed to the chains through LDS. Wave 0 runs the chains (lane r adds row r's products in
// element order); waves 1-4 each form one quarter of every super-block for all 64 rows and
// hand it over in slot h = quarter / 2 (the super-block's half h: [row][128 + 4 pad] floats).
// A slot holds one half at a time: its producers form the next super-block's products in
// registers while the chain reads the slot, and write them once the chain has released it.
// The counters in LDS only grow: ready[h] counts the quarters written (two per super-block),
// freed[h] the halves the chain has read. Neither side waits on anything the other side
// delivers later, so the waits end; their poll bound only guarantees that every wave exits.
constexpr uint32_t kRingRows = 64;
constexpr uint32_t kRingPitch = kQKK / 2 + 4;  // floats per row of a half-super-block slot
constexpr size_t kRingLds = 2 * kRingRows * kRingPitch * 4;
constexpr uint32_t kRingPoll = 1u << 22;  // s_sleep rounds per wait (~0.1 s), then go on

__device__ __forceinline__ void ring_wait(const uint32_t* counter, uint32_t target) {
  for (uint32_t i = 0; i < kRingPoll; ++i) {
    if (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
}

// Counts one hand-over once this wave's LDS accesses have completed (reads in registers,
// writes in LDS).
__device__ __forceinline__ void ring_signal(uint32_t* counter, uint32_t lane) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int Qr>
__device__ __forceinline__ void ring_producer(const MatvecSeg& seg, cfloat* x, uint32_t nsb, size_t col_bytes,
                                              uint32_t row, uint32_t lane, float* ring, uint32_t* ready,
                                              const uint32_t* freed) {
  constexpr int h = Qr / 2;
  float4* dst = reinterpret_cast<float4*>(ring + static_cast<size_t>(h * kRingRows + lane) * kRingPitch) + 16 * (Qr % 2);
  // Weights three super-blocks ahead: the loads of super-blocks c + 1 .. c + 3 are in flight
  // while c's products are formed and handed over (one super-block ahead leaves every step
  // waiting out a whole HBM latency). Three register sets, the loop unrolled by three so that
  // each keeps its registers. The activations (the same for every lane) come through the
  // scalar cache as operands.
  PlanarBlock b0, b1, b2;
  // Past the last super-block the last is loaded again (unconditional loads keep the
  // compiler's count of loads in flight exact, so each step waits only for its own).
  auto fetch = [&](PlanarBlock& b, uint32_t c) {
    quarter_fetch<Qr>(seg.w + static_cast<size_t>(min(c, nsb - 1)) * col_bytes, seg.n_out, row, b);
  };
  // Super-block c: the first 32 products are formed before the wait for the slot and the
  // other 32 after it (while the chain reads the other half), so 32 registers hold products.
  // Steps past the last super-block (the loop is unrolled by three) form products of the last
  // one again but hand nothing over: only LDS work is conditional, so the compiler's count of
  // loads in flight stays exact across the steps.
  auto step = [&](PlanarBlock& b, uint32_t c) {
    const bool live = c < nsb;
    cfloat* xc = x + static_cast<size_t>(min(c, nsb - 1)) * kQKK + 64 * Qr;
    float4 xs[8], pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[i] = float4{xc[4 * i], xc[4 * i + 1], xc[4 * i + 2], xc[4 * i + 3]};
    quarter_products<Qr, 0, 8>(b, xs, pv);
    // Formed here, before the wait (the compiler would otherwise sink them to their stores).
#pragma unroll
    for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(pv[i].x), "+v"(pv[i].y), "+v"(pv[i].z), "+v"(pv[i].w));
    if (live) {
      if (c > 0) ring_wait(&freed[h], c);  // the chain has read this half of super-block c - 1
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = pv[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[i] = float4{xc[32 + 4 * i], xc[33 + 4 * i], xc[34 + 4 * i], xc[35 + 4 * i]};
    quarter_products<Qr, 8, 8>(b, xs, pv);
    if (live) {
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[8 + i] = pv[i];
      ring_signal(&ready[h], lane);
    }
    fetch(b, c + 3);
  };
  fetch(b0, 0);
  fetch(b1, 1);
  fetch(b2, 2);
  for (uint32_t c = 0; c < nsb; c += 3) {
    step(b0, c);
    step(b1, c + 1);
    step(b2, c + 2);
  }
}

// Three waves per SIMD (two workgroups per CU) leave each lane up to 168 registers, which the
// three prefetched weight sets need.
__global__ __launch_bounds__(320) __attribute__((amdgpu_waves_per_eu(3))) void q6k_planar_ring_kernel(
    MatvecArgs args, uint32_t n_in, size_t col_bytes) {
  extern __shared__ __attribute__((aligned(16))) float ring[];
  __shared__ uint32_t ready[2], freed[2];
  const uint32_t tid = threadIdx.x, lane = tid % 64;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / 64);  // uniform: branches per wave
  if (tid < 2) {
    ready[tid] = 0;
    freed[tid] = 0;
  }
  __syncthreads();
  const uint32_t nsb = args.nb;
  const MatvecSeg seg = args.seg[0];
  const uint32_t r0 = blockIdx.x * kRingRows;
  if (wave == 0) {
    float acc = 0.0f;
    for (uint32_t c = 0; c < nsb; ++c) {
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        ring_wait(&ready[h], 2 * (c + 1));
        const float4* src = reinterpret_cast<const float4*>(ring + static_cast<size_t>(h * kRingRows + lane) * kRingPitch);
        // 128 products in 4 rounds of 32, each round's reads issued a round ahead of its adds
        // (empty asm statements and scheduling barriers pin both for the compiler and for the
        // scheduler); the slot is released once the last round's reads have landed.
        float4 va[8], vb[8];
        auto read8 = [&](float4 (&v)[8], int t) {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = src[8 * t + i];
          asm volatile("" ::: "memory");
          __builtin_amdgcn_sched_barrier(0);
        };
        auto add8 = [&](const float4 (&v)[8]) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            acc += v[i].x;
            acc += v[i].y;
            acc += v[i].z;
            acc += v[i].w;
          }
          asm volatile("" : "+v"(acc)::"memory");  // the adds happen here, before the next reads
          __builtin_amdgcn_sched_barrier(0);
        };
        read8(va, 0);
        read8(vb, 1);
        add8(va);
        read8(va, 2);
        add8(vb);
        read8(vb, 3);
        add8(va);
        ring_signal(&freed[h], lane);
        add8(vb);
      }
    }
    if (r0 + lane < seg.n_out) seg.y[r0 + lane] = acc;
  } else {
    const uint32_t row = min(r0 + lane, seg.n_out - 1);  // rows past n_out repeat the last (not stored)
    cfloat* x = (cfloat*)(reinterpret_cast<const float*>(args.xq));
    switch (wave) {
      case 1: ring_producer<0>(seg, x, nsb, col_bytes, row, lane, ring, ready, freed); break;
      case 2: ring_producer<1>(seg, x, nsb, col_bytes, row, lane, ring, ready, freed); break;
      case 3: ring_producer<2>(seg, x, nsb, col_bytes, row, lane, ring, ready, freed); break;
      default: ring_producer<3>(seg, x, nsb, col_bytes, row, lane, ring, ready, freed); break;
    }
  }
}

// Grants the ring kernel its 66 KB of LDS (above the 64 KB default); false when it cannot.
bool ring_granted() {
  static int granted = -1;
  if (granted < 0) {
    granted = hipFuncSetAttribute(reinterpret_cast<const void*>(q6k_planar_ring_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kRingLds)) == hipSuccess;
    (void)hipGetLastError();
  }
  return granted == 1;
}

template <int R>
size_t chain_lds(uint32_t nsb) { return static_cast<size_t>(R) * nsb * kChainPitch * 4; }

// Grants the chain kernel its LDS (above 64 KB needs the attribute); false when it cannot.
template <int R>
bool chain_granted(size_t lds) {
  static int limit = -1;
  if (limit < 0) {
    int dev = 0, v = 0;
    limit = hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
                    hipFuncSetAttribute(reinterpret_cast<const void*>(q6k_planar_chain_kernel<R>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, v) == hipSuccess
                ? v
                : 65536;
    (void)hipGetLastError();
  }
  return lds <= static_cast<size_t>(limit);
}

}  // namespace

size_t q6k_planar_column_bytes(uint32_t n_out) {
  return static_cast<size_t>(208) * n_out + ((static_cast<size_t>(2) * n_out + 15) & ~static_cast<size_t>(15));
}

int q6k_repack_launch(const uint8_t* src, uint8_t* dst, uint32_t n_out, uint32_t nsb) {
  if (n_out == 0 || nsb == 0) return kOk;
  if ((reinterpret_cast<uintptr_t>(src) & 1u) != 0 || (reinterpret_cast<uintptr_t>(dst) & 15u) != 0)
    return fail(kInvalidArgument, "q6k_repack: native rows must be 2-byte and the planar copy 16-byte aligned");
  const size_t total = static_cast<size_t>(n_out) * nsb;
  hipLaunchKernelGGL(q6k_repack_kernel, dim3(static_cast<uint32_t>(ceil_div(total, 256))), dim3(256), 0, stream(), src,
                     dst, n_out, nsb, q6k_planar_column_bytes(n_out));
  return check_launch("q6k_repack");
}

std::atomic<int> g_q6k_path{0};

uint32_t device_cus() {
  static std::atomic<uint32_t> cus{0};
  uint32_t n = cus.load(std::memory_order_relaxed);
  if (n == 0) {
    int dev = 0, v = 0;
    n = hipGetDevice(&dev) == hipSuccess &&
                hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
            ? static_cast<uint32_t>(v)
            : 256;
    cus.store(n, std::memory_order_relaxed);
  }
  return n;
}

// The one-row kernel for a shape: products then chains for a short matrix whose products fit
// 8-row workgroups (up to 2048 rows and 19 super-blocks); the streamed ring while one round of
// its 64-row workgroups, two per CU, covers the rows; else one lane per row, whose time does
// not grow with the rows until the matrix streams at HBM rate (C2 sweep and the Llama-3 output,
// measured on MI355X).
int one_row_path(uint32_t n_out, uint32_t nsb) {
  if (n_out <= kChainMaxOut && chain_lds<8>(nsb) <= 163840) return 2;
  if (ceil_div(n_out, kRingRows) <= 2 * static_cast<size_t>(device_cus())) return 3;
  return 1;
}

void matvec_q6k_force_path(int path) { g_q6k_path.store(path, std::memory_order_relaxed); }

// The one-lane-per-row kernel's workgroups for one activation row: the launcher's choice of 256
// or 64 rows per workgroup with a single chunk of rows.
uint32_t q6k_planar_argmax_parts(uint32_t n_out) {
  const bool wide = ceil_div(n_out, 256) >= 256;
  return static_cast<uint32_t>(ceil_div(n_out, wide ? 256 : 64));
}

int matvec_q6k_planar_launch(MatvecArgs& a, uint32_t n_in) {
  const uint32_t n_out = a.seg[0].n_out;
  if (a.m == 0 || n_out == 0) return kOk;
  // n_in 0 has no super-block to read (every kernel below reads the first one).
  if (n_in == 0 || n_in % kQKK != 0)
    return fail(kInvalidArgument, "matmul_q6_k_planar: n_in %u is not a positive multiple of 256", n_in);
  if ((reinterpret_cast<uintptr_t>(a.seg[0].w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(a.xq) & 15u) != 0)
    return fail(kInvalidArgument, "matmul_q6_k_planar: the planar weights and the activations must be 16-byte aligned");
  const size_t col_bytes = q6k_planar_column_bytes(n_out);
  int path = g_q6k_path.load(std::memory_order_relaxed);
  if (a.argmax_part != nullptr) {
    // Greedy keys come from the one-lane-per-row kernel alone.
    if (a.m != 1) return fail(kInvalidArgument, "matmul_q6_k_planar: greedy keys for %u rows (one row only)", a.m);
    path = 1;
  }
  if (a.m == 1 && path == 0) path = one_row_path(n_out, a.nb);
  // One activation row: the streamed-ring kernel, 64 output rows per workgroup.
  if (a.m == 1 && path == 3 && ring_granted()) {
    launch(q6k_planar_ring_kernel, dim3(static_cast<uint32_t>(ceil_div(n_out, kRingRows))), dim3(320), kRingLds, a,
           n_in, col_bytes);
    return check_launch("q6k_planar_ring");
  }
  // One activation row: the products-then-chains kernel, R rows per workgroup as the LDS allows
  // (R * n_in / 256 super-blocks of 1040 bytes).
  if (a.m == 1 && path == 2) {
    const uint32_t nsb = a.nb;
    int rows = 8;
    while (rows > 1 && chain_lds<8>(nsb) / 8 * rows > 163840) rows /= 2;
    const uint32_t blocks = static_cast<uint32_t>(ceil_div(n_out, rows));
    bool ok = false;
    switch (rows) {
      case 8: ok = chain_granted<8>(chain_lds<8>(nsb)); if (ok) launch(q6k_planar_chain_kernel<8>, dim3(blocks), dim3(256), chain_lds<8>(nsb), a, n_in, col_bytes); break;
      case 4: ok = chain_granted<4>(chain_lds<4>(nsb)); if (ok) launch(q6k_planar_chain_kernel<4>, dim3(blocks), dim3(256), chain_lds<4>(nsb), a, n_in, col_bytes); break;
      case 2: ok = chain_granted<2>(chain_lds<2>(nsb)); if (ok) launch(q6k_planar_chain_kernel<2>, dim3(blocks), dim3(256), chain_lds<2>(nsb), a, n_in, col_bytes); break;
      default: ok = chain_granted<1>(chain_lds<1>(nsb)); if (ok) launch(q6k_planar_chain_kernel<1>, dim3(blocks), dim3(256), chain_lds<1>(nsb), a, n_in, col_bytes); break;
    }
    if (ok) return check_launch("q6k_planar_chain");
  }
  // Activation rows per workgroup: up to kQ6MaxRows (each lane then runs that many chains, and
  // every weight slice is read once per that many rows), but fewer while that leaves under 1024
  // waves of 64 rows: a lane's chains run one element after another, so a short matrix needs
  // the rows spread over more waves more than it needs fewer weight reads. One launch covers
  // every row, in chunks of equal size (20 rows: 7, 7 and 6 rather than 8, 8 and 4, whose last
  // chunk would run eight chains per lane for four rows).
  uint32_t mm = 1;
  while (mm < kQ6MaxRows && mm < a.m) mm *= 2;
  while (mm > 1 && ceil_div(a.m, mm) * ceil_div(n_out, 64) < 1024) mm /= 2;
  mm = static_cast<uint32_t>(ceil_div(a.m, ceil_div(a.m, mm)));
  const size_t lds = 0;
  const uint32_t chunks = static_cast<uint32_t>(ceil_div(a.m, mm));
  // 256 rows per workgroup when that still gives a workgroup per CU, else 64.
  const bool wide = ceil_div(n_out, 256) * chunks >= 256;
  const uint32_t th = wide ? 256 : 64;
  const uint32_t blocks = static_cast<uint32_t>(ceil_div(n_out, th));
  if (blocks > 65535) return fail(kUnsupported, "matmul_q6_k_planar: %u output rows", n_out);
  const dim3 grid(chunks, blocks);
  const uint32_t m_total = a.m;
#define AXON_Q6P(MM_)                                                                                       \
  case MM_:                                                                                                 \
    if (wide) launch(q6k_planar_kernel<MM_, 256>, grid, dim3(256), lds, a, n_in, col_bytes, m_total);      \
    else launch(q6k_planar_kernel<MM_, 64>, grid, dim3(64), lds, a, n_in, col_bytes, m_total);              \
    break;
  switch (mm) {
    AXON_Q6P(8)
    AXON_Q6P(7)
    AXON_Q6P(6)
    AXON_Q6P(5)
    AXON_Q6P(4)
    AXON_Q6P(3)
    AXON_Q6P(2)
    default:
      if (wide) launch(q6k_planar_kernel<1, 256>, grid, dim3(256), lds, a, n_in, col_bytes, m_total);
      else launch(q6k_planar_kernel<1, 64>, grid, dim3(64), lds, a, n_in, col_bytes, m_total);
      break;
  }
#undef AXON_Q6P
  return check_launch("q6k_planar");
}

int matvec_q6k_launch(MatvecArgs& a, uint32_t n_in) {
  const uint32_t n_out = a.seg[0].n_out;
  if (a.m == 0 || n_out == 0) return kOk;
  if (n_in == 0 || n_in % kQKK != 0)
    return fail(kInvalidArgument, "matmul_q6_k: n_in %u is not a positive multiple of 256", n_in);
  if ((reinterpret_cast<uintptr_t>(a.seg[0].w) & 1u) != 0)
    return fail(kInvalidArgument, "matmul_q6_k: weights must be 2-byte aligned");
  if ((reinterpret_cast<uintptr_t>(a.xq) & 3u) != 0)
    return fail(kInvalidArgument, "matmul_q6_k: activations must be 4-byte aligned");
  const MatvecArgs base = a;
  const float* x = reinterpret_cast<const float*>(a.xq);
  const uint32_t nsb = n_in / kQKK;
  const bool stream_ok = nsb % 2 == 0 && (reinterpret_cast<uintptr_t>(a.seg[0].w) & 3u) == 0 &&
                         (reinterpret_cast<uintptr_t>(a.xq) & 15u) == 0 &&
                         static_cast<size_t>(kStreamRows) * nsb * kBytesQ6_K < (size_t(1) << 31);
  if (stream_ok) {
    const dim3 grid(static_cast<uint32_t>(ceil_div(n_out, kStreamRows)));
    for (uint32_t done = 0; done < base.m;) {
      const uint32_t mm = std::min<uint32_t>(4, base.m - done);
      MatvecArgs g = base;
      g.m = mm;
      g.xq = reinterpret_cast<const uint8_t*>(x + static_cast<size_t>(done) * n_in);
      g.seg[0].y = base.seg[0].y + static_cast<size_t>(done) * base.seg[0].y_stride;
      const size_t lds = static_cast<size_t>(kStreamRows) * kWin * 4 + 2 * static_cast<size_t>(mm) * kQKK * 4;
      switch (mm) {
      case 4: launch(q6k_stream_kernel<4>, grid, dim3(kStreamRows), lds, g, n_in); break;
      case 3: launch(q6k_stream_kernel<3>, grid, dim3(kStreamRows), lds, g, n_in); break;
      case 2: launch(q6k_stream_kernel<2>, grid, dim3(kStreamRows), lds, g, n_in); break;
      default: launch(q6k_stream_kernel<1>, grid, dim3(kStreamRows), lds, g, n_in); break;
      }
      const int rc = check_launch("q6k_stream");
      if (rc != kOk) return rc;
      done += mm;
    }
    return kOk;
  }
  uint32_t done = 0;
  while (done < base.m) {
    uint32_t mm = std::min<uint32_t>(4, base.m - done);
    while (mm > 1 && static_cast<size_t>(mm) * n_in * 4 > 65536) --mm;
    const size_t lds = static_cast<size_t>(mm) * n_in * 4;
    if (lds > 65536) return fail(kUnsupported, "matmul_q6_k: n_in %u too large for LDS", n_in);
    MatvecArgs g = base;
    g.m = mm;
    g.xq = reinterpret_cast<const uint8_t*>(x + static_cast<size_t>(done) * n_in);
    g.seg[0].y = base.seg[0].y + static_cast<size_t>(done) * base.seg[0].y_stride;
    const dim3 grid(static_cast<uint32_t>(ceil_div(n_out, kThreads)));
    switch (mm) {
    case 4: launch(matvec_q6k_kernel<4>, grid, dim3(kThreads), lds, g, n_in); break;
    case 3: launch(matvec_q6k_kernel<3>, grid, dim3(kThreads), lds, g, n_in); break;
    case 2: launch(matvec_q6k_kernel<2>, grid, dim3(kThreads), lds, g, n_in); break;
    default: launch(matvec_q6k_kernel<1>, grid, dim3(kThreads), lds, g, n_in); break;
    }
    const int rc = check_launch("matvec_q6k");
    if (rc != kOk) return rc;
    done += mm;
  }
  return kOk;
}

}  // namespace axon_hip
