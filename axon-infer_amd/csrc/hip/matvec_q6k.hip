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
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr uint32_t kQ6MaxRows = 8;  // activation rows per workgroup of the planar kernel

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
  const uint32_t row = blockIdx.y * TH + tid;
  if (row >= seg.n_out) return;
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
    if (m < static_cast<int>(mm)) seg.y[static_cast<size_t>(m0 + m) * seg.y_stride + row] = acc[m];
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

int matvec_q6k_planar_launch(MatvecArgs& a, uint32_t n_in) {
  const uint32_t n_out = a.seg[0].n_out;
  if (a.m == 0 || n_out == 0) return kOk;
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k_planar: n_in %u is not a multiple of 256", n_in);
  if ((reinterpret_cast<uintptr_t>(a.seg[0].w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(a.xq) & 15u) != 0)
    return fail(kInvalidArgument, "matmul_q6_k_planar: the planar weights and the activations must be 16-byte aligned");
  const size_t col_bytes = q6k_planar_column_bytes(n_out);
  // Activation rows per workgroup: up to kQ6MaxRows (each lane then runs that many chains, and
  // every weight slice is read once per that many rows), but fewer while that leaves under 1024
  // waves of 64 rows: a lane's chains run one element after another, so a short matrix needs
  // the rows spread over more waves more than it needs fewer weight reads. One launch covers
  // every row.
  uint32_t mm = 1;
  while (mm < kQ6MaxRows && mm < a.m) mm *= 2;
  while (mm > 1 && ceil_div(a.m, mm) * ceil_div(n_out, 64) < 1024) mm /= 2;
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
    AXON_Q6P(4)
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
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k: n_in %u is not a multiple of 256", n_in);
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
