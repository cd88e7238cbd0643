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
// One lane owns one output row (a wave owns 64 rows) and walks it in element order. The rows'
// bytes come through LDS one 210-byte super-block at a time: the wave copies 64 rows x 212
// bytes with coalesced dword loads into one buffer while it computes from the other, so the
// HBM stream of the next super-block overlaps the arithmetic on the current one.
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr int kRows = 64;       // one wave, one row per lane
constexpr int kChunkDw = 53;    // dwords staged per row and super-block (210 bytes + alignment)

// Loads this lane's share of super-block c of rows [r0, r0 + nr): dword k of the flattened
// (row, dword) pairs lane + 64 i. Dwords outside the super-block's bytes are read as halves so no
// access leaves the row.
__device__ __forceinline__ void q6k_fetch(const uint8_t* __restrict__ w, size_t row_bytes, uint32_t r0,
                                          uint32_t nr, uint32_t c, uint32_t lane, uint32_t (&reg)[kChunkDw]) {
#pragma unroll
  for (int i = 0; i < kChunkDw; ++i) {
    const uint32_t p = lane + 64 * i;
    const uint32_t rr = p / kChunkDw;
    const uint32_t k = p - rr * kChunkDw;
    uint32_t v = 0;
    if (rr < nr) {
      const uint8_t* sb = w + (r0 + rr) * row_bytes + static_cast<size_t>(c) * kBytesQ6_K;
      const uintptr_t shift = reinterpret_cast<uintptr_t>(sb) & 3u;  // 0 or 2
      const uint8_t* a = sb - shift + 4 * k;
      if (shift == 2 && k == 0) {
        v = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(sb)) << 16;
      } else if (shift == 0 && k == kChunkDw - 1) {
        v = *reinterpret_cast<const uint16_t*>(a);
      } else {
        v = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(a));
      }
    }
    reg[i] = v;
  }
}

// 32 consecutive elements: quants from the nibble at `nsh` of ql and the two bits at `hsh` of
// qh, the first 16 with int8 scale byte 0 of sc2 and the next 16 with byte 1.
template <int MM>
__device__ __forceinline__ void q6k_quarter(float (&acc)[MM], const uint32_t (&ql)[8], const uint32_t (&qh)[8],
                                            uint32_t nsh, uint32_t hsh, float d, uint32_t sc2, const float* xs,
                                            uint32_t n_in, uint32_t e0) {
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const float scale = static_cast<float>(static_cast<int8_t>((sc2 >> (8 * half)) & 0xffu));
    const float ds = d * scale;       // exact
    const float neg32 = -32.0f * ds;  // exact
#pragma unroll
    for (int l4 = 4 * half; l4 < 4 * half + 4; ++l4) {
      const uint32_t q = ((ql[l4] >> nsh) & 0x0f0f0f0fu) | (((qh[l4] >> hsh) & 0x03030303u) << 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = fmaf(ds, static_cast<float>((q >> (8 * e)) & 0xffu), neg32);  // (d*scale)*(q-32), exactly
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[m] += v * xs[m * n_in + e0 + 4 * l4 + e];
      }
    }
  }
}

template <int MM>
__global__ __launch_bounds__(64) void matvec_q6k_kernel(MatvecArgs args, uint32_t n_in) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t lane = threadIdx.x;
  const uint32_t nsb = args.nb;
  const MatvecSeg seg = args.seg[0];
  const uint32_t r0 = blockIdx.x * kRows;
  const uint32_t nr = min(static_cast<uint32_t>(kRows), seg.n_out - r0);
  const size_t row_bytes = static_cast<size_t>(nsb) * kBytesQ6_K;
  const float* x = reinterpret_cast<const float*>(args.xq);

  float* xs = reinterpret_cast<float*>(smem);                             // [MM][n_in]
  uint32_t* buf0 = reinterpret_cast<uint32_t*>(smem + args.lds_tile);     // [64][53] dwords, x2
  uint32_t* buf1 = buf0 + kRows * kChunkDw;
  for (uint32_t m = 0; m < MM; ++m) {
    for (uint32_t i = lane; i < n_in; i += 64) xs[m * n_in + i] = x[static_cast<size_t>(m) * n_in + i];
  }
  uint32_t reg[kChunkDw];
  q6k_fetch(seg.w, row_bytes, r0, nr, 0, lane, reg);
#pragma unroll
  for (int i = 0; i < kChunkDw; ++i) buf0[lane + 64 * i] = reg[i];
  __syncthreads();

  // Where this lane's super-block bytes start inside its 212-byte LDS row.
  const uint32_t shift = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(seg.w + (r0 + lane) * row_bytes) & 3u);
  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.0f;

  for (uint32_t c = 0; c < nsb; ++c) {
    uint32_t* cur = (c & 1) ? buf1 : buf0;
    uint32_t* nxt = (c & 1) ? buf0 : buf1;
    if (c + 1 < nsb) q6k_fetch(seg.w, row_bytes, r0, nr, c + 1, lane, reg);
    // Super-block shift alternates with c's parity when the row start is 4-byte aligned.
    const uint32_t sh = (shift + 2 * (c & 1)) & 3u;
    const uint8_t* rbase = reinterpret_cast<const uint8_t*>(cur);
    const uint32_t off = lane * kChunkDw * 4 + sh;
    uint32_t dsc[1];
    lds_read_unaligned<1>(rbase, off + 208, dsc);
    const float d = half_bits_to_float(dsc[0] & 0xffffu);
    uint32_t scw[4];
    lds_read_unaligned<4>(rbase, off + 192, scw);
#pragma unroll 1
    for (int n = 0; n < 2; ++n) {
      uint32_t qa[8], qb[8], qh[8];
      lds_read_unaligned<8>(rbase, off + 64 * n, qa);        // ql[0..31] of this half
      lds_read_unaligned<8>(rbase, off + 64 * n + 32, qb);   // ql[32..63]
      lds_read_unaligned<8>(rbase, off + 128 + 32 * n, qh);
      const uint32_t e0 = c * kQKK + 128 * n;
      const uint32_t sw = scw[2 * n] ;
      const uint32_t sw2 = scw[2 * n + 1];
      // Quarters in element order: q1 (ql low, qh bits 0-1), q2 (ql+32 low, bits 2-3),
      // q3 (ql high, bits 4-5), q4 (ql+32 high, bits 6-7); scales is, is+2, is+4, is+6.
      q6k_quarter<MM>(acc, qa, qh, 0, 0, d, sw & 0xffffu, xs, n_in, e0);
      q6k_quarter<MM>(acc, qb, qh, 0, 2, d, sw >> 16, xs, n_in, e0 + 32);
      q6k_quarter<MM>(acc, qa, qh, 4, 4, d, sw2 & 0xffffu, xs, n_in, e0 + 64);
      q6k_quarter<MM>(acc, qb, qh, 4, 6, d, sw2 >> 16, xs, n_in, e0 + 96);
    }
    if (c + 1 < nsb) {
#pragma unroll
      for (int i = 0; i < kChunkDw; ++i) nxt[lane + 64 * i] = reg[i];
    }
    __syncthreads();
  }
  if (lane < nr) {
#pragma unroll
    for (int m = 0; m < MM; ++m) seg.y[static_cast<size_t>(m) * seg.y_stride + r0 + lane] = acc[m];
  }
}

}  // namespace

int matvec_q6k_launch(MatvecArgs& a, uint32_t n_in) {
  const uint32_t n_out = a.seg[0].n_out;
  if (a.m == 0 || n_out == 0) return kOk;
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k: n_in %u is not a multiple of 256", n_in);
  if ((reinterpret_cast<uintptr_t>(a.seg[0].w) & 1u) != 0)
    return fail(kInvalidArgument, "matmul_q6_k: weights must be 2-byte aligned");
  const MatvecArgs base = a;
  const float* x = reinterpret_cast<const float*>(a.xq);
  const size_t tile = 2ull * kRows * kChunkDw * 4 + 16;
  uint32_t done = 0;
  while (done < base.m) {
    uint32_t mm = std::min<uint32_t>(4, base.m - done);
    while (mm > 1 && static_cast<size_t>(mm) * n_in * 4 + tile > 65536) --mm;
    const size_t xbytes = (static_cast<size_t>(mm) * n_in * 4 + 15) & ~size_t(15);
    const size_t lds = xbytes + tile;
    if (lds > 65536) return fail(kUnsupported, "matmul_q6_k: n_in %u too large for one LDS tile", n_in);
    MatvecArgs g = base;
    g.m = mm;
    g.lds_tile = static_cast<uint32_t>(xbytes);
    g.xq = reinterpret_cast<const uint8_t*>(x + static_cast<size_t>(done) * n_in);
    g.seg[0].y = base.seg[0].y + static_cast<size_t>(done) * base.seg[0].y_stride;
    const dim3 grid(static_cast<uint32_t>(ceil_div(n_out, kRows)));
    switch (mm) {
    case 4: hipLaunchKernelGGL(matvec_q6k_kernel<4>, grid, dim3(kRows), lds, stream(), g, n_in); break;
    case 3: hipLaunchKernelGGL(matvec_q6k_kernel<3>, grid, dim3(kRows), lds, stream(), g, n_in); break;
    case 2: hipLaunchKernelGGL(matvec_q6k_kernel<2>, grid, dim3(kRows), lds, stream(), g, n_in); break;
    default: hipLaunchKernelGGL(matvec_q6k_kernel<1>, grid, dim3(kRows), lds, stream(), g, n_in); break;
    }
    const int rc = check_launch("matvec_q6k");
    if (rc != kOk) return rc;
    done += mm;
  }
  return kOk;
}

}  // namespace axon_hip
