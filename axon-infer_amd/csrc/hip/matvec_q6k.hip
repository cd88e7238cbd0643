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
// registers: the lane loads the next 210-byte super-block (53 dwords) while it works on the
// current one, so the row streams from HBM under the arithmetic. Activation rows sit in LDS
// and are read as broadcasts.
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

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

}  // namespace

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
