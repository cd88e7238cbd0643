// The decode matvec with its neighbours folded in: one launch per weight group of a layer for
// one to four activation rows (batch-1 and small-batch decode).
//
// Input:
//   kInQ8    the activation rows arrive as Q8_0 blocks;
//   kInF32   float rows, quantized in every workgroup exactly as quantize_row_q8_0
//            (trickymind1324/axon-infer src/core/dtype.cpp:338-354);
//   kInNorm  float rows, RMSNorm'd (src/kernels/ref/rmsnorm.cpp:10-21) then quantized, as
//            src/model/llama.cpp:500 and 598 do before the q|k|v and gate|up matmuls.
// matvec_dma_kernel copies the weight rows (and Q8_0 blocks) straight into LDS with LDS-DMA
// buffer loads: no staging registers, so many workgroups stay resident, every copy of the
// launch is in flight at once, and the float prologue runs while the weights arrive.
// matvec_fused_kernel stages through registers for rows that are not 4-byte multiples.
// Body: the integer-exact block dots and the left-to-right float accumulation of
// matvec_q8.hip (src/kernels/ref/quant.cpp:44-69, 161-181).
// Epilogue (output):
//   kOutStore / kOutAdd   y = acc / y += acc (the residual add, llama.cpp:594-595, 621-623);
//   kOutSilu              segment 0 is gate and segment 1 up, the same rows in one workgroup:
//                         h = gate / (1 + exp(-gate)) * up (src/kernels/ref/silu.cpp:8-13);
//   kOutRope              segments q, k, v: bias (llama.cpp:507-511), then the Normal-style
//                         rotation of pairs (2i, 2i+1) with host-built cos/sin
//                         (src/kernels/ref/rope.cpp:13-37), q to its buffer, k and v into the
//                         row's KV cache at its position (llama.cpp:493-497, 520-537).
// The float prologues recompute the row norm and the Q8_0 blocks in every workgroup with the
// same reduction tree as rmsnorm_regs_kernel, so all paths agree bit for bit.
#include "blockdot.h"
#include "common.h"
#include "matvec.h"

namespace axon_hip {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 4;  // float activation chunks of 8 held per thread

// Where a workgroup's weight rows are. The SiLU pairing runs gate and up rows together: up
// row r sits at tile row pitch_rows + r.
struct WgRows {
  int s;
  uint32_t r0, nr, n_wrows, pitch_rows;
  bool silu;
};

__device__ __forceinline__ WgRows wg_rows(const FusedArgs& args) {
  WgRows g;
  g.silu = args.out_mode == kOutSilu;
  const uint32_t wg = blockIdx.x;
  g.s = 0;
  if (!g.silu && args.n_seg > 1 && wg >= args.wg_begin[1]) g.s = 1;
  if (!g.silu && args.n_seg > 2 && wg >= args.wg_begin[2]) g.s = 2;
  g.r0 = (wg - args.wg_begin[g.s]) * args.rows;
  g.nr = min(args.rows, args.n_out[g.s] - g.r0);
  g.n_wrows = g.silu ? 2 * g.nr : g.nr;
  g.pitch_rows = g.silu ? args.rows : 0;
  return g;
}

// Block terms, ordered chains and the epilogue, once the weight tile and the activation blocks
// are in LDS. Reuses the tile for the chain results.
template <int T>
__device__ __forceinline__ void fused_body(const FusedArgs& args, const WgRows& g, uint8_t* tile, const ActBlock* act,
                                           float* terms) {
  constexpr int bs = wbytes<T>();
  const uint32_t tid = threadIdx.x;
  const uint32_t nb = args.nb;
  const uint32_t M = args.m;
  const uint32_t R = args.rows;
  const uint32_t row_bytes = nb * bs;
  const uint32_t tpitch = term_pitch(nb);
  const uint32_t nr = g.nr;
  const int s = g.s;
  const uint32_t r0 = g.r0;
  // Each thread keeps one block column b (its activation block read once per row of x) and
  // walks the weight rows of that column: with nb <= 256 the threads form floor(256 / nb) row
  // groups, otherwise columns b, b + 256, ... each take every row.
  const uint32_t groups = nb <= kThreads ? kThreads / nb : 1;
  const uint32_t col0 = nb <= kThreads ? tid % nb : tid;
  const uint32_t rg = nb <= kThreads ? tid / nb : 0;
  if (rg < groups) {
    for (uint32_t b = col0; b < nb; b += kThreads) {
      for (uint32_t m = 0; m < M; ++m) {
        const ActBlock a = act[m * nb + b];
        for (uint32_t r = rg; r < g.n_wrows; r += groups) {
          const uint32_t trow = (g.silu && r >= nr) ? g.pitch_rows + (r - nr) : r;
          terms[(m * 2 * R + trow) * tpitch + b] = fused_term<T>(tile, trow * row_bytes + b * bs, a);
        }
      }
    }
  }
  __syncthreads();
  float* outv = reinterpret_cast<float*>(tile);  // [M][2R], the tile is no longer needed
  if (tid < M * g.n_wrows) {
    const uint32_t m = tid / g.n_wrows;
    const uint32_t r = tid - m * g.n_wrows;
    const uint32_t trow = (g.silu && r >= nr) ? g.pitch_rows + (r - nr) : r;
    outv[m * 2 * R + trow] = ordered_sum(terms + (m * 2 * R + trow) * tpitch, nb);
  }
  __syncthreads();

  if (args.out_mode == kOutStore || args.out_mode == kOutAdd) {
    if (tid < M * nr) {
      const uint32_t m = tid / nr;
      const uint32_t r = tid - m * nr;
      const float acc = outv[m * 2 * R + r];
      float* y = args.y[s] + static_cast<size_t>(m) * args.y_stride[s] + r0 + r;
      *y = args.out_mode == kOutAdd ? *y + acc : acc;
    }
  } else if (g.silu) {
    if (tid < M * nr) {
      const uint32_t m = tid / nr;
      const uint32_t r = tid - m * nr;
      const float gt = outv[m * 2 * R + r];
      const float u = outv[m * 2 * R + g.pitch_rows + r];
      const float h = gt / (1.0f + exp_libm(-gt)) * u;
      args.y[0][static_cast<size_t>(m) * args.y_stride[0] + r0 + r] = h;
      // Q8_0 blocks of h (the launcher gives each workgroup whole blocks: 32 rows, so the 32
      // outputs of one block sit in 32 aligned lanes, r = lane % 32).
      if (args.outq != nullptr) {
        const size_t nbq = args.n_out[0] / kQK;
        quantize_block_lanes(h, r & 31u, args.outq + (static_cast<size_t>(m) * nbq + (r0 + r) / kQK) * kBytesQ8_0);
      }
    }
  } else {
    // kOutRope: one thread per (row, pair of outputs).
    const uint32_t np = nr / 2;
    if (tid < M * np) {
      const uint32_t m = tid / np;
      const uint32_t pr = tid - m * np;
      const uint32_t o = r0 + 2 * pr;  // even: the pair (o, o + 1) lies in one head
      float x0 = outv[m * 2 * R + 2 * pr];
      float x1 = outv[m * 2 * R + 2 * pr + 1];
      if (args.bias[s] != nullptr) {
        x0 = x0 + args.bias[s][o];
        x1 = x1 + args.bias[s][o + 1];
      }
      const int32_t pos = args.pos[m];
      if (s < 2) {
        const uint32_t i = (o % args.head_dim) / 2;
        if (i < args.rot_half) {
          const float2 cs = reinterpret_cast<const float2*>(args.rope_table)[static_cast<size_t>(pos) * args.rot_half + i];
          const float a0 = x0, a1 = x1;
          x0 = a0 * cs.x - a1 * cs.y;
          x1 = a0 * cs.y + a1 * cs.x;
        }
      }
      if (s == 0) {
        float* q = args.y[0] + static_cast<size_t>(m) * args.y_stride[0] + o;
        q[0] = x0;
        q[1] = x1;
      } else {
        const size_t kv_row = args.n_out[1];
        const size_t at = args.cache_off[m] + (s == 1 ? args.k_layer_off : args.v_layer_off) +
                          static_cast<size_t>(pos) * kv_row + o;
        if (args.cache_f16) {  // rounded in once (llama.cpp:525-532)
          uint16_t* c = static_cast<uint16_t*>(args.cache) + at;
          c[0] = static_cast<uint16_t>(float_to_half_bits(x0));
          c[1] = static_cast<uint16_t>(float_to_half_bits(x1));
        } else {
          float* c = static_cast<float*>(args.cache) + at;
          c[0] = x0;
          c[1] = x1;
        }
      }
    }
  }
}

// The float prologue, row by row: thread t loads chunks c = t + 256 k (elements 8c .. 8c + 7)
// of the row (at most kMaxChunks per thread, checked by the launcher), RMSNorm's them
// (kInNorm, one chunk per thread) with rmsnorm_row_256's reduction tree and quantizes them
// into act.
__device__ __forceinline__ void float_prologue(const FusedArgs& args, ActBlock* act, double* red) {
  const uint32_t tid = threadIdx.x;
  const uint32_t nb = args.nb;
  const uint32_t n_in = nb * kQK;
  const uint32_t n_chunks = n_in / 8;
  const uint32_t part = tid & 3;
  const bool norm = args.in_mode == kInNorm;
  for (uint32_t m = 0; m < args.m; ++m) {
    float xv[kMaxChunks][8];
    float wv[8];
    const float* xr = args.x + static_cast<size_t>(m) * args.x_stride;
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i) {
      const uint32_t c = tid + i * kThreads;
      if (c < n_chunks) {
        const float4 a = reinterpret_cast<const float4*>(xr + c * 8)[0];
        const float4 b = reinterpret_cast<const float4*>(xr + c * 8)[1];
        xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
        xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
      }
    }
    float inv = 1.0f;
    if (norm) {
      // One chunk per thread: the sum of squares in double with rmsnorm_row_256's tree (8
      // elements per thread in order, the wave butterfly, the waves in order).
      const bool has = tid < n_chunks;
      double ss = 0.0;
      if (has) {
        const float4 e = reinterpret_cast<const float4*>(args.norm_w + tid * 8)[0];
        const float4 f = reinterpret_cast<const float4*>(args.norm_w + tid * 8)[1];
        wv[0] = e.x; wv[1] = e.y; wv[2] = e.z; wv[3] = e.w; wv[4] = f.x; wv[5] = f.y; wv[6] = f.z; wv[7] = f.w;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const double v = static_cast<double>(xv[0][k]);
          ss += v * v;
        }
      }
      ss = block_sum_double_256(ss, red);
      inv = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(n_in) + static_cast<double>(args.eps)));
    }
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i) {
      const uint32_t c = tid + i * kThreads;
      if (c < n_chunks) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = norm ? xv[0][k] * inv * wv[k] : xv[i][k];
        quantize8_to_act(v, part, act[m * nb + c / 4]);
      }
    }
  }
}

// Rows of a multiple of 4 bytes: the weight rows and Q8_0 blocks go straight into LDS by DMA;
// a float prologue runs while they arrive.
template <int T>
__global__ __launch_bounds__(kThreads) void matvec_dma_kernel(FusedArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ double red[kThreads / 64];
  constexpr int bs = wbytes<T>();
  const uint32_t tid = threadIdx.x;
  const WgRows g = wg_rows(args);
  const uint32_t row_bytes = args.nb * bs;
  ActBlock* act = reinterpret_cast<ActBlock*>(smem);
  uint8_t* tile = smem + args.lds_tile;
  uint8_t* raw = smem + args.lds_scratch;
  dma_to_lds(args.w[g.s] + static_cast<size_t>(g.r0) * row_bytes, tile, g.nr * row_bytes, tid, kThreads);
  if (g.silu) {
    dma_to_lds(args.w[1] + static_cast<size_t>(g.r0) * row_bytes, tile + static_cast<size_t>(g.pitch_rows) * row_bytes,
               g.nr * row_bytes, tid, kThreads);
  }
  if (args.in_mode == kInQ8) {
    dma_to_lds(args.xq, raw, args.m * args.nb * kBytesQ8_0, tid, kThreads);
  } else {
    float_prologue(args, act, red);
  }
  wait_memory();
  __syncthreads();
  if (args.in_mode == kInQ8) {
    for (uint32_t i = tid; i < args.m * args.nb; i += kThreads) act[i] = unpack_q8_0_lds(raw, i * kBytesQ8_0);
    __syncthreads();
  }
  fused_body<T>(args, g, tile, act, reinterpret_cast<float*>(raw));
}

// One activation row RMSNorm'd in the prologue (q|k|v and gate|up at batch 1), rows of a
// multiple of 4 bytes: matvec_dma_kernel with its copies ordered for latency. Every copy is
// LDS-DMA issued from inline assembly, this wave's chunks of the activation row and of the norm
// gains first, then the weights; vmcnt drains in issue order, so each wave waits for its own
// two staging copies alone while its weight copies stay in flight, and the norm/quantize
// prologue runs while the weights arrive. The prologue's operations are float_prologue's for one
// row with one chunk per thread, in the same order. The staging area (norm1_stage_bytes) lies
// past the shared layout: the row [256][8] and the gains [256][8].

// dma_to_lds from inline assembly; returns this wave's number of copies (uniform in the wave).
__device__ __forceinline__ uint32_t dma_to_lds_asm(const uint8_t* src, uint8_t* dst, uint32_t bytes, uint32_t tid,
                                                   uint32_t nthreads) {
  const RsrcWords rsrc = raw_buffer_words(src, bytes);
  const uint32_t lane = tid & 63u;
  const uint32_t wave0 = tid & ~63u;
  const uint32_t dst_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(dst)));
  const bool wide = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | bytes) & 15u) == 0;
  const uint32_t units = bytes / (wide ? 16u : 4u);
  uint32_t n = 0;
  for (uint32_t base = wave0; base < units; base += nthreads) {
    if (base + lane < units) {
      if (wide) lds_dma16(rsrc, (base + lane) * 16u, dst_lds + base * 16u);
      else lds_dma4(rsrc, (base + lane) * 4u, dst_lds + base * 4u);
    }
    ++n;
  }
  return n;
}

constexpr uint32_t kNorm1Stage = 2 * kThreads * 32;  // row and gains, one 8-float chunk per thread
constexpr size_t kNorm1MinWeights = 32 * 1024;        // weight bytes per workgroup that pay for staging

template <int T>
__global__ __launch_bounds__(kThreads) void matvec_norm1_kernel(FusedArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ double red[kThreads / 64];
  constexpr int bs = wbytes<T>();
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave0 = tid & ~63u;
  const WgRows g = wg_rows(args);
  const uint32_t row_bytes = args.nb * bs;
  ActBlock* act = reinterpret_cast<ActBlock*>(smem);
  uint8_t* tile = smem + args.lds_tile;
  uint8_t* raw = smem + args.lds_scratch;
  const uint32_t n_in = args.nb * kQK;
  const uint32_t n_chunks = n_in / 8;  // at most kThreads (the launcher checks)
  float* xs = reinterpret_cast<float*>(smem + args.lds_stage);  // [256][8]
  float* ws = xs + kThreads * 8;                                // [256][8]
  // 1. Staging: wave w copies chunks wave0 .. wave0 + 63 (2 KB, two copies) of the row and of
  // the gains. Reads past the row return zeros (raw buffer bounds) into the staging area.
  if (wave0 < n_chunks) {
    const RsrcWords xsrc = raw_buffer_words(args.x, n_in * 4);
    const RsrcWords wsrc = raw_buffer_words(args.norm_w, n_in * 4);
    const uint32_t xs_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(xs)));
    const uint32_t ws_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(ws)));
    lds_dma16(xsrc, wave0 * 32 + lane * 16, xs_lds + wave0 * 32);
    lds_dma16(xsrc, wave0 * 32 + 1024 + lane * 16, xs_lds + wave0 * 32 + 1024);
    lds_dma16(wsrc, wave0 * 32 + lane * 16, ws_lds + wave0 * 32);
    lds_dma16(wsrc, wave0 * 32 + 1024 + lane * 16, ws_lds + wave0 * 32 + 1024);
  }
  // 2. The weight copies.
  uint32_t copies = dma_to_lds_asm(args.w[g.s] + static_cast<size_t>(g.r0) * row_bytes, tile, g.nr * row_bytes, tid, kThreads);
  if (g.silu) {
    copies += dma_to_lds_asm(args.w[1] + static_cast<size_t>(g.r0) * row_bytes,
                             tile + static_cast<size_t>(g.pitch_rows) * row_bytes, g.nr * row_bytes, tid, kThreads);
  }
  // 3. The prologue once this wave's staging copies (older than its weight copies) landed.
  wait_vm_upto(copies);
  const bool has = tid < n_chunks;
  float xv[8], wv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    xv[k] = xs[tid * 8 + k];
    wv[k] = ws[tid * 8 + k];
  }
  double ss = 0.0;
  if (has) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const double v = static_cast<double>(xv[k]);
      ss += v * v;
    }
  }
  ss = block_sum_double_256(ss, red);
  const float inv = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(n_in) + static_cast<double>(args.eps)));
  if (has) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = xv[k] * inv * wv[k];
    quantize8_to_act(v, tid & 3, act[tid / 4]);
  }
  // 4. Every copy, then the body.
  wait_vm<0>();
  __syncthreads();
  fused_body<T>(args, g, tile, act, reinterpret_cast<float*>(raw));
}

// Rows of any even byte count: the same with the weights staged through registers.
template <int T>
__global__ __launch_bounds__(kThreads) void matvec_fused_kernel(FusedArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ double red[kThreads / 64];
  constexpr int bs = wbytes<T>();
  const uint32_t tid = threadIdx.x;
  const uint32_t nb = args.nb;
  const uint32_t M = args.m;
  const uint32_t row_bytes = nb * bs;
  const WgRows g = wg_rows(args);
  ActBlock* act = reinterpret_cast<ActBlock*>(smem);
  uint8_t* tile = smem + args.lds_tile;
  uint8_t* raw = smem + args.lds_scratch;
  const uint32_t xthreads = args.in_mode == kInQ8 ? 64u : 0u;
  if (tid >= xthreads) {
    stage_bytes(args.w[g.s] + static_cast<size_t>(g.r0) * row_bytes, tile, g.nr * row_bytes, tid - xthreads,
                kThreads - xthreads);
    if (g.silu) {
      stage_bytes(args.w[1] + static_cast<size_t>(g.r0) * row_bytes,
                  tile + static_cast<size_t>(g.pitch_rows) * row_bytes, g.nr * row_bytes, tid - xthreads,
                  kThreads - xthreads);
    }
  } else {
    stage_bytes(args.xq, raw, M * nb * kBytesQ8_0, tid, xthreads);
  }
  if (args.in_mode == kInQ8) {
    __syncthreads();
    for (uint32_t i = tid; i < M * nb; i += kThreads) act[i] = unpack_q8_0_lds(raw, i * kBytesQ8_0);
  } else {
    float_prologue(args, act, red);
  }
  __syncthreads();
  fused_body<T>(args, g, tile, act, reinterpret_cast<float*>(raw));
}

size_t fused_lds(int bs, uint32_t m, uint32_t nb, uint32_t rows, bool silu, size_t* act_out, size_t* tile_out) {
  const size_t row_bytes = static_cast<size_t>(nb) * bs;
  const uint32_t wrows = silu ? 2 * rows : rows;
  const size_t act = (static_cast<size_t>(m) * nb * sizeof(ActBlock) + 15) & ~size_t(15);
  const size_t tile = std::max<size_t>((wrows * row_bytes + 16 + 15) & ~size_t(15), static_cast<size_t>(m) * 2 * rows * 4);
  const size_t raw = static_cast<size_t>(m) * nb * kBytesQ8_0 + 16;
  const size_t terms = static_cast<size_t>(m) * 2 * rows * term_pitch(nb) * 4 + 64;
  *act_out = act;
  *tile_out = tile;
  return act + tile + std::max(raw, terms);
}

// Dynamic LDS the decode matvec kernels may use once granted above the default 64 KB (asked
// for once per instantiation), or 64 KB when the device does not grant more.
template <typename K>
size_t grant_lds(K kernel) {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      v <= 65536 || hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, v - 256) != hipSuccess)
    return 65536;
  return static_cast<size_t>(v);
}

size_t norm1_lds_limit(int type) {
  static size_t limits[3] = {0, 0, 0};
  const int t = type == Q8_0 ? 0 : type == Q4_0 ? 1 : 2;
  if (limits[t] == 0) {
    limits[t] = t == 0 ? grant_lds(matvec_norm1_kernel<Q8_0>)
                       : t == 1 ? grant_lds(matvec_norm1_kernel<Q4_0>) : grant_lds(matvec_norm1_kernel<Q4_1>);
  }
  return limits[t] - 256;
}

size_t wide_lds_limit(int type, bool dma) {
  static size_t limits[2][3] = {{0, 0, 0}, {0, 0, 0}};
  const int t = type == Q8_0 ? 0 : type == Q4_0 ? 1 : 2;
  size_t& l = limits[dma ? 1 : 0][t];
  if (l == 0) {
    if (dma) l = t == 0 ? grant_lds(matvec_dma_kernel<Q8_0>) : t == 1 ? grant_lds(matvec_dma_kernel<Q4_0>) : grant_lds(matvec_dma_kernel<Q4_1>);
    else l = t == 0 ? grant_lds(matvec_fused_kernel<Q8_0>) : t == 1 ? grant_lds(matvec_fused_kernel<Q4_0>) : grant_lds(matvec_fused_kernel<Q4_1>);
  }
  return l;
}

}  // namespace

bool matvec_fused_fits(int type, int in_mode, uint32_t m, uint32_t nb, bool silu) {
  const int bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  size_t act, tile;
  if (m < 1 || m > 4 || fused_lds(bs, m, nb, silu ? 1 : 2, silu, &act, &tile) > 65536 - 256) return false;
  if (in_mode == kInQ8) return true;
  const uint32_t cpt = ceil_div(nb * kQK / 8, kThreads);
  // The norm prologue reproduces rmsnorm_row_256's reduction only with one chunk per thread.
  return cpt <= kMaxChunks && (in_mode != kInNorm || cpt == 1);
}

int matvec_fused_launch(int type, FusedArgs& a) {
  if (a.m == 0) return kOk;
  if (a.m > 4) return fail(kInvalidArgument, "matvec_fused: %u rows (at most 4)", a.m);
  if (!matvec_fused_fits(type, a.in_mode, a.m, a.nb, a.out_mode == kOutSilu))
    return fail(kUnsupported, "matvec_fused: %u rows of %u blocks do not fit one launch", a.m, a.nb);
  if (a.in_mode != kInQ8 && ((reinterpret_cast<uintptr_t>(a.x) | (a.x_stride * 4u) |
                              (a.in_mode == kInNorm ? reinterpret_cast<uintptr_t>(a.norm_w) : 0u)) & 15u))
    return fail(kInvalidArgument, "matvec_fused: float activations must be 16-byte aligned");
  const bool silu = a.out_mode == kOutSilu;
  const bool rope = a.out_mode == kOutRope;
  if (silu && (a.n_seg != 2 || a.n_out[0] != a.n_out[1])) return fail(kInvalidArgument, "matvec_fused: SiLU pairs need gate and up of one size");
  if (rope && (a.n_seg != 3 || a.n_out[1] != a.n_out[2] || (a.n_out[0] | a.n_out[1] | a.head_dim) & 1))
    return fail(kInvalidArgument, "matvec_fused: q|k|v rope epilogue shapes");
  const int bs = type == Q8_0 ? kBytesQ8_0 : type == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
  const size_t row_bytes = static_cast<size_t>(a.nb) * bs;
  // LDS-DMA needs 4-byte multiples for every copy: the rows, the weight bases and the blocks.
  uintptr_t bases = a.in_mode == kInQ8 ? reinterpret_cast<uintptr_t>(a.xq) : 0u;
  for (int s = 0; s < a.n_seg; ++s) bases |= reinterpret_cast<uintptr_t>(a.w[s]);
  const bool dma = row_bytes % 4 == 0 && (bases & 3u) == 0 &&
                   (a.in_mode != kInQ8 || (static_cast<size_t>(a.m) * a.nb * kBytesQ8_0) % 4 == 0);
  uint32_t total_out = 0;
  for (int s = 0; s < (silu ? 1 : a.n_seg); ++s) total_out += a.n_out[s];
  // About 20 KB of weights per workgroup: under a thousand workgroups for the largest decode
  // matrices (all resident at once), at least 512 for the smallest (below).
  const size_t tile_target = dma ? (silu ? 10240 : 20480) : (silu ? 8192 : 16384);
  uint32_t rows = static_cast<uint32_t>(std::max<size_t>(1, tile_target / row_bytes));
  rows = std::min<uint32_t>(rows, std::max<uint32_t>(1, total_out / 512));
  rows = std::min<uint32_t>(rows, (silu ? 128 : 256) / a.m);
  if (rope) rows = std::max<uint32_t>(2, rows & ~1u);
  // A Q8_0 output needs whole blocks per workgroup: 32 rows, whose tile may exceed 64 KB of LDS.
  const bool outq = a.outq != nullptr;
  if (outq) rows = kQK;
  const size_t kLdsLimit = (outq ? wide_lds_limit(type, dma) : 65536) - 256;  // static LDS beside it
  for (;;) {
    size_t act = 0, tile = 0;
    const size_t lds = fused_lds(bs, a.m, a.nb, rows, silu, &act, &tile);
    if (lds <= kLdsLimit) {
      a.rows = rows;
      a.lds_tile = static_cast<uint32_t>(act);
      a.lds_scratch = static_cast<uint32_t>(act + tile);
      uint32_t wg = 0;
      for (int s = 0; s < a.n_seg; ++s) {
        a.wg_begin[s] = wg;
        if (!silu || s == 0) wg += static_cast<uint32_t>(ceil_div(a.n_out[s], rows));
      }
      if (silu) a.wg_begin[1] = 0;
      // One RMSNorm'd row (one chunk per thread) under at least kNorm1MinWeights of weight copies
      // per workgroup: the staged kernel, its staging after the layout. With fewer, the weights
      // land before the prologue ends either way, and staging the row through LDS only adds its
      // latency (q|k|v at 6 rows per workgroup: 6.16 us plain, 6.64 us staged; gate|up at
      // 2 x 32 rows: 11.44 us plain, 10.88 us staged).
      a.lds_stage = static_cast<uint32_t>((lds + 15) & ~size_t(15));
      const size_t lds1 = a.lds_stage + kNorm1Stage;
      const size_t wg_weights = rows * row_bytes * (silu ? 2 : 1);
      const bool norm1 = dma && a.m == 1 && a.in_mode == kInNorm && a.nb * kQK / 8 <= kThreads &&
                         wg_weights >= kNorm1MinWeights && lds1 <= norm1_lds_limit(type);
      if (norm1) {
        switch (type) {
        case Q8_0: launch(matvec_norm1_kernel<Q8_0>, dim3(wg), dim3(kThreads), lds1, a); break;
        case Q4_0: launch(matvec_norm1_kernel<Q4_0>, dim3(wg), dim3(kThreads), lds1, a); break;
        case Q4_1: launch(matvec_norm1_kernel<Q4_1>, dim3(wg), dim3(kThreads), lds1, a); break;
        default: return fail(kUnsupported, "matvec_fused: weight type %d", type);
        }
      } else if (dma) {
        switch (type) {
        case Q8_0: launch(matvec_dma_kernel<Q8_0>, dim3(wg), dim3(kThreads), lds, a); break;
        case Q4_0: launch(matvec_dma_kernel<Q4_0>, dim3(wg), dim3(kThreads), lds, a); break;
        case Q4_1: launch(matvec_dma_kernel<Q4_1>, dim3(wg), dim3(kThreads), lds, a); break;
        default: return fail(kUnsupported, "matvec_fused: weight type %d", type);
        }
      } else {
        switch (type) {
        case Q8_0: launch(matvec_fused_kernel<Q8_0>, dim3(wg), dim3(kThreads), lds, a); break;
        case Q4_0: launch(matvec_fused_kernel<Q4_0>, dim3(wg), dim3(kThreads), lds, a); break;
        case Q4_1: launch(matvec_fused_kernel<Q4_1>, dim3(wg), dim3(kThreads), lds, a); break;
        default: return fail(kUnsupported, "matvec_fused: weight type %d", type);
        }
      }
      return check_launch("matvec_fused");
    }
    if (outq || rows <= (rope ? 2u : 1u)) return fail(kUnsupported, "matvec_fused: %u blocks x %u rows exceed LDS", a.nb, a.m);
    rows = rope ? std::max<uint32_t>(2, (rows / 2) & ~1u) : rows / 2;
  }
}

}  // namespace axon_hip
