// Grouped-query attention over KV-cache spans, one workgroup per (query row, kv head): the
// table's attention / attention_kv / attention_kv_heads(_f16) entries and the ragged batched
// entry that serves every sequence of a continuous batch in one launch per layer.
//
// Follows trickymind1324/axon-infer src/kernels/ref/attention.cpp:27-59 (and 77-113 for the
// fp16 cache) with softmax from src/kernels/ref/softmax.cpp:10-25:
//   scores[j] = scale * dot(q, k_j), the dot left to right in float, j <= pos;
//   softmax: max, e_j = exp(s_j - max) in float, sum in double, p_j = e_j * float(1 / sum);
//   o[d] = sum over j in ascending order of p_j * v_j[d], in float.
// The score dots run one position per lane (each lane walks d in order), the value mix one
// (head, d) pair per lane (each lane walks j in order), so both float reductions keep the
// scalar table's order. The exponential is evaluated in double and rounded once, and the double
// sum is reduced as a tree; both differ from the scalar table only in rare last-bit cases.
//
// The workgroup's query heads share one kv head, so every K and V row is read from HBM once
// per query row. Scores live in LDS when they fit, otherwise in a global scratch.
#include "common.h"
#include "elementwise.h"

namespace axon_hip {

namespace {

constexpr int kThreads = 256;
// The fused kernel's LDS: q [group][hd], the scores [group][pitch] when they fit, and a value
// tile [hd][kVPitch] (kVTile positions, transposed).
constexpr uint32_t kVTile = 64;
constexpr uint32_t kVPitch = kVTile + 4;
constexpr uint32_t kVGroup = 8;  // positions per register set in the whole-tile value mix
constexpr uint32_t kVMaxItems = kVTile * 128 / 4 / kThreads;  // 4-float items per thread, hd <= 128
// The blocked many-row kernel: blocks of rows only while they leave this many workgroups (two
// per CU), LDS up to this many bytes (two workgroups per CU).
constexpr uint32_t kBlockMinWorkgroups = 512;
constexpr size_t kBlockMaxLds = 80 * 1024;
constexpr int kBlockWaves = 3;  // waves per SIMD the blocked kernel's registers allow

__host__ __device__ inline uint32_t round4(uint32_t v) { return (v + 3) & ~3u; }
__host__ __device__ inline size_t vtile_bytes(uint32_t hd) { return static_cast<size_t>(hd) * kVPitch * 4; }

template <bool F16>
__device__ __forceinline__ float kv_at(const void* base, size_t i) {
  if constexpr (F16) {
    return half_value(reinterpret_cast<const uint16_t*>(base)[i]);
  } else {
    return reinterpret_cast<const float*>(base)[i];
  }
}

// One query row r and kv head g on the whole workgroup; lds holds the q rows, the scores (when
// they fit) and a V tile. With a.outq and 32-dim multiples of head_dim, each half-wave's 32
// outputs are one Q8_0 block of wo's input, quantized as they are stored.
template <bool F16, bool GLOBAL>
__device__ __forceinline__ void attention_row(const AttnArgs& a, uint32_t r, uint32_t g, float* lds) {
  const uint32_t tid = threadIdx.x;
  const uint32_t hd = a.head_dim;
  const uint32_t group = a.n_head / a.n_kv;
  const uint32_t h_lo = max(g * group, a.head_begin);
  const uint32_t h_hi = min(g * group + group, a.head_end);
  if (h_lo >= h_hi) return;
  const uint32_t nh = h_hi - h_lo;

  const int64_t k_off = (a.k_off != nullptr ? a.k_off[r] : 0) + a.k_off_c;
  const int64_t v_off = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * hd;

  float* qs = lds;                                   // [nh][hd]
  __shared__ double red_d[kThreads / 64];
  __shared__ float red_f[kThreads / 64];
  // The global scratch holds [row][head - head_begin][max_vis]: the heads of this launch only.
  float* sc = GLOBAL ? a.scratch + (static_cast<size_t>(r) * (a.head_end - a.head_begin) + (h_lo - a.head_begin)) *
                                       a.max_vis
                     : lds + group * hd;
  const uint32_t pitch = GLOBAL ? a.max_vis : round4(n_vis);

  // 16-byte loads of K rows when every row of this span is 16-byte aligned.
  constexpr uint32_t es = F16 ? 2 : 4;
  const bool vec4 = hd == 64 && ((reinterpret_cast<uintptr_t>(a.kv) + static_cast<uintptr_t>(k_off) * es) & 15u) == 0 &&
                    ((kv_row * es) & 15u) == 0;
  const float* q = a.q + static_cast<size_t>(r) * a.q_stride + static_cast<size_t>(h_lo) * hd;
  for (uint32_t i = tid; i < nh * hd; i += kThreads) qs[i] = q[i];
  __syncthreads();

  // Scores: one position per lane, each dot in d order.
  for (uint32_t j = tid; j < n_vis; j += kThreads) {
    const size_t krow = k_off + j * kv_row + static_cast<size_t>(g) * hd;
    if (vec4) {
      float kr[64];
      if constexpr (F16) {
        const uint4* kp = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.kv) + krow);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint4 t = kp[i];
          const uint32_t w4[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            kr[8 * i + 2 * k] = half_value(w4[k] & 0xffffu);
            kr[8 * i + 2 * k + 1] = half_value(w4[k] >> 16);
          }
        }
      } else {
        const float4* kp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kv) + krow);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float4 t = kp[i];
          kr[4 * i] = t.x;
          kr[4 * i + 1] = t.y;
          kr[4 * i + 2] = t.z;
          kr[4 * i + 3] = t.w;
        }
      }
      for (uint32_t h = 0; h < nh; ++h) {
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < 64; ++d) acc += qs[h * 64 + d] * kr[d];
        sc[h * pitch + j] = a.scale * acc;
      }
    } else {
      for (uint32_t h = 0; h < nh; ++h) {
        float acc = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) acc += qs[h * hd + d] * kv_at<F16>(a.kv, krow + d);
        sc[h * pitch + j] = a.scale * acc;
      }
    }
  }
  __syncthreads();

  // Softmax per head.
  for (uint32_t h = 0; h < nh; ++h) {
    float* s = sc + h * pitch;
    float m = -INFINITY;
    for (uint32_t j = tid; j < n_vis; j += kThreads) m = fmaxf(m, s[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red_f[tid >> 6] = m;
    __syncthreads();
    m = red_f[0];
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red_f[w]);
    double sum = 0.0;
    for (uint32_t j = tid; j < n_vis; j += kThreads) {
      const float e = exp_libm(s[j] - m);
      s[j] = e;
      sum += static_cast<double>(e);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if ((tid & 63) == 0) red_d[tid >> 6] = sum;
    __syncthreads();
    sum = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) sum += red_d[w];
    const float inv = static_cast<float>(1.0 / sum);
    for (uint32_t j = tid; j < n_vis; j += kThreads) s[j] *= inv;
    __syncthreads();
  }

  // Value mix: one (head, d) per lane, positions in ascending order.
  float* out = a.out + static_cast<size_t>(r) * a.out_stride + static_cast<size_t>(h_lo) * hd;
  const uint32_t pairs = nh * hd;
  // Every half-wave stores 32 consecutive outputs of one head (pairs is a multiple of 32).
  const bool quant = a.outq != nullptr && hd % kQK == 0;
  auto store_out = [&](uint32_t t, float v) {
    out[t] = v;
    if (quant) {
      const size_t col = static_cast<size_t>(h_lo) * hd + t;
      quantize_block_lanes(v, tid & 31u, a.outq + (static_cast<size_t>(r) * (a.out_stride / kQK) + col / kQK) * kBytesQ8_0);
    }
  };
  constexpr uint32_t es2 = F16 ? 8 : 16;  // bytes of one 4-element load
  const bool tiled = hd % 4 == 0 && hd <= 128 && pairs <= 4 * kThreads &&
                     ((reinterpret_cast<uintptr_t>(a.kv) + static_cast<uintptr_t>(v_off) * es) % es2) == 0 &&
                     (kv_row * es) % es2 == 0;
  if (tiled) {
    // V tiles of kVTile positions, loaded by the whole workgroup (the next tile's loads in
    // flight while the current one is walked) and stored transposed, [d][position], so a lane
    // reads four positions of its dim, and four of its head's probabilities, per 16-byte read.
    float* vt = lds + group * hd + (GLOBAL ? 0 : group * pitch);
    const uint32_t quads = hd / 4;
    const uint32_t items = kVTile * quads;
    const size_t vcol = v_off + static_cast<size_t>(g) * hd;
    float4 reg[kVMaxItems];
    auto load_tile = [&](uint32_t j0) {
#pragma unroll
      for (uint32_t k = 0; k < kVMaxItems; ++k) {
        const uint32_t it = tid + k * kThreads;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const uint32_t jj = it / quads, dq = it - jj * quads;
        if (it < items && j0 + jj < n_vis) {
          const size_t e = vcol + static_cast<size_t>(j0 + jj) * kv_row + 4 * dq;
          if constexpr (F16) {
            const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.kv) + e);
            v = make_float4(half_value(h.x & 0xffffu), half_value(h.x >> 16), half_value(h.y & 0xffffu),
                            half_value(h.y >> 16));
          } else {
            v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kv) + e);
          }
        }
        reg[k] = v;
      }
    };
    const bool p4 = pitch % 4 == 0;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    load_tile(0);
    for (uint32_t j0 = 0; j0 < n_vis; j0 += kVTile) {
      __syncthreads();  // the previous tile has been read
#pragma unroll
      for (uint32_t k = 0; k < kVMaxItems; ++k) {
        const uint32_t it = tid + k * kThreads;
        if (it < items) {
          const uint32_t jj = it / quads, dq = it - jj * quads;
          float* col = vt + 4 * dq * kVPitch + jj;
          col[0] = reg[k].x;
          col[kVPitch] = reg[k].y;
          col[2 * kVPitch] = reg[k].z;
          col[3 * kVPitch] = reg[k].w;
        }
      }
      __syncthreads();
      if (j0 + kVTile < n_vis) load_tile(j0 + kVTile);
      const uint32_t cnt = min(kVTile, n_vis - j0);
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t t = tid + q * kThreads;
        if (t < pairs) {
          const uint32_t h = t / hd;
          const uint32_t d = t - h * hd;
          const float* pp = sc + h * pitch + j0;
          const float* vv = vt + d * kVPitch;
          float sum = acc[q];
          uint32_t j = 0;
          if (p4 && cnt == kVTile) {
            // A whole tile, kG positions at a time from two register sets: each set's LDS reads
            // are issued a group ahead of its adds, so the chain does not wait on them (read just
            // before their adds, each 4 positions' reads stalled the chain).
            constexpr uint32_t kG = kVGroup, kQ = kG / 4;
            float4 pa[kQ], va[kQ], pb[kQ], vb[kQ];
            auto get = [&](uint32_t j1, float4 (&p4r)[kQ], float4 (&v4r)[kQ]) {
#pragma unroll
              for (uint32_t i = 0; i < kQ; ++i) {
                p4r[i] = *reinterpret_cast<const float4*>(pp + j1 + 4 * i);
                v4r[i] = *reinterpret_cast<const float4*>(vv + j1 + 4 * i);
              }
            };
            auto run = [&](const float4 (&p4r)[kQ], const float4 (&v4r)[kQ]) {
#pragma unroll
              for (uint32_t i = 0; i < kQ; ++i) {
                sum += p4r[i].x * v4r[i].x;
                sum += p4r[i].y * v4r[i].y;
                sum += p4r[i].z * v4r[i].z;
                sum += p4r[i].w * v4r[i].w;
              }
            };
            get(0, pa, va);
            get(kG, pb, vb);
#pragma unroll
            for (uint32_t j1 = 0; j1 < kVTile; j1 += 2 * kG) {
              run(pa, va);
              if (j1 + 2 * kG < kVTile) get(j1 + 2 * kG, pa, va);
              run(pb, vb);
              if (j1 + 3 * kG < kVTile) get(j1 + 3 * kG, pb, vb);
            }
            j = kVTile;
          }
          if (p4) {
            for (; j + 4 <= cnt; j += 4) {
              const float4 p4v = *reinterpret_cast<const float4*>(pp + j);
              const float4 v4 = *reinterpret_cast<const float4*>(vv + j);
              sum += p4v.x * v4.x;
              sum += p4v.y * v4.y;
              sum += p4v.z * v4.z;
              sum += p4v.w * v4.w;
            }
          }
          for (; j < cnt; ++j) sum += pp[j] * vv[j];
          acc[q] = sum;
        }
      }
    }
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
      const uint32_t t = tid + q * kThreads;
      if (t < pairs) store_out(t, acc[q]);
    }
    return;
  }
  for (uint32_t t = tid; t < pairs; t += kThreads) {
    const uint32_t h = t / hd;
    const uint32_t d = t - h * hd;
    const float* p = sc + h * pitch;
    const size_t vbase = v_off + static_cast<size_t>(g) * hd + d;
    float acc = 0.0f;
    uint32_t j = 0;
    for (; j + 4 <= n_vis; j += 4) {
      const float v0 = kv_at<F16>(a.kv, vbase + (j + 0) * kv_row);
      const float v1 = kv_at<F16>(a.kv, vbase + (j + 1) * kv_row);
      const float v2 = kv_at<F16>(a.kv, vbase + (j + 2) * kv_row);
      const float v3 = kv_at<F16>(a.kv, vbase + (j + 3) * kv_row);
      acc += p[j] * v0;
      acc += p[j + 1] * v1;
      acc += p[j + 2] * v2;
      acc += p[j + 3] * v3;
    }
    for (; j < n_vis; ++j) acc += p[j] * kv_at<F16>(a.kv, vbase + j * kv_row);
    store_out(t, acc);
  }
}

template <bool F16, bool GLOBAL>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  attention_row<F16, GLOBAL>(a, blockIdx.x, blockIdx.y, lds);
}

// ---- Many-row launches, several query rows of one sequence per workgroup --------------------
// attention_block_kernel<F16, G, R>: one workgroup per (block of R consecutive query rows, kv
// head), for kv groups of G query heads of 64 dims. When the R rows read one K/V span (the rows
// of a sequence's prefill chunk) and their scores fit the launch's LDS, each K and V row is read
// once for all of them:
//   scores   one position per lane; its K row, held in registers, serves the dot of every
//            (row, head) pair that sees the position, each dot over d in order;
//   softmax  one wave per (row, head) pair: max, exp, the fused kernel's 256-thread double-sum
//            tree (lane l carries the partial sums of threads l, l + 64, l + 128, l + 192), scale;
//   mix      lane = dim; the wave's pairs (wave, wave + 4, ...) are independent chains over
//            positions in ascending order, all reading the one V tile staged in LDS.
// Every float operation and its order are the one-row body's. The rows of any other block (the
// decode rows of a ragged batch) run the one-row body in turn. Blocks are dispatched from the
// last rows down: in a prefill those see the most positions. (A grid of one workgroup per row
// whose other workgroups returned at once measured slower than one per block: 311 against
// 92 us for 512 rows of 32/8 heads.)
template <uint32_t G, uint32_t R>
__host__ __device__ constexpr uint32_t block_pairs() { return G * R; }

// A pair's row of probabilities spans whole V tiles.
__host__ __device__ inline uint32_t block_pitch(uint32_t n_vis) { return (n_vis + kVTile - 1) / kVTile * kVTile; }

__host__ __device__ inline size_t block_lds(uint32_t pairs, uint32_t n_vis) {
  return static_cast<size_t>(pairs) * block_pitch(n_vis) * 4 + vtile_bytes(64);
}

// The rows r0 .. r0 + RR - 1 of one K/V span (nv[i] positions each, 0 for a row past the
// launch) on the whole workgroup: scores, softmax and value mix as described above. VEC: the
// span's K and V rows are 16-byte aligned (vector loads); else element loads.
template <bool F16, uint32_t G, uint32_t RR, bool VEC>
__device__ __forceinline__ void block_rows(const AttnArgs& a, uint32_t r0, uint32_t g, const uint32_t (&nv)[RR],
                                           int64_t k_off, int64_t v_off, float* lds, uint32_t* nv_s,
                                           const uint64_t* exp_tab) {
  constexpr uint32_t kPairs = block_pairs<G, RR>();
  constexpr uint32_t kChains = (kPairs + 3) / 4;
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * 64;
  uint32_t nmax = 0;
#pragma unroll
  for (uint32_t i = 0; i < RR; ++i) nmax = max(nmax, nv[i]);
  if (tid < RR) nv_s[tid] = tid == 0 ? nv[0] : tid == 1 ? nv[RR > 1 ? 1 : 0] : tid == 2 ? nv[RR > 2 ? 2 : 0] : nv[RR - 1];
  __syncthreads();  // nv_s is written (and the previous rows' readers of LDS are done)
  auto vis = [&](uint32_t i) { return nv_s[i]; };

  const uint32_t pitch = block_pitch(nmax);
  float* sc = lds;                  // [pair][pitch], pair = row * G + head
  float* vt = sc + kPairs * pitch;  // [64][kVPitch]

  // Scores: one position per lane; its K row, held in registers, serves the dot of every pair
  // that sees the position. The q rows are wave-uniform and read through the constant address
  // space (scalar loads: the kernel never writes them), so the dots read no LDS.
  using cfloat = const __attribute__((address_space(4))) float;
  const size_t kcol = static_cast<size_t>(k_off) + static_cast<size_t>(g) * 64;
  for (uint32_t j = tid; j < nmax; j += kThreads) {
    const size_t krow = kcol + j * kv_row;
    float kr[64];
    if constexpr (!VEC) {
#pragma unroll
      for (int d = 0; d < 64; ++d) kr[d] = kv_at<F16>(a.kv, krow + d);
    } else if constexpr (F16) {
      const uint4* kp = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.kv) + krow);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint4 t = kp[c];
        const uint32_t w4[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          kr[8 * c + 2 * k] = half_value(w4[k] & 0xffffu);
          kr[8 * c + 2 * k + 1] = half_value(w4[k] >> 16);
        }
      }
    } else {
      const float4* kp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kv) + krow);
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float4 t = kp[c];
        kr[4 * c] = t.x;
        kr[4 * c + 1] = t.y;
        kr[4 * c + 2] = t.z;
        kr[4 * c + 3] = t.w;
      }
    }
#pragma unroll
    for (uint32_t i = 0; i < RR; ++i) {
      if (j < nv[i]) {
        cfloat* qrow = (cfloat*)(a.q + static_cast<size_t>(r0 + i) * a.q_stride + static_cast<size_t>(g) * G * 64);
#pragma unroll 1
        for (uint32_t h = 0; h < G; ++h) {
          cfloat* qh = qrow + h * 64;
          float acc = 0.0f;
#pragma unroll
          for (int d = 0; d < 64; ++d) acc += qh[d] * kr[d];
          sc[(i * G + h) * pitch + j] = a.scale * acc;
        }
      }
    }
  }
  __syncthreads();

  // Softmax, one wave per pair, the wave's pairs (wave, wave + 4, ...) side by side. Each pair's
  // row is zeroed past its positions to the end of the last V tile, so that the value mix can run
  // whole tiles.
  uint32_t cpair[kChains], cvis[kChains];
  float* cs[kChains];
  uint32_t nhi = 0;
#pragma unroll
  for (uint32_t c = 0; c < kChains; ++c) {
    const uint32_t pr = wave + 4 * c;
    cpair[c] = min(pr, kPairs - 1);
    cvis[c] = pr < kPairs ? vis(cpair[c] / G) : 0;
    cs[c] = sc + cpair[c] * pitch;
    nhi = max(nhi, cvis[c]);
  }
  {
    float m[kChains];
#pragma unroll
    for (uint32_t c = 0; c < kChains; ++c) m[c] = -INFINITY;
    for (uint32_t j = lane; j < nhi; j += 64) {
#pragma unroll
      for (uint32_t c = 0; c < kChains; ++c)
        if (j < cvis[c]) m[c] = fmaxf(m[c], cs[c][j]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
      for (uint32_t c = 0; c < kChains; ++c) m[c] = fmaxf(m[c], __shfl_xor(m[c], off, 64));
    }
    double part[kChains][4];
#pragma unroll
    for (uint32_t c = 0; c < kChains; ++c)
#pragma unroll
      for (int w = 0; w < 4; ++w) part[c][w] = 0.0;
    for (uint32_t j = lane; j < nhi; j += 64) {
#pragma unroll
      for (uint32_t c = 0; c < kChains; ++c)
        if (j < cvis[c]) cs[c][j] = exp_libm_from(cs[c][j] - m[c], exp_tab);
    }
    for (uint32_t j0 = 0; j0 < nhi; j0 += 256) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t j = j0 + 64 * w + lane;
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c)
          if (j < cvis[c]) part[c][w] += static_cast<double>(cs[c][j]);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
      for (uint32_t c = 0; c < kChains; ++c)
#pragma unroll
        for (int w = 0; w < 4; ++w) part[c][w] += __shfl_xor(part[c][w], off, 64);
    }
    float inv[kChains];
#pragma unroll
    for (uint32_t c = 0; c < kChains; ++c) {
      double sum = 0.0;
#pragma unroll
      for (int w = 0; w < 4; ++w) sum += part[c][w];
      inv[c] = static_cast<float>(1.0 / sum);
    }
    for (uint32_t j = lane; j < pitch; j += 64) {
#pragma unroll
      for (uint32_t c = 0; c < kChains; ++c)
        if (wave + 4 * c < kPairs) cs[c][j] = j < cvis[c] ? cs[c][j] * inv[c] : 0.0f;
    }
  }

  // Value mix over V tiles of kVTile positions, stored transposed ([d][position]); the next
  // tile's loads fly while the current one is walked. A pair's positions past its own are added
  // as 0 * 0 (both factors selected to zero), which leaves its sum unchanged.
  constexpr uint32_t kItems = kVTile * 16 / kThreads;  // float4 per thread per tile
  const size_t vcol = static_cast<size_t>(v_off) + static_cast<size_t>(g) * 64;
  float4 reg[kItems];
  auto load_tile = [&](uint32_t j0) {
#pragma unroll
    for (uint32_t k = 0; k < kItems; ++k) {
      const uint32_t it = tid + k * kThreads;
      const uint32_t jj = it / 16, dq = it % 16;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (j0 + jj < nmax) {
        const size_t e = vcol + static_cast<size_t>(j0 + jj) * kv_row + 4 * dq;
        if constexpr (!VEC) {
          v = make_float4(kv_at<F16>(a.kv, e), kv_at<F16>(a.kv, e + 1), kv_at<F16>(a.kv, e + 2), kv_at<F16>(a.kv, e + 3));
        } else if constexpr (F16) {
          const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.kv) + e);
          v = make_float4(half_value(h.x & 0xffffu), half_value(h.x >> 16), half_value(h.y & 0xffffu),
                          half_value(h.y >> 16));
        } else {
          v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kv) + e);
        }
      }
      reg[k] = v;
    }
  };
  float acc[kChains];
#pragma unroll
  for (uint32_t c = 0; c < kChains; ++c) acc[c] = 0.0f;
  const float* vv = vt + lane * kVPitch;
  load_tile(0);
  for (uint32_t j0 = 0; j0 < nmax; j0 += kVTile) {
    __syncthreads();  // the previous tile has been read (and, the first time, the softmax is done)
#pragma unroll
    for (uint32_t k = 0; k < kItems; ++k) {
      const uint32_t it = tid + k * kThreads;
      const uint32_t jj = it / 16, dq = it % 16;
      float* col = vt + 4 * dq * kVPitch + jj;
      col[0] = reg[k].x;
      col[kVPitch] = reg[k].y;
      col[2 * kVPitch] = reg[k].z;
      col[3 * kVPitch] = reg[k].w;
    }
    __syncthreads();
    if (j0 + kVTile < nmax) load_tile(j0 + kVTile);
    // Positions of this tile each chain adds (a chain past kPairs counts as whole: its sum is
    // never stored).
    bool full = true;
    uint32_t cnt[kChains];
#pragma unroll
    for (uint32_t c = 0; c < kChains; ++c) {
      cnt[c] = wave + 4 * c >= kPairs ? kVTile : cvis[c] > j0 ? min(kVTile, cvis[c] - j0) : 0;
      full = full && cnt[c] == kVTile;
    }
    // kSetQ * 4 positions per register set, two sets: each set's LDS reads are issued a set ahead
    // of its adds.
    constexpr uint32_t kSetQ = 1, kSet = 4 * kSetQ;
    float4 va[kSetQ], vb[kSetQ], pa[kChains][kSetQ], pb[kChains][kSetQ];
    auto get = [&](uint32_t j1, float4 (&v)[kSetQ], float4 (&pv)[kChains][kSetQ]) {
#pragma unroll
      for (uint32_t u = 0; u < kSetQ; ++u) v[u] = *reinterpret_cast<const float4*>(vv + j1 + 4 * u);
#pragma unroll
      for (uint32_t c = 0; c < kChains; ++c)
#pragma unroll
        for (uint32_t u = 0; u < kSetQ; ++u) pv[c][u] = *reinterpret_cast<const float4*>(cs[c] + j0 + j1 + 4 * u);
    };
    auto run = [&](const float4 (&v)[kSetQ], const float4 (&pv)[kChains][kSetQ]) {
#pragma unroll
      for (uint32_t u = 0; u < kSetQ; ++u) {
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) acc[c] += pv[c][u].x * v[u].x;
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) acc[c] += pv[c][u].y * v[u].y;
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) acc[c] += pv[c][u].z * v[u].z;
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) acc[c] += pv[c][u].w * v[u].w;
      }
    };
    auto run_masked = [&](const float4 (&v)[kSetQ], const float4 (&pv)[kChains][kSetQ], uint32_t j1) {
      auto term = [&](uint32_t c, uint32_t jj, float pq, float vq) {
        const bool in = jj < cnt[c];
        acc[c] += (in ? pq : 0.0f) * (in ? vq : 0.0f);
      };
#pragma unroll
      for (uint32_t u = 0; u < kSetQ; ++u) {
        const uint32_t jj = j1 + 4 * u;
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) term(c, jj, pv[c][u].x, v[u].x);
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) term(c, jj + 1, pv[c][u].y, v[u].y);
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) term(c, jj + 2, pv[c][u].z, v[u].z);
#pragma unroll
        for (uint32_t c = 0; c < kChains; ++c) term(c, jj + 3, pv[c][u].w, v[u].w);
      }
    };
    get(0, va, pa);
    get(kSet, vb, pb);
    if (full) {
#pragma unroll
      for (uint32_t j1 = 0; j1 < kVTile; j1 += 2 * kSet) {
        run(va, pa);
        if (j1 + 2 * kSet < kVTile) get(j1 + 2 * kSet, va, pa);
        run(vb, pb);
        if (j1 + 3 * kSet < kVTile) get(j1 + 3 * kSet, vb, pb);
      }
    } else {
#pragma unroll
      for (uint32_t j1 = 0; j1 < kVTile; j1 += 2 * kSet) {
        run_masked(va, pa, j1);
        if (j1 + 2 * kSet < kVTile) get(j1 + 2 * kSet, va, pa);
        run_masked(vb, pb, j1 + kSet);
        if (j1 + 3 * kSet < kVTile) get(j1 + 3 * kSet, vb, pb);
      }
    }
  }
  const size_t nbq = a.out_stride / kQK;
#pragma unroll
  for (uint32_t c = 0; c < kChains; ++c) {
    const uint32_t pr = wave + 4 * c;
    const uint32_t r = r0 + pr / G;
    if (pr < kPairs && cvis[c] > 0) {
      const size_t col = static_cast<size_t>(g * G + pr % G) * 64 + lane;
      a.out[static_cast<size_t>(r) * a.out_stride + col] = acc[c];
      if (a.outq != nullptr)
        quantize_block_lanes(acc[c], lane & 31u, a.outq + (static_cast<size_t>(r) * nbq + col / kQK) * kBytesQ8_0);
    }
  }
}

template <bool F16, uint32_t G, uint32_t R>
__global__ __launch_bounds__(kThreads, kBlockWaves) void attention_block_kernel(AttnArgs a, uint32_t n_rows, uint32_t lds_bytes) {
  static_assert(R >= 1 && R <= 4 && G * R <= 16, "block shape");
  constexpr uint32_t es = F16 ? 2 : 4;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ uint32_t nv_s[R];
  __shared__ uint64_t exp_tab[32];
  const uint32_t tid = threadIdx.x;
  const uint32_t g = blockIdx.x % a.n_kv;
  const uint32_t n_blocks = (n_rows + R - 1) / R;
  const uint32_t r0 = (n_blocks - 1 - blockIdx.x / a.n_kv) * R;
  if (tid < 32) exp_tab[tid] = kExp2Tab[tid];

  // Each row's span and positions; the block shares row r0's span when every other row has it.
  int64_t k_off[R], v_off[R];
  uint32_t nv[R];
  bool shared = true;
#pragma unroll
  for (uint32_t i = 0; i < R; ++i) {
    const uint32_t r = min(r0 + i, n_rows - 1);
    k_off[i] = (a.k_off != nullptr ? a.k_off[r] : 0) + a.k_off_c;
    v_off[i] = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;
    nv[i] = r0 + i < n_rows
                ? (a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1)
                : 0;
    if (i > 0 && nv[i] > 0) shared = shared && k_off[i] == k_off[0] && v_off[i] == v_off[0];
  }
  uint32_t nmax = 0;
#pragma unroll
  for (uint32_t i = 0; i < R; ++i) nmax = max(nmax, nv[i]);
  const uintptr_t base = reinterpret_cast<uintptr_t>(a.kv);
  auto aligned = [&](uint32_t i) {
    return ((base + static_cast<uintptr_t>(k_off[i]) * es) & 15u) == 0 &&
           ((base + static_cast<uintptr_t>(v_off[i]) * es) & 15u) == 0;
  };
  if (shared && aligned(0) && block_lds(G * R, nmax) <= lds_bytes) {
    block_rows<F16, G, R, true>(a, r0, g, nv, k_off[0], v_off[0], lds, nv_s, exp_tab);
    return;
  }
  // One row at a time (a single row's scores always fit: the launch is sized for max_vis).
#pragma unroll
  for (uint32_t i = 0; i < R; ++i) {
    if (nv[i] == 0) continue;
    const uint32_t one[1] = {nv[i]};
    if (aligned(i)) block_rows<F16, G, 1, true>(a, r0 + i, g, one, k_off[i], v_off[i], lds, nv_s, exp_tab);
    else block_rows<F16, G, 1, false>(a, r0 + i, g, one, k_off[i], v_off[i], lds, nv_s, exp_tab);
  }
}

// The block kernel's LDS beyond 64 KB must be granted once per instantiation; false when the
// launch's LDS exceeds what the device grants.
template <bool F16, uint32_t G, uint32_t R>
bool block_lds_granted(size_t need) {
  static int limit = -1;
  if (limit < 0) {
    int dev = 0, v = 0;
    limit = (hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess)
                ? v
                : 65536;
    limit = std::min(limit, static_cast<int>(kBlockMaxLds));
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(attention_block_kernel<F16, G, R>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, limit) != hipSuccess)
      limit = 65536;
  }
  return need <= static_cast<size_t>(limit);
}

// The launch's LDS: the one-row body's at max_vis, raised to the blocks' need up to
// kBlockMaxLds; blocks whose scores do not fit run one row per workgroup.
template <bool F16, uint32_t G, uint32_t R>
bool try_block(const AttnArgs& a, uint32_t n_rows) {
  const size_t one = block_lds(G, a.max_vis);
  const size_t lds = std::max(one, std::min(block_lds(G * R, a.max_vis), kBlockMaxLds));
  if (!block_lds_granted<F16, G, R>(lds)) return false;
  hipLaunchKernelGGL((attention_block_kernel<F16, G, R>), dim3((n_rows + R - 1) / R * a.n_kv), dim3(kThreads), lds, stream(), a,
                     n_rows, static_cast<uint32_t>(lds));
  return true;
}

// The largest block of R rows (R * G <= 16) that still leaves kBlockMinWorkgroups workgroups,
// else single rows.
template <uint32_t G>
bool launch_block_g(const AttnArgs& a, uint32_t n_rows) {
  auto enough = [&](uint32_t r) { return (n_rows + r - 1) / r * a.n_kv >= kBlockMinWorkgroups; };
  if constexpr (G <= 4) {
    if (enough(4)) return a.f16 ? try_block<true, G, 4>(a, n_rows) : try_block<false, G, 4>(a, n_rows);
  }
  if (enough(2)) return a.f16 ? try_block<true, G, 2>(a, n_rows) : try_block<false, G, 2>(a, n_rows);
  return a.f16 ? try_block<true, G, 1>(a, n_rows) : try_block<false, G, 1>(a, n_rows);
}

// The blocked kernel for whole-head launches of 64-dim heads and kv groups of 3, 4, 7 or 8
// query heads; false when it does not apply (the one-row kernel runs instead).
bool launch_block(const AttnArgs& a, uint32_t n_rows) {
  if (a.head_dim != 64 || a.head_begin != 0 || a.head_end != a.n_head) return false;
  switch (a.n_head / a.n_kv) {
  case 3: return launch_block_g<3>(a, n_rows);
  case 4: return launch_block_g<4>(a, n_rows);
  case 7: return launch_block_g<7>(a, n_rows);
  case 8: return launch_block_g<8>(a, n_rows);
  default: return false;
  }
}

// ---- Decode-shaped launches: scores and value mix as two kernels ----------------------------
// With few query rows the one-workgroup-per-(row, kv head) kernel above runs on a handful of
// CUs and its value loop waits on memory. These two kernels spread the same arithmetic wider:
//   attn_scores_kernel  one lane per (row, position), every head of the kv group, written to
//                       a global score buffer S[row][head][max_vis];
//   attn_mix_kernel     one workgroup per (row, kv head, slice of kDc head dims): softmax of the
//                       group's score rows (identical in every slice), then the value mix, each
//                       lane owning one (head, dim) and walking positions in order over value
//                       tiles staged in LDS by the whole workgroup.
// Every float operation and its order are those of the fused kernel.

// Head dims per mix workgroup: 8 (more workgroups, deeper tiles) or 32 (one whole Q8_0 block of
// each head, so the epilogue can quantize the output). Either way a value tile is 2048 floats.
constexpr uint32_t kTileFloats = 2048;

__host__ __device__ inline uint32_t score_pitch(uint32_t max_vis) { return (max_vis + 3) & ~3u; }

template <bool F16>
__global__ __launch_bounds__(kThreads) void attn_scores_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float qs[];  // [group][hd]
  const uint32_t r = blockIdx.x;
  const uint32_t g = blockIdx.y;
  const uint32_t tid = threadIdx.x;
  const uint32_t hd = a.head_dim;
  const uint32_t group = a.n_head / a.n_kv;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const uint32_t j0 = blockIdx.z * kThreads;
  if (j0 >= n_vis) return;
  const int64_t k_off = (a.k_off != nullptr ? a.k_off[r] : 0) + a.k_off_c;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * hd;
  const float* q = a.q + static_cast<size_t>(r) * a.q_stride + static_cast<size_t>(g) * group * hd;
  for (uint32_t i = tid; i < group * hd; i += kThreads) qs[i] = q[i];
  __syncthreads();
  const uint32_t j = j0 + tid;
  if (j >= n_vis) return;
  float* out = a.scratch + (static_cast<size_t>(r) * a.n_head + static_cast<size_t>(g) * group) * a.max_vis + j;
  const size_t krow = k_off + j * kv_row + static_cast<size_t>(g) * hd;
  const bool vec4 = !F16 && hd == 64 &&
                    ((reinterpret_cast<uintptr_t>(reinterpret_cast<const float*>(a.kv) + krow) & 15u) == 0);
  if (vec4) {
    float kr[64];
    const float4* kp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kv) + krow);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4 t = kp[i];
      kr[4 * i] = t.x;
      kr[4 * i + 1] = t.y;
      kr[4 * i + 2] = t.z;
      kr[4 * i + 3] = t.w;
    }
    for (uint32_t h = 0; h < group; ++h) {
      float acc = 0.0f;
#pragma unroll
      for (int d = 0; d < 64; ++d) acc += qs[h * 64 + d] * kr[d];
      out[static_cast<size_t>(h) * a.max_vis] = a.scale * acc;
    }
  } else {
    for (uint32_t h = 0; h < group; ++h) {
      float acc = 0.0f;
      for (uint32_t d = 0; d < hd; ++d) acc += qs[h * hd + d] * kv_at<F16>(a.kv, krow + d);
      out[static_cast<size_t>(h) * a.max_vis] = a.scale * acc;
    }
  }
}

template <bool F16, uint32_t kDc>
__global__ __launch_bounds__(kThreads) void attn_mix_kernel(AttnArgs a) {
  constexpr uint32_t kTile = kTileFloats / kDc;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ double red_d[kThreads / 64];
  __shared__ float red_f[kThreads / 64];
  const uint32_t r = blockIdx.x;
  const uint32_t g = blockIdx.y;
  const uint32_t d0 = blockIdx.z * kDc;
  const uint32_t tid = threadIdx.x;
  const uint32_t hd = a.head_dim;
  const uint32_t group = a.n_head / a.n_kv;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const int64_t v_off = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * hd;
  const uint32_t dc = min(kDc, hd - d0);

  const uint32_t pitch = score_pitch(n_vis);
  float* p = lds;                               // [group][pitch]
  float* vt = lds + group * pitch;              // [2][kTile][kDc]
  const float* s = a.scratch + (static_cast<size_t>(r) * a.n_head + static_cast<size_t>(g) * group) * a.max_vis;
  for (uint32_t i = tid; i < group * n_vis; i += kThreads) {
    const uint32_t h = i / n_vis;
    const uint32_t j = i - h * n_vis;
    p[h * pitch + j] = s[static_cast<size_t>(h) * a.max_vis + j];
  }
  __syncthreads();
  for (uint32_t h = 0; h < group; ++h) {
    float* row = p + h * pitch;
    float m = -INFINITY;
    for (uint32_t j = tid; j < n_vis; j += kThreads) m = fmaxf(m, row[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red_f[tid >> 6] = m;
    __syncthreads();
    m = red_f[0];
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red_f[w]);
    double sum = 0.0;
    for (uint32_t j = tid; j < n_vis; j += kThreads) {
      const float e = exp_libm(row[j] - m);
      row[j] = e;
      sum += static_cast<double>(e);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if ((tid & 63) == 0) red_d[tid >> 6] = sum;
    __syncthreads();
    sum = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) sum += red_d[w];
    const float inv = static_cast<float>(1.0 / sum);
    for (uint32_t j = tid; j < n_vis; j += kThreads) row[j] *= inv;
    __syncthreads();
  }

  // Value tiles: tile t holds positions [t*kTile, t*kTile + kTile) x dims [d0, d0 + dc).
  constexpr uint32_t kPer = kTile * kDc / kThreads;
  const uint32_t n_tiles = (n_vis + kTile - 1) / kTile;
  const uint32_t per_tile = kTile * kDc;  // floats
  auto fetch = [&](uint32_t t, float (&reg)[kPer]) {
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) {
      const uint32_t i = tid + k * kThreads;
      const uint32_t jj = i / kDc;
      const uint32_t dd = i - jj * kDc;
      const uint32_t j = t * kTile + jj;
      reg[k] = (j < n_vis && dd < dc) ? kv_at<F16>(a.kv, v_off + j * kv_row + static_cast<size_t>(g) * hd + d0 + dd) : 0.0f;
    }
  };
  float reg[kPer];
  fetch(0, reg);
#pragma unroll
  for (uint32_t k = 0; k < kPer; ++k) vt[tid + k * kThreads] = reg[k];
  __syncthreads();
  const bool lane_active = tid < group * kDc;
  const uint32_t h = tid / kDc;
  const uint32_t dd = tid - h * kDc;
  float acc = 0.0f;
  for (uint32_t t = 0; t < n_tiles; ++t) {
    float* cur = vt + (t & 1) * per_tile;
    float* nxt = vt + ((t + 1) & 1) * per_tile;
    if (t + 1 < n_tiles) fetch(t + 1, reg);
    if (lane_active && dd < dc) {
      const float* pr = p + h * pitch + t * kTile;
      const uint32_t cnt = min(kTile, n_vis - t * kTile);
      if (cnt == kTile) {
        // positions in order; scores read four at a time, values one per position
#pragma unroll
        for (uint32_t jj = 0; jj < kTile; jj += 4) {
          const float4 pp = *reinterpret_cast<const float4*>(pr + jj);
          acc += pp.x * cur[(jj + 0) * kDc + dd];
          acc += pp.y * cur[(jj + 1) * kDc + dd];
          acc += pp.z * cur[(jj + 2) * kDc + dd];
          acc += pp.w * cur[(jj + 3) * kDc + dd];
        }
      } else {
        for (uint32_t jj = 0; jj < cnt; ++jj) acc += pr[jj] * cur[jj * kDc + dd];
      }
    }
    if (t + 1 < n_tiles) {
#pragma unroll
      for (uint32_t k = 0; k < kPer; ++k) nxt[tid + k * kThreads] = reg[k];
    }
    __syncthreads();
  }
  if (lane_active && dd < dc) {
    const size_t col = static_cast<size_t>(g * group + h) * hd + d0 + dd;
    a.out[static_cast<size_t>(r) * a.out_stride + col] = acc;
    // The Q8_0 block of dims [d0, d0 + 32) of head h: one half-wave (wo's input, llama.cpp:401-417).
    if (kDc == kQK && a.outq != nullptr) {
      const size_t nbq = a.out_stride / kQK;
      quantize_block_lanes(acc, dd, a.outq + (static_cast<size_t>(r) * nbq + col / kQK) * kBytesQ8_0);
    }
  }
}

// ---- Decode-shaped launches, 64-dim heads of an fp32 cache --------------------------------
//   attn_scores64_kernel  one workgroup per (row, kv head, 64 positions): the 64 K rows go into
//                         LDS by 16-byte DMA copies, wave h computes query head h's scores, one
//                         lane per position, each dot over d in order.
//   attn_mix64_kernel     one wave per (row, query head): the softmax statistics, then the
//                         value mix with lane = dim, positions in order, V streaming through a
//                         ring of LDS tiles that DMA keeps kRing tiles ahead.
// The float operations and their order are the fused kernel's, and the double sum of the
// softmax follows the fused kernel's 256-thread tree (each lane carries the partial sums of
// threads lane, lane + 64, lane + 128, lane + 192).
// attn_scores64_kernel's LDS: 64 K rows of 64 elements, the group's q rows.
inline size_t scores64_lds(bool f16, uint32_t group) { return 64 * 64 * (f16 ? 2 : 4) + static_cast<size_t>(group) * 64 * 4; }

// F16: the cache holds fp16 bit patterns; each K value is widened exactly before its product.
// The 64 K rows go into LDS unpadded by 16-byte copies (4 rows of floats, or 8 of fp16, per
// copy), each row's 16-byte chunks stored XOR-swizzled by the row: chunk c of row j sits in slot
// c ^ (j % chunks), so the lanes (one row each) reading chunk c in the same step hit different
// banks, while each lane still reads its row's chunks, and adds its products, in order.
template <bool F16>
__global__ __launch_bounds__(1024) void attn_scores64_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];  // K [64][64 elements], q [group][64]
  const uint32_t r = blockIdx.x;
  const uint32_t g = blockIdx.y;
  const uint32_t j0 = blockIdx.z * 64;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  if (j0 >= n_vis) return;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t group = a.n_head / a.n_kv;
  const uint32_t rows = min(64u, n_vis - j0);
  const size_t kv_row = static_cast<size_t>(a.n_kv) * 64;
  const int64_t k_off = (a.k_off != nullptr ? a.k_off[r] : 0) + a.k_off_c;
  constexpr uint32_t es = F16 ? 2 : 4;         // bytes per cache element
  constexpr uint32_t kChunks = 64 * es / 16;   // 16-byte chunks per K row: 16, or 8 in fp16
  constexpr uint32_t kRowsPer = 64 / kChunks;  // rows per copy: 4, or 8
  float* kt = lds;
  float* qs = lds + 64 * 64 * es / 4;
  // K rows j0 .. j0 + 63 of kv head g (rows past n_vis repeat the last one); copy i moves rows
  // kRowsPer i .. kRowsPer i + kRowsPer - 1, waves taking copies in turn.
  const uint8_t* kbase = static_cast<const uint8_t*>(a.kv) + (k_off + static_cast<size_t>(j0) * kv_row + g * 64) * es;
  const RsrcWords rsrc = raw_buffer_words(kbase, static_cast<uint32_t>((static_cast<size_t>(rows - 1) * kv_row + 64) * es));
  const uint32_t kt_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(kt)));
  for (uint32_t i = wave; i < 64 / kRowsPer; i += group) {
    const uint32_t row = kRowsPer * i + lane / kChunks;
    const uint32_t chunk = (lane % kChunks) ^ (row % kChunks);
    lds_dma16(rsrc, static_cast<uint32_t>(min(row, rows - 1) * kv_row * es) + chunk * 16, kt_lds + i * 1024);
  }
  const float* q = a.q + static_cast<size_t>(r) * a.q_stride + static_cast<size_t>(g) * group * 64;
  for (uint32_t i = tid; i < group * 64; i += blockDim.x) qs[i] = q[i];
  wait_memory();
  __syncthreads();
  const uint32_t j = j0 + lane;
  if (j >= n_vis) return;
  const uint4* kr = reinterpret_cast<const uint4*>(kt) + lane * kChunks;
  const float* qh = qs + wave * 64;
  const uint32_t sw = lane % kChunks;
  float acc = 0.0f;
  if constexpr (F16) {
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
      const uint4 h = kr[c ^ sw];
      const float4 qa = *reinterpret_cast<const float4*>(qh + 8 * c);
      const float4 qb = *reinterpret_cast<const float4*>(qh + 8 * c + 4);
      acc += mul_half_bits(qa.x, h.x);
      acc += mul_half_bits_hi(qa.y, h.x);
      acc += mul_half_bits(qa.z, h.y);
      acc += mul_half_bits_hi(qa.w, h.y);
      acc += mul_half_bits(qb.x, h.z);
      acc += mul_half_bits_hi(qb.y, h.z);
      acc += mul_half_bits(qb.z, h.w);
      acc += mul_half_bits_hi(qb.w, h.w);
    }
  } else {
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
      const uint4 u = kr[c ^ sw];
      const float4 q4 = *reinterpret_cast<const float4*>(qh + 4 * c);
      acc += q4.x * __uint_as_float(u.x);
      acc += q4.y * __uint_as_float(u.y);
      acc += q4.z * __uint_as_float(u.z);
      acc += q4.w * __uint_as_float(u.w);
    }
  }
  a.scratch[(static_cast<size_t>(r) * a.n_head + g * group + wave) * a.max_vis + j] = a.scale * acc;
}

constexpr uint32_t kMixTile = 32;  // positions per V tile (8 KB)
constexpr uint32_t kRing = 6;      // V tiles in flight (kRing * 8 DMA ops <= vmcnt's 63)
// The probabilities of one head's row (rows of more positions take the other paths).
constexpr uint32_t kMixMaxVis = 2304;

// The V rings are filled by LDS-DMA issued from inline assembly (common.h), and their waits
// are explicit: the compiler's own wait counting, which cannot tell the copies into one ring
// slot from those into another across loop iterations, would otherwise drain every copy before
// each tile.

__global__ __launch_bounds__(64) void attn_mix64_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float ring[kRing * kMixTile * 64];
  __shared__ __attribute__((aligned(16))) float p[kMixMaxVis];
  const uint32_t r = blockIdx.x;
  const uint32_t h = blockIdx.y;
  const uint32_t lane = threadIdx.x;
  const uint32_t group = a.n_head / a.n_kv;
  const uint32_t g = h / group;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * 64;
  const int64_t v_off = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;
  const float* s = a.scratch + (static_cast<size_t>(r) * a.n_head + h) * a.max_vis;

  // V tile t = rows t*32 .. t*32+31 (rows past n_vis repeat the last one): 8 copies of 4 rows
  // (64 lanes x 16 bytes = 1 KB contiguous in LDS) into ring slot t % kRing.
  const float* vbase = reinterpret_cast<const float*>(a.kv) + v_off + g * 64;
  const RsrcWords rsrc =
      raw_buffer_words(vbase, static_cast<uint32_t>((static_cast<size_t>(n_vis - 1) * kv_row + 64) * 4));
  const uint32_t ring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(ring)));
  const uint32_t n_tiles = (n_vis + kMixTile - 1) / kMixTile;
  // The head's scores into p first (64 per copy), so that the softmax reads LDS.
  const RsrcWords ssrc = raw_buffer_words(s, n_vis * 4);
  const uint32_t p_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(p)));
  for (uint32_t j0 = 0; j0 < n_vis; j0 += 64) lds_dma4(ssrc, 4 * (j0 + lane), p_lds + 4 * j0);
  auto copy_tile = [&](uint32_t t) {
    const uint32_t dst = ring_lds + (t % kRing) * kMixTile * 64 * 4;
#pragma unroll
    for (uint32_t k = 0; k < kMixTile / 4; ++k) {
      const uint32_t row = min(t * kMixTile + 4 * k + lane / 16, n_vis - 1);
      lds_dma16(rsrc, static_cast<uint32_t>(row * kv_row * 4 + (lane % 16) * 16), dst + 4 * k * 64 * 4);
    }
  };
  for (uint32_t t = 0; t < kRing; ++t) copy_tile(t);

  // Softmax in p while the V tiles arrive (the score copies are older than the 48 tile copies):
  // max, e_j = exp(s_j - max) with the double sum of the fused kernel's tree, p_j = e_j *
  // float(1 / sum). Lanes read back only the positions they copied until the max is known.
  asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
  float m = -INFINITY;
  for (uint32_t j = lane; j < n_vis; j += 64) m = fmaxf(m, p[j]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  double part[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    for (uint32_t j = lane + 64 * w; j < n_vis; j += 256) {
      const float e = exp_libm(p[j] - m);
      p[j] = e;
      part[w] += static_cast<double>(e);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part[w] += __shfl_xor(part[w], off, 64);
  }
  double sum = 0.0;
#pragma unroll
  for (int w = 0; w < 4; ++w) sum += part[w];
  const float inv = static_cast<float>(1.0 / sum);
  for (uint32_t j = lane; j < n_vis; j += 64) p[j] = p[j] * inv;

  // Value mix, positions in order, software-pipelined: while tile t is mixed from registers,
  // the LDS reads of tile t + 1 are in flight. Tile t's slot takes tile t + kRing as soon as
  // its registers are loaded (copies past the last tile re-read the last row, never used).
  // Before tile t + 1 is read from LDS its 8 copies are the oldest of the kRing * 8 in flight.
  float acc = 0.0f;
  float va[kMixTile], pa[kMixTile], vb[kMixTile], pb[kMixTile];
  auto load_tile = [&](uint32_t t, float (&v)[kMixTile], float (&pp)[kMixTile]) {
    const float* vt = ring + (t % kRing) * kMixTile * 64;
    const float* pt = p + t * kMixTile;
#pragma unroll
    for (uint32_t i = 0; i < kMixTile; ++i) v[i] = vt[i * 64 + lane];
#pragma unroll
    for (uint32_t i = 0; i < kMixTile; i += 4) {
      const float4 q4 = *reinterpret_cast<const float4*>(pt + i);
      pp[i] = q4.x;
      pp[i + 1] = q4.y;
      pp[i + 2] = q4.z;
      pp[i + 3] = q4.w;
    }
  };
  auto mix_tile = [&](const float (&v)[kMixTile], const float (&pp)[kMixTile], uint32_t t) {
    const uint32_t cnt = min(kMixTile, n_vis - t * kMixTile);
#pragma unroll
    for (uint32_t i = 0; i < kMixTile; ++i) {
      if (i < cnt) acc += pp[i] * v[i];
    }
  };
  // One step: tile t's registers are loaded into (v, pp); refill its slot, start reading tile
  // t + 1 into (vn, pn), then mix tile t.
  auto step = [&](uint32_t t, float (&v)[kMixTile], float (&pp)[kMixTile], float (&vn)[kMixTile],
                  float (&pn)[kMixTile]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    copy_tile(t + kRing);
    if (t + 1 < n_tiles) {
      asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
      load_tile(t + 1, vn, pn);
    }
    mix_tile(v, pp, t);
  };
  asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
  load_tile(0, va, pa);
  for (uint32_t t = 0; t < n_tiles; t += 2) {
    step(t, va, pa, vb, pb);
    if (t + 1 < n_tiles) step(t + 1, vb, pb, va, pa);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy outlives the wave
  const size_t col = static_cast<size_t>(h) * 64 + lane;
  a.out[static_cast<size_t>(r) * a.out_stride + col] = acc;
  if (a.outq != nullptr) {
    const size_t nbq = a.out_stride / kQK;
    quantize_block_lanes(acc, lane & 31u, a.outq + (static_cast<size_t>(r) * nbq + col / kQK) * kBytesQ8_0);
  }
}

// One workgroup per (row, kv head) for groups of G = 1, 2, 4 or 8 query heads: wave w owns
// query head g * G + w (lane = dim), its softmax in its own row of p, and one G-th of the copies
// of every V tile, which all G waves then mix. The V rows of the group are streamed once.
constexpr uint32_t kGRing = 3;  // V tiles in flight

// Rows of p hold whole 64-position copies (the last copy of a row writes up to 63 past n_vis).
__host__ __device__ inline uint32_t mixg_pitch(uint32_t max_vis) { return (max_vis + 63) & ~63u; }

size_t mixg_lds(uint32_t group, uint32_t max_vis) {
  return (static_cast<size_t>(kGRing) * kMixTile * 64 + static_cast<size_t>(group) * mixg_pitch(max_vis)) * 4;
}

template <int G>
__global__ __launch_bounds__(G * 64) void attn_mixg_kernel(AttnArgs a) {
  constexpr uint32_t kOps = 8 / G;  // copies per wave per tile (a tile is 8 copies of 1 KB)
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* ring = lds;                                  // [kGRing][kMixTile][64]
  const uint32_t pitch = mixg_pitch(a.max_vis);
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t w = tid >> 6;
  float* p = lds + kGRing * kMixTile * 64 + w * pitch;  // this head's probabilities
  const uint32_t r = blockIdx.x;
  const uint32_t g = blockIdx.y;
  const uint32_t h = g * G + w;
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * 64;
  const int64_t v_off = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;
  const float* s = a.scratch + (static_cast<size_t>(r) * a.n_head + h) * a.max_vis;

  const float* vbase = reinterpret_cast<const float*>(a.kv) + v_off + g * 64;
  const RsrcWords rsrc =
      raw_buffer_words(vbase, static_cast<uint32_t>((static_cast<size_t>(n_vis - 1) * kv_row + 64) * 4));
  const uint32_t ring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(ring)));
  const uint32_t n_tiles = (n_vis + kMixTile - 1) / kMixTile;
  // This head's scores into its row of p (64 per copy), older than every V copy.
  const RsrcWords ssrc = raw_buffer_words(s, n_vis * 4);
  const uint32_t p_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(p)));
  for (uint32_t j0 = 0; j0 < n_vis; j0 += 64) lds_dma4(ssrc, 4 * (j0 + lane), p_lds + 4 * j0);
  // Copy k (0..7) of tile t moves rows t*32 + 4k .. t*32 + 4k + 3; wave w issues k = w, w + G, ...
  // A tile wholly below n_vis takes this lane's fixed offsets plus a uniform tile offset;
  // others (the last tile, and the copies past it that keep the wait counts uniform) clamp each
  // row to the last one.
  const uint32_t row_bytes = static_cast<uint32_t>(kv_row * 4);
  uint32_t lane_off[kOps];
#pragma unroll
  for (uint32_t i = 0; i < kOps; ++i) lane_off[i] = (4 * (w + i * G) + lane / 16) * row_bytes + (lane % 16) * 16;
  auto copy_tile = [&](uint32_t t) {
    const uint32_t dst = ring_lds + (t % kGRing) * kMixTile * 64 * 4;
    if ((t + 1) * kMixTile <= n_vis) {
#pragma unroll
      for (uint32_t i = 0; i < kOps; ++i) {
        lds_dma16_so(rsrc, lane_off[i], t * kMixTile * row_bytes, dst + 4 * (w + i * G) * 64 * 4);
      }
    } else {
#pragma unroll
      for (uint32_t i = 0; i < kOps; ++i) {
        const uint32_t k = w + i * G;
        const uint32_t row = min(t * kMixTile + 4 * k + lane / 16, n_vis - 1);
        lds_dma16(rsrc, row * row_bytes + (lane % 16) * 16, dst + 4 * k * 64 * 4);
      }
    }
  };
  for (uint32_t t = 0; t < kGRing; ++t) copy_tile(t);

  // Softmax of this head in p (the fused kernel's operations and double-sum tree).
  wait_vm<kGRing * kOps>();
  float m = -INFINITY;
  for (uint32_t j = lane; j < n_vis; j += 64) m = fmaxf(m, p[j]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  double part[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    for (uint32_t j = lane + 64 * q; j < n_vis; j += 256) {
      const float e = exp_libm(p[j] - m);
      p[j] = e;
      part[q] += static_cast<double>(e);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part[q] += __shfl_xor(part[q], off, 64);
  }
  double sum = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) sum += part[q];
  const float inv = static_cast<float>(1.0 / sum);
  for (uint32_t j = lane; j < n_vis; j += 64) p[j] = p[j] * inv;

  // Value mix, positions in order; tile t + 1 is read from LDS while tile t is mixed from
  // registers. A slot is refilled once every wave has read it.
  float acc = 0.0f;
  float va[kMixTile], pa[kMixTile], vb[kMixTile], pb[kMixTile];
  auto load_tile = [&](uint32_t t, float (&v)[kMixTile], float (&pp)[kMixTile]) {
    const float* vt = ring + (t % kGRing) * kMixTile * 64;
    const float* pt = p + t * kMixTile;
#pragma unroll
    for (uint32_t i = 0; i < kMixTile; ++i) v[i] = vt[i * 64 + lane];
#pragma unroll
    for (uint32_t i = 0; i < kMixTile; i += 4) {
      const float4 q4 = *reinterpret_cast<const float4*>(pt + i);
      pp[i] = q4.x;
      pp[i + 1] = q4.y;
      pp[i + 2] = q4.z;
      pp[i + 3] = q4.w;
    }
  };
  auto mix_tile = [&](const float (&v)[kMixTile], const float (&pp)[kMixTile], uint32_t t) {
    const uint32_t cnt = min(kMixTile, n_vis - t * kMixTile);
    if (cnt == kMixTile) {
#pragma unroll
      for (uint32_t i = 0; i < kMixTile; ++i) acc += pp[i] * v[i];
    } else {
      for (uint32_t i = 0; i < cnt; ++i) acc += pp[i] * v[i];
    }
  };
  auto step = [&](uint32_t t, float (&v)[kMixTile], float (&pp)[kMixTile], float (&vn)[kMixTile],
                  float (&pn)[kMixTile]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();  // every wave has tile t in registers: its slot takes tile t + kGRing
    copy_tile(t + kGRing);
    if (t + 1 < n_tiles) {
      wait_vm<(kGRing - 1) * kOps>();  // this wave's copies of tile t + 1 landed
      __syncthreads();                 // everyone's
      load_tile(t + 1, vn, pn);
    }
    mix_tile(v, pp, t);
  };
  wait_vm<(kGRing - 1) * kOps>();
  __syncthreads();
  load_tile(0, va, pa);
  for (uint32_t t = 0; t < n_tiles; t += 2) {
    step(t, va, pa, vb, pb);
    if (t + 1 < n_tiles) step(t + 1, vb, pb, va, pa);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy outlives the workgroup
  const size_t col = static_cast<size_t>(h) * 64 + lane;
  a.out[static_cast<size_t>(r) * a.out_stride + col] = acc;
  if (a.outq != nullptr) {
    const size_t nbq = a.out_stride / kQK;
    quantize_block_lanes(acc, lane & 31u, a.outq + (static_cast<size_t>(r) * nbq + col / kQK) * kBytesQ8_0);
  }
}

// One workgroup per (row, kv head, 32-dim half of the head), for decode rows of an fp32 cache
// with 64-dim heads. Against attn_mixg_kernel it changes where the work runs, not the float
// operations or their order:
//   - V streams through a deep LDS ring (up to 96 KB) filled by LDS-DMA, only the half of each
//     V row this workgroup mixes (128 bytes). A copy moves 8 positions (64 lanes x 16 bytes), a
//     tile is 4 copies (32 positions), issued by the first min(G, 4) waves. Only tiles below
//     n_vis are copied; the waits count the copies actually issued.
//   - Two waves per head run the softmax: wave (head, s) holds the double partial sums
//     part[2s] and part[2s + 1] of the fixed tree (part[q] takes positions lane + 64 q + 256 k,
//     k ascending), on registers, and the head's max and sum meet in LDS. The sum is
//     part[0] + part[1] + part[2] + part[3] in that order, as everywhere else.
//   - The chains run on ceil(G / 2) waves, wave c holding heads 2c (lanes 0..31) and 2c + 1
//     (lanes 32..63) of one dim each, so one LDS read of a V value serves two heads. They run
//     over half a ring at a time between one wait and two barriers, and form the 32 products of
//     tile t + 1 while they add those of tile t (each product rounds to float before its add,
//     so the bits are those of acc += p * v).
constexpr uint32_t kDTile = 32;                // positions per tile (4 KB)
// Rows of p hold whole 64-position copies; 4 more floats put the two heads a chain wave reads
// in different LDS banks.
__host__ __device__ inline uint32_t mixd_pitch(uint32_t max_vis) { return ((max_vis + 63) & ~63u) + 4; }
constexpr uint32_t kSPer = kMixMaxVis / 256;   // positions per lane per partial sum

// F16: the cache holds fp16 bit patterns, so a V half-row is 64 bytes and a tile two copies.
template <int G, bool F16>
struct MixD {
  static constexpr uint32_t kCopies = F16 ? 2 : 4;            // 1 KB copies per tile
  static constexpr uint32_t kTileBytes = kDTile * (F16 ? 64 : 128);
  static constexpr uint32_t kCw = G < kCopies ? G : kCopies;  // copying waves
  static constexpr uint32_t kCmax = (kCopies + kCw - 1) / kCw;  // most copies per wave per tile
  // LDS beside p: with G <= 4 two workgroups share a CU (half the LDS each), so a batch of
  // rows runs in one wave of workgroups; larger groups take a whole CU's LDS.
  static constexpr uint32_t kBudget = (G <= 4 ? 81920 : 163840) - G * (kMixMaxVis + 4) * 4 - 512;
  static constexpr uint32_t kR0 = (kBudget < 98304 ? kBudget : 98304) / kTileBytes;
  // Tiles in flight, even (two halves). A wave holds at most kMixMaxVis / 128 score copies and
  // kRing * kCmax V copies outstanding, within the 63 that vmcnt counts (and the 31 that
  // wait_vm_upto waits on).
  static constexpr uint32_t kRing = (kR0 * kCmax > 27 ? 27 / kCmax : kR0) & ~1u;
};

template <int G, bool F16>
size_t mixd_lds(uint32_t max_vis) {
  return static_cast<size_t>(MixD<G, F16>::kRing) * MixD<G, F16>::kTileBytes +
         static_cast<size_t>(G) * mixd_pitch(max_vis) * 4 + 512;
}


template <int G, bool F16>
__global__ __launch_bounds__(G * 128) void attn_mixd_kernel(AttnArgs a) {
  using M = MixD<G, F16>;
  constexpr uint32_t kR = M::kRing;
  constexpr uint32_t kCw = M::kCw;
  constexpr uint32_t kH = kR / 2;
  static_assert(kR >= 4 && kR * M::kCmax <= 27, "ring depth");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* ring = lds;                                   // [kR][kDTile][32] float or fp16 elements
  float* pbase = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(lds) + kR * M::kTileBytes);  // [G][pitch]
  const uint32_t pitch = mixd_pitch(a.max_vis);
  float* red_m = pbase + G * pitch;                       // [G][2] maxima (64 bytes)
  double* red_s = reinterpret_cast<double*>(red_m + 16);  // [G][4] partial sums (256 bytes); the row at +320
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t w = tid >> 6;
  // Workgroups start in the order of their linear index (x fastest), and a chain's length is its
  // row's visible positions: the linear index is read as (rank, kv head, half) with rank 0 the
  // row of most positions, so the longest rows start first and the short ones fill in behind.
  const uint32_t lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t rank = lin / (gridDim.y * gridDim.z);
  const uint32_t g = (lin / gridDim.z) % gridDim.y;
  const uint32_t half = lin % gridDim.z;
  uint32_t r = gridDim.x - 1 - rank;  // without n_vis, row r sees n_past + r + 1 positions
  if (a.n_vis != nullptr) {
    // Row i's rank: the rows with more positions, or as many and a lower index, come before it.
    // The rows' lengths go through LDS (p's space, free until the scores are copied in).
    uint32_t* slot = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(red_m) + 320);
    int32_t* nv = reinterpret_cast<int32_t*>(pbase);
    for (uint32_t i = tid; i < gridDim.x; i += blockDim.x) nv[i] = a.n_vis[i];
    __syncthreads();
    for (uint32_t i = tid; i < gridDim.x; i += blockDim.x) {
      const int32_t ni = nv[i];
      uint32_t rk = 0;
      for (uint32_t j = 0; j < gridDim.x; ++j) {
        const int32_t nj = nv[j];
        rk += (nj > ni || (nj == ni && j < i)) ? 1u : 0u;
      }
      if (rk == rank) *slot = i;
    }
    __syncthreads();
    r = *slot;
  }
  const uint32_t n_vis = a.n_vis != nullptr ? static_cast<uint32_t>(a.n_vis[r]) : static_cast<uint32_t>(a.n_past) + r + 1;
  const size_t kv_row = static_cast<size_t>(a.n_kv) * 64;
  const int64_t v_off = (a.v_off != nullptr ? a.v_off[r] : 0) + a.v_off_c;

  // Softmax role: head sh, partial sums 2 ss and 2 ss + 1.
  const uint32_t sh = w >> 1, ss = w & 1u;
  float* p = pbase + sh * pitch;
  const float* s = a.scratch + (static_cast<size_t>(r) * a.n_head + g * G + sh) * a.max_vis;
  const uint32_t p_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(p)));
  const RsrcWords ssrc = raw_buffer_words(s, n_vis * 4);
  // This wave's score groups (64 positions each): j0 = 64 (2 ss + i % 2) + 256 (i / 2).
  for (uint32_t i = 0;; ++i) {
    const uint32_t j0 = 64 * (2 * ss + (i & 1u)) + 256 * (i >> 1);
    if (j0 >= n_vis) break;
    lds_dma4(ssrc, 4 * (j0 + lane), p_lds + 4 * j0);
  }

  constexpr uint32_t es = F16 ? 2 : 4;        // bytes per cache element
  constexpr uint32_t kCopies = M::kCopies;
  constexpr uint32_t kPerCopy = kDTile / kCopies;  // positions per 1 KB copy: 8, or 16 in fp16
  const uint8_t* vbase = static_cast<const uint8_t*>(a.kv) + (v_off + g * 64 + half * 32) * es;
  const RsrcWords rsrc =
      raw_buffer_words(vbase, static_cast<uint32_t>((static_cast<size_t>(n_vis - 1) * kv_row + 32) * es));
  const uint32_t ring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(ring)));
  const uint32_t n_tiles = (n_vis + kDTile - 1) / kDTile;
  // Copy k of a tile moves its positions kPerCopy k .. kPerCopy (k + 1) - 1 (lane / (64 /
  // kPerCopy) picks the position, the rest of the lane its 16 bytes of the half-row); wave
  // w < kCw issues k = w, w + kCw, ... A tile wholly below n_vis takes this lane's fixed offsets
  // plus a uniform tile offset; the last tile clamps each position to the last one.
  const uint32_t copies = w < kCw ? (kCopies - w + kCw - 1) / kCw : 0;  // this wave's copies per tile
  const uint32_t row_bytes = static_cast<uint32_t>(kv_row * es);
  const uint32_t lane_row = lane / (64 / kPerCopy), lane_byte = (lane % (64 / kPerCopy)) * 16;
  auto copy_tile = [&](uint32_t t) {
    if (t >= n_tiles) return;
    const uint32_t dst = ring_lds + (t % kR) * M::kTileBytes;
    const bool whole = (t + 1) * kDTile <= n_vis;
    for (uint32_t k = w; k < kCopies && w < kCw; k += kCw) {
      if (whole) {
        lds_dma16_so(rsrc, (kPerCopy * k + lane_row) * row_bytes + lane_byte, t * kDTile * row_bytes, dst + k * 1024);
      } else {
        const uint32_t row = min(t * kDTile + kPerCopy * k + lane_row, n_vis - 1);
        lds_dma16(rsrc, row * row_bytes + lane_byte, dst + k * 1024);
      }
    }
  };
  for (uint32_t t = 0; t < kR; ++t) copy_tile(t);
  // Waiting for tile u leaves the copies of the tiles issued after it outstanding.
  auto wait_tile = [&](uint32_t u, uint32_t issued) { wait_vm_upto(issued > u + 1 ? (issued - u - 1) * copies : 0); };

  // Softmax. x[2 k + i] holds position lane + 64 (2 ss + i) + 256 k; positions past n_vis hold
  // -inf, whose exponential adds an exact zero to the double sums.
  wait_vm_upto(min(n_tiles, kR) * copies);  // the scores, older than every V copy
  float x[2 * kSPer];
#pragma unroll
  for (uint32_t k = 0; k < kSPer; ++k) {
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
      const uint32_t j0 = 64 * (2 * ss + i) + 256 * k;
      if (j0 < n_vis) {
        const float v = p[j0 + lane];
        x[2 * k + i] = j0 + lane < n_vis ? v : -INFINITY;
      }
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (uint32_t k = 0; k < kSPer; ++k) {
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
      if (64 * (2 * ss + i) + 256 * k < n_vis) m = fmaxf(m, x[2 * k + i]);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) red_m[2 * sh + ss] = m;
  __syncthreads();
  m = fmaxf(red_m[2 * sh], red_m[2 * sh + 1]);
  double part[2] = {0.0, 0.0};
#pragma unroll
  for (uint32_t k = 0; k < kSPer; ++k) {
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
      if (64 * (2 * ss + i) + 256 * k < n_vis) {
        x[2 * k + i] = exp_libm(x[2 * k + i] - m);
        part[i] += static_cast<double>(x[2 * k + i]);
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    part[0] += __shfl_xor(part[0], off, 64);
    part[1] += __shfl_xor(part[1], off, 64);
  }
  if (lane == 0) {
    red_s[4 * sh + 2 * ss] = part[0];
    red_s[4 * sh + 2 * ss + 1] = part[1];
  }
  __syncthreads();
  double sum = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) sum += red_s[4 * sh + q];
  const float inv = static_cast<float>(1.0 / sum);
#pragma unroll
  for (uint32_t k = 0; k < kSPer; ++k) {
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
      const uint32_t j0 = 64 * (2 * ss + i) + 256 * k;
      if (j0 < n_vis) p[j0 + lane] = x[2 * k + i] * inv;
    }
  }

  // Value mix, positions in order, half a ring at a time.
  constexpr uint32_t kChains = (G + 1) / 2;  // chain waves
  const uint32_t d = lane & 31u;
  const uint32_t hl = 2 * w + (lane >> 5);  // this lane's head within the group
  const bool chain = w < kChains;
  const bool live = hl < G;
  const float* ph = pbase + (live ? hl : 2 * w) * pitch;  // its probabilities
  float acc = 0.0f;
  float va[kDTile], pa[kDTile], vb[kDTile], pb[kDTile];
  auto load_tile = [&](uint32_t t, float (&v)[kDTile], float (&pp)[kDTile]) {
    const float* pt = ph + t * kDTile;
    if constexpr (F16) {  // each value kept as its fp16 bits (the multiply widens it)
      const uint16_t* vt = reinterpret_cast<const uint16_t*>(ring) + (t % kR) * kDTile * 32 + d;
#pragma unroll
      for (uint32_t i = 0; i < kDTile; ++i) v[i] = __uint_as_float(vt[i * 32]);
    } else {
      const float* vt = ring + (t % kR) * kDTile * 32 + d;
#pragma unroll
      for (uint32_t i = 0; i < kDTile; ++i) v[i] = vt[i * 32];
    }
#pragma unroll
    for (uint32_t i = 0; i < kDTile; i += 4) {
      const float4 q4 = *reinterpret_cast<const float4*>(pt + i);
      pp[i] = q4.x;
      pp[i + 1] = q4.y;
      pp[i + 2] = q4.z;
      pp[i + 3] = q4.w;
    }
  };
  auto mul = [](float pv, float v) {
    if constexpr (F16) return mul_half_bits(pv, __float_as_uint(v));
    else return pv * v;
  };
  auto mul_tile = [&](float (&v)[kDTile], const float (&pp)[kDTile]) {
#pragma unroll
    for (uint32_t i = 0; i < kDTile; ++i) v[i] = mul(pp[i], v[i]);
  };
  auto add_tile = [&](const float (&prod)[kDTile], uint32_t t) {
    const uint32_t cnt = min(kDTile, n_vis - t * kDTile);
    if (cnt == kDTile) {
#pragma unroll
      for (uint32_t i = 0; i < kDTile; ++i) acc += prod[i];
    } else {
      for (uint32_t i = 0; i < cnt; ++i) acc += prod[i];
    }
  };
  // A whole tile's adds with the next tile's products between them: each product fills the
  // wait of one dependent add (written apart, the compiler emits the 32 adds, then the 32
  // multiplies).
  auto add_mul = [&](const float (&prod)[kDTile], float (&v)[kDTile], const float (&pp)[kDTile]) {
#pragma unroll
    for (uint32_t i = 0; i < kDTile; ++i) {
      acc += prod[i];
      v[i] = mul(pp[i], v[i]);
    }
  };
  uint32_t issued = min(n_tiles, kR);
  for (uint32_t t0 = 0; t0 < n_tiles; t0 += kH) {
    const uint32_t t1 = min(n_tiles, t0 + kH);
    wait_tile(t1 - 1, issued);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();  // everyone's copies of [t0, t1), and (first time) every p write
    if (chain) {
      // Tile t + 1 is read while tile t's products are added, and its products are formed
      // after them, so neither the LDS reads nor the multiplies stall the adds.
      // A tile followed by another in [t0, t1) is whole (t1 <= n_tiles).
      load_tile(t0, va, pa);
      mul_tile(va, pa);
      for (uint32_t t = t0; t < t1; t += 2) {
        if (t + 1 < t1) {
          load_tile(t + 1, vb, pb);
          add_mul(va, vb, pb);
          if (t + 2 < t1) {
            load_tile(t + 2, va, pa);
            add_mul(vb, va, pa);
          } else {
            add_tile(vb, t + 1);
          }
        } else {
          add_tile(va, t);
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();  // every wave is done with the half [t0, t1)
    for (uint32_t t = t0 + kR; t < t1 + kR; ++t) copy_tile(t);
    issued = min(n_tiles, t1 + kR);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy outlives the workgroup
  if (chain && live) {
    const size_t col = static_cast<size_t>(g * G + hl) * 64 + half * 32 + d;
    a.out[static_cast<size_t>(r) * a.out_stride + col] = acc;
    if (a.outq != nullptr) {
      const size_t nbq = a.out_stride / kQK;
      quantize_block_lanes(acc, d, a.outq + (static_cast<size_t>(r) * nbq + col / kQK) * kBytesQ8_0);
    }
  }
}

// Dynamic LDS above 64 KB must be granted per kernel; 0 when the device cannot.
template <int G, bool F16>
size_t mixd_lds_granted(uint32_t max_vis) {
  static int limit = -1;
  if (limit < 0) {
    int dev = 0, v = 0;
    limit = (hipGetDevice(&dev) == hipSuccess &&
             hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess)
                ? v
                : 65536;
    const int want = static_cast<int>(mixd_lds<G, F16>(kMixMaxVis));
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(attn_mixd_kernel<G, F16>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, std::min(want, limit)) != hipSuccess)
      limit = 65536;
  }
  const size_t need = mixd_lds<G, F16>(max_vis);
  return need <= static_cast<size_t>(limit) ? need : 0;
}

// The mix kernel's granted LDS for a group size (3, 4, 7, 8), 0 when it has none or none fits.
template <bool F16>
size_t mixd_grant_for(uint32_t group, uint32_t max_vis) {
  switch (group) {
  case 3: return mixd_lds_granted<3, F16>(max_vis);
  case 4: return mixd_lds_granted<4, F16>(max_vis);
  case 7: return mixd_lds_granted<7, F16>(max_vis);
  case 8: return mixd_lds_granted<8, F16>(max_vis);
  default: return 0;
  }
}

template <bool F16>
void launch_mixd(uint32_t group, dim3 grid, size_t lds, const AttnArgs& a) {
  switch (group) {
  case 3: hipLaunchKernelGGL((attn_mixd_kernel<3, F16>), grid, dim3(384), lds, stream(), a); break;
  case 4: hipLaunchKernelGGL((attn_mixd_kernel<4, F16>), grid, dim3(512), lds, stream(), a); break;
  case 7: hipLaunchKernelGGL((attn_mixd_kernel<7, F16>), grid, dim3(896), lds, stream(), a); break;
  case 8: hipLaunchKernelGGL((attn_mixd_kernel<8, F16>), grid, dim3(1024), lds, stream(), a); break;
  default: break;
  }
}

bool scores_fit_lds(const AttnArgs& a) {
  const uint32_t group = a.n_head / a.n_kv;
  return static_cast<size_t>(group) * (a.head_dim + round4(a.max_vis)) * 4 + vtile_bytes(a.head_dim) <= 65536;
}

}  // namespace

// Decode-shaped launches (few rows, every head) take the two-kernel path when its LDS fits.
bool use_split(const AttnArgs& a, uint32_t n_rows) {
  const uint32_t group = a.n_head / a.n_kv;
  const size_t lds = (static_cast<size_t>(group) * score_pitch(a.max_vis) + 2 * kTileFloats) * 4;
  return a.split && a.head_begin == 0 && a.head_end == a.n_head && static_cast<size_t>(n_rows) * a.n_kv < 512 &&
         lds <= 65536 && group * 32 <= kThreads && a.head_dim % 32 == 0;
}

size_t attention_scratch_floats(const AttnArgs& a, uint32_t n_rows) {
  if (scores_fit_lds(a) && !use_split(a, n_rows)) return 0;
  return static_cast<size_t>(n_rows) * a.n_head * a.max_vis;
}

int attention_launch(const AttnArgs& a, uint32_t n_rows) {
  if (n_rows == 0) return kOk;
  if (a.n_kv == 0 || a.n_head % a.n_kv != 0)
    return fail(kInvalidArgument, "attention: %u heads over %u kv heads", a.n_head, a.n_kv);
  if (a.head_begin > a.head_end || a.head_end > a.n_head)
    return fail(kInvalidArgument, "attention: heads [%u, %u) of %u", a.head_begin, a.head_end, a.n_head);
  if (a.head_begin == a.head_end) return kOk;
  const uint32_t group = a.n_head / a.n_kv;
  if (a.scratch != nullptr && use_split(a, n_rows) && a.head_dim == 64 && group <= 16 && a.max_vis <= kMixMaxVis) {
    // The mix kernel for this group, if its LDS is granted; an fp16 cache without one takes
    // the split kernels below.
    const size_t dlds = a.f16 ? mixd_grant_for<true>(group, a.max_vis) : mixd_grant_for<false>(group, a.max_vis);
    if (!a.f16 || dlds != 0) {
      const dim3 sgrid(n_rows, a.n_kv, (a.max_vis + 63) / 64);
      const dim3 dgrid(n_rows, a.n_kv, 2);
      if (a.f16) {
        const size_t slds = scores64_lds(true, group);
        hipLaunchKernelGGL(attn_scores64_kernel<true>, sgrid, dim3(group * 64), slds, stream(), a);
        launch_mixd<true>(group, dgrid, dlds, a);
        return check_launch("attention (decode, fp16)");
      }
      const size_t slds = scores64_lds(false, group);
      hipLaunchKernelGGL(attn_scores64_kernel<false>, sgrid, dim3(group * 64), slds, stream(), a);
      const size_t glds = mixg_lds(group, a.max_vis);
      const dim3 ggrid(n_rows, a.n_kv);
      if (dlds != 0) {
        launch_mixd<false>(group, dgrid, dlds, a);
      } else if (glds <= 65536 && (group == 1 || group == 2 || group == 4 || group == 8)) {
        if (group == 1) hipLaunchKernelGGL(attn_mixg_kernel<1>, ggrid, dim3(64), glds, stream(), a);
        if (group == 2) hipLaunchKernelGGL(attn_mixg_kernel<2>, ggrid, dim3(128), glds, stream(), a);
        if (group == 4) hipLaunchKernelGGL(attn_mixg_kernel<4>, ggrid, dim3(256), glds, stream(), a);
        if (group == 8) hipLaunchKernelGGL(attn_mixg_kernel<8>, ggrid, dim3(512), glds, stream(), a);
      } else {
        hipLaunchKernelGGL(attn_mix64_kernel, dim3(n_rows, a.n_head), dim3(64), 0, stream(), a);
      }
      return check_launch("attention (decode)");
    }
  }
  if (a.scratch != nullptr && use_split(a, n_rows)) {
    const dim3 sgrid(n_rows, a.n_kv, (a.max_vis + kThreads - 1) / kThreads);
    const size_t slds = static_cast<size_t>(group) * a.head_dim * 4;
    const size_t mlds = (static_cast<size_t>(group) * score_pitch(a.max_vis) + 2 * kTileFloats) * 4;
    // Quantized output: 32-dim slices (whole Q8_0 blocks); float output: 8-dim slices.
    const bool q = a.outq != nullptr;
    const dim3 mgrid(n_rows, a.n_kv, a.head_dim / (q ? 32 : 8));
    if (a.f16) {
      hipLaunchKernelGGL(attn_scores_kernel<true>, sgrid, dim3(kThreads), slds, stream(), a);
      if (q) hipLaunchKernelGGL((attn_mix_kernel<true, 32>), mgrid, dim3(kThreads), mlds, stream(), a);
      else hipLaunchKernelGGL((attn_mix_kernel<true, 8>), mgrid, dim3(kThreads), mlds, stream(), a);
    } else {
      hipLaunchKernelGGL(attn_scores_kernel<false>, sgrid, dim3(kThreads), slds, stream(), a);
      if (q) hipLaunchKernelGGL((attn_mix_kernel<false, 32>), mgrid, dim3(kThreads), mlds, stream(), a);
      else hipLaunchKernelGGL((attn_mix_kernel<false, 8>), mgrid, dim3(kThreads), mlds, stream(), a);
    }
    return check_launch("attention (split)");
  }
  if (scores_fit_lds(a) && launch_block(a, n_rows)) return check_launch("attention (blocked rows)");
  if (a.outq != nullptr && a.head_dim % kQK != 0) {
    // The fused kernel quantizes whole 32-dim blocks only: quantize its output rows afterwards.
    AttnArgs b = a;
    b.outq = nullptr;
    const int rc = attention_launch(b, n_rows);
    if (rc != kOk) return rc;
    return quantize_rows_launch(a.out, a.outq, a.n_head * a.head_dim, n_rows, a.out_stride);
  }
  const dim3 grid(n_rows, a.n_kv);
  const bool lds_ok = scores_fit_lds(a);
  if (!lds_ok && a.scratch == nullptr) return fail(kInvalidArgument, "attention: %u positions need a score scratch", a.max_vis);
  if (!lds_ok && !a.split && a.head_end - a.head_begin > 1) {
    // A table call (src/kernels/kernels.h:67-75) brings scratch for one head's scores,
    // n_q * (n_past + n_q) floats: its heads run one launch each, in stream order, each
    // reusing that scratch.
    for (uint32_t h = a.head_begin; h < a.head_end; ++h) {
      AttnArgs b = a;
      b.head_begin = h;
      b.head_end = h + 1;
      const int rc = attention_launch(b, n_rows);
      if (rc != kOk) return rc;
    }
    return kOk;
  }
  const size_t tile = a.head_dim <= 128 ? vtile_bytes(a.head_dim) : 0;
  const size_t lds = (lds_ok ? static_cast<size_t>(group) * (a.head_dim + round4(a.max_vis)) * 4
                             : static_cast<size_t>(group) * a.head_dim * 4) + tile;
  if (lds > 65536) return fail(kUnsupported, "attention: %zu bytes of LDS", lds);
  if (a.f16) {
    if (lds_ok) hipLaunchKernelGGL((attention_kernel<true, false>), grid, dim3(kThreads), lds, stream(), a);
    else hipLaunchKernelGGL((attention_kernel<true, true>), grid, dim3(kThreads), lds, stream(), a);
  } else {
    if (lds_ok) hipLaunchKernelGGL((attention_kernel<false, false>), grid, dim3(kThreads), lds, stream(), a);
    else hipLaunchKernelGGL((attention_kernel<false, true>), grid, dim3(kThreads), lds, stream(), a);
  }
  return check_launch("attention");
}

}  // namespace axon_hip
