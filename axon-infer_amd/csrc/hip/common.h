// Device-side building blocks shared by every kernel of the hip table: the GGUF block formats,
// exact half/bfloat conversions, LDS staging of unaligned block streams, and the launch
// plumbing (the library stream, status codes, the thread-local error message).
//
// All code here is gfx950 (CDNA4) only: 64-lane wavefronts, 160 KB of LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstddef>
#include <cstdint>

namespace axon_hip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kQK = 32;     // elements per Q8_0 / Q4_0 / Q4_1 block
constexpr int kQKK = 256;   // elements per Q6_K super-block
constexpr int kBytesQ8_0 = 34;
constexpr int kBytesQ4_0 = 18;
constexpr int kBytesQ4_1 = 20;
constexpr int kBytesQ6_K = 210;

// ggml type ids (GGUF tensor types), the subset the table handles.
enum DType : int { F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q8_0 = 8, Q6_K = 14, BF16 = 30 };

// Status codes returned across the C ABI.
enum Status : int {
  kOk = 0,
  kInvalidArgument = -1,
  kUnsupported = -2,
  kNoDevice = -3,
  kHipError = -4,
  kOutOfMemory = -5,
};

// ------------------------------------------------------------------------------------------
// Exact conversions (IEEE binary16 / bfloat16 <-> binary32), written with integer operations
// so that NaN payloads, signed zeros and subnormals come out bit for bit as the scalar table
// produces them (trickymind1324/axon-infer src/core/dtype.cpp:198-272).

// The hardware conversion is exact for every finite half (subnormals included: half denormals
// are on); infinities and NaNs take the bit-level form so NaN payloads pass through unchanged.
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  const uint32_t f = __float_as_uint(static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h))));
  const uint32_t special = ((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13);
  // A select by mask, so the conversion stays one basic block (a branch here splits every loop
  // that widens a block scale and stops the scheduler from overlapping its LDS reads).
  const uint32_t m = 0u - static_cast<uint32_t>(((h >> 10) & 0x1fu) == 0x1fu);
  return __uint_as_float((f & ~m) | (special & m));
}

// fp16 bits to float by the hardware conversion, for values read into arithmetic: exact for
// every finite value (fp16 denormals are kept: the kernels' FP16/FP64 denormal mode) and for
// infinities; a NaN converts to a NaN (its payload may differ from half_bits_to_float's).
__device__ __forceinline__ float half_value(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// p * half_value(h) for the fp16 bits h in the low half of hb, rounded once as that product of
// two floats is: v_fma_mix_f32 widens h exactly (fp16 denormals kept) and forms p * h + (-0),
// and adding -0 leaves every product as it is, -0 included. One instruction in place of the
// conversion and the multiply.
__device__ __forceinline__ float mul_half_bits(float p, uint32_t hb) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(p), "v"(hb), "v"(-0.0f));
  return r;
}

// The same for the fp16 bits in the high half of hb.
__device__ __forceinline__ float mul_half_bits_hi(float p, uint32_t hb) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(p), "v"(hb), "v"(-0.0f));
  return r;
}

// Round to nearest even, overflow to infinity, gradual underflow, NaN kept non-zero.
__device__ __forceinline__ uint32_t float_to_half_bits(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t e = (x >> 23) & 0xffu;
  const uint32_t m = x & 0x7fffffu;
  if (e == 0xffu) {
    const uint32_t payload = m >> 13;
    return sign | 0x7c00u | (m != 0 && payload == 0 ? 1u : payload);
  }
  const int ue = static_cast<int>(e) - 127;
  if (ue > 15) return sign | 0x7c00u;
  if (ue >= -14) {
    // The carry of a mantissa round-up walks into the exponent, up to infinity (0x7c00).
    uint32_t r = (static_cast<uint32_t>(ue + 15) << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) ++r;
    return sign | r;
  }
  if (ue >= -25) {
    const uint32_t full = m | 0x800000u;
    const uint32_t shift = static_cast<uint32_t>(-1 - ue);  // 14 .. 24
    uint32_t hm = full >> shift;
    const uint32_t rest = full & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rest > halfway || (rest == halfway && (hm & 1u))) ++hm;
    return sign | hm;
  }
  return sign;
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t h) { return __uint_as_float(h << 16); }

// The binary32 exponential of the host C library the scalar table runs on (std::exp(float) in
// the reference's softmax and SiLU, src/kernels/ref/softmax.cpp:18, silu.cpp:11): glibc 2.35's
// expf, the published ARM optimized-routines method (Szabolcs Nagy, 2017). It is not correctly
// rounded (it differs from the once-rounded binary64 exp on about 1 in 10^4 arguments near 0), so
// bit parity needs its steps, restated here: with N = 32, k = round(x N / ln 2) and
// r = x N / ln 2 - k (one fused multiply-add), exp(x) = 2^(k/N) (1 + C2 r + C1 r^2 + C0 r^3) in
// binary64, rounded once to binary32. 2^(k/N) is kExp2Tab[k mod N] with k/N added to its exponent
// field; entry i is 2^(i/N) rounded to binary64, less i << 47 (so that adding k << 47 carries
// the whole of k/N into the exponent). Checked against the host's expf on every binary32
// argument of the main range (x in (-103.97, 88.72), 2.24e9 values): identical. Outside it
// expf is 0 (underflow), +inf (overflow) or NaN (x + x).
__device__ const uint64_t kExp2Tab[32] = {
  0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
  0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
  0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
  0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
  0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
  0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
  0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
  0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// exp_libm with the table read from `tab` (kExp2Tab, or a copy of it in LDS).
__device__ __forceinline__ float exp_libm_from(float x, const uint64_t* tab) {
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;  // N / ln 2
  constexpr double kShift = 0x1.8p+52;                    // adds and strips to round to an integer
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
  if (x != x) return x + x;
  if (x > 0x1.62e42ep6f) return __builtin_inff();
  if (x < -0x1.9fe368p6f) return 0.0f;
  const double xd = static_cast<double>(x);
  double kd = kInvLn2N * xd + kShift;
  const uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
  kd -= kShift;
  const double r = fma(kInvLn2N, xd, -kd);
  const double s = __longlong_as_double(static_cast<long long>(tab[ki & 31u] + (ki << 47)));
  const double p = kC0 * r + kC1;
  const double r2 = r * r;
  double y = kC2 * r + 1.0;
  y = p * r2 + y;
  return static_cast<float>(y * s);
}

__device__ __forceinline__ float exp_libm(float x) { return exp_libm_from(x, kExp2Tab); }

// ------------------------------------------------------------------------------------------
// Byte streams in LDS. GGUF blocks are 18, 20, 34 or 210 bytes, so a block starts on a 2-byte
// boundary at best. Tiles are copied HBM -> LDS with the widest aligned loads the tile allows
// (coalesced across the workgroup), and blocks are then read out of LDS as aligned dwords and
// funnel-shifted into place.

// Copies nbytes (a multiple of 2) from global src to LDS dst (2-byte aligned), using 16-, 4-
// or 2-byte accesses, whichever the alignment of src, dst and nbytes permits. Each thread issues up
// to eight loads before its first LDS store, so a whole tile is in flight at once. Every
// thread of the block must call it; it does not synchronise.
template <typename T>
__device__ __forceinline__ void stage_units(const T* __restrict__ s, T* d, uint32_t n, uint32_t tid,
                                            uint32_t nthreads) {
  for (uint32_t base = tid; base < n; base += 8 * nthreads) {
    T v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t i = base + k * nthreads;
      if (i < n) v[k] = __builtin_nontemporal_load(s + i);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t i = base + k * nthreads;
      if (i < n) d[i] = v[k];
    }
  }
}

__device__ __forceinline__ void stage_bytes(const uint8_t* __restrict__ src, uint8_t* dst,
                                            uint32_t nbytes, uint32_t tid, uint32_t nthreads) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst);
  if (((a | nbytes) & 15u) == 0) {
    stage_units(reinterpret_cast<const u32x4*>(src), reinterpret_cast<u32x4*>(dst), nbytes >> 4, tid, nthreads);
  } else if (((a | nbytes) & 3u) == 0) {
    stage_units(reinterpret_cast<const uint32_t*>(src), reinterpret_cast<uint32_t*>(dst), nbytes >> 2, tid, nthreads);
  } else {
    stage_units(reinterpret_cast<const uint16_t*>(src), reinterpret_cast<uint16_t*>(dst), nbytes >> 1, tid, nthreads);
  }
}

// Copies n_rows rows of row_bytes each from global src (rows src_pitch bytes apart) to LDS
// dst (rows dst_pitch bytes apart), with 4-byte accesses when src, src_pitch, dst_pitch and
// row_bytes allow it and 2-byte accesses otherwise, eight loads in flight per thread. Does not
// synchronise.
template <typename T>
__device__ __forceinline__ void stage_rows_units(const uint8_t* __restrict__ src, size_t src_pitch, uint8_t* dst,
                                                 uint32_t dst_pitch, uint32_t n_rows, uint32_t per_row,
                                                 uint32_t tid, uint32_t nthreads) {
  const uint32_t n = per_row * n_rows;
  for (uint32_t base = tid; base < n; base += 8 * nthreads) {
    T v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t j = base + k * nthreads;
      if (j < n) {
        const uint32_t r = j / per_row;
        v[k] = __builtin_nontemporal_load(reinterpret_cast<const T*>(src + r * src_pitch) + (j - r * per_row));
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t j = base + k * nthreads;
      if (j < n) {
        const uint32_t r = j / per_row;
        reinterpret_cast<T*>(dst + r * dst_pitch)[j - r * per_row] = v[k];
      }
    }
  }
}

__device__ __forceinline__ void stage_rows(const uint8_t* __restrict__ src, size_t src_pitch, uint8_t* dst,
                                           uint32_t dst_pitch, uint32_t n_rows, uint32_t row_bytes,
                                           uint32_t tid, uint32_t nthreads) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(src);
  if (((a | src_pitch | dst_pitch | row_bytes) & 3u) == 0) {
    stage_rows_units<uint32_t>(src, src_pitch, dst, dst_pitch, n_rows, row_bytes >> 2, tid, nthreads);
  } else {
    stage_rows_units<uint16_t>(src, src_pitch, dst, dst_pitch, n_rows, row_bytes >> 1, tid, nthreads);
  }
}

// Reads N consecutive dwords starting at LDS byte offset `off` (2-byte aligned).
template <int N>
__device__ __forceinline__ void lds_read_unaligned(const uint8_t* lds, uint32_t off, uint32_t (&out)[N]) {
  const uint32_t* base = reinterpret_cast<const uint32_t*>(lds + (off & ~3u));
  const uint32_t shift = (off & 3u) * 8u;
  uint32_t w[N + 1];
#pragma unroll
  for (int i = 0; i <= N; ++i) w[i] = base[i];
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], shift);
}

// Q8_0 activation block as staged in LDS: 32 int8 quants in 8 dwords, the scale widened to
// float, and the sum of the quants (the Q4_0 offset and Q4_1 minimum terms need it).
struct __attribute__((aligned(8))) ActBlock {
  int32_t qs[8];
  float d;
  int32_t sum;
};

// Converts the raw Q8_0 block at LDS byte offset `off` into an ActBlock.
__device__ __forceinline__ ActBlock unpack_q8_0_lds(const uint8_t* lds, uint32_t off) {
  uint32_t w[9];
  lds_read_unaligned<9>(lds, off, w);
  ActBlock a;
  a.d = half_bits_to_float(w[0] & 0xffffu);
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a.qs[i] = static_cast<int32_t>(__builtin_amdgcn_alignbit(w[i + 1], w[i], 16));
    s = __builtin_amdgcn_sdot4(a.qs[i], 0x01010101, s, false);
  }
  a.sum = s;
  return a;
}

// Signed dot of 8 dwords of int8 against 8 dwords of int8.
__device__ __forceinline__ int32_t dot32(const int32_t (&a)[8], const int32_t (&b)[8]) {
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) s = __builtin_amdgcn_sdot4(a[i], b[i], s, false);
  return s;
}

// Q8_0 quantization of one 32-element block held one element per lane in a 32-lane half-wave
// (src/core/dtype.cpp:338-354): amax, d = amax / 127 (IEEE division), id = 1 / d or 0,
// fp16(d), q = int8(roundf(x * id)), ties away from zero. `lane` is 0..31 within the half.
__device__ __forceinline__ void quantize_block_lanes(float x, uint32_t lane, uint8_t* block) {
  float amax = fabsf(x);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const int32_t q = static_cast<int32_t>(roundf(x * id));
  const int32_t q_next = __shfl_down(q, 1, 32);
  if (lane == 0) *reinterpret_cast<uint16_t*>(block) = static_cast<uint16_t>(float_to_half_bits(d));
  if ((lane & 1) == 0) {
    *reinterpret_cast<uint16_t*>(block + 2 + lane) =
        static_cast<uint16_t>((q & 0xff) | ((q_next & 0xff) << 8));
  }
}

// ------------------------------------------------------------------------------------------
// Greedy selection keys: (value, index) packed so that the largest key is the first maximum
// (std::ranges::max_element): the value's bits mapped to an unsigned order (-0 as +0) above the
// complemented index. Key 0 stands for "no value" (NaN is never a key).
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0;  // -0 == +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(~i);
}

__device__ __forceinline__ uint64_t max_key_wave(uint64_t k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(k, off, 64);
    k = o > k ? o : k;
  }
  return k;
}

// ------------------------------------------------------------------------------------------
// Whole-row work for one 256-thread workgroup, shared by the standalone kernels and the fused
// matvec's prologue, so that both produce the same bits.

// Sum over the 256 threads of a workgroup in a fixed order: the wave butterfly, then the four
// waves in order. red: 4 doubles of LDS. Every thread gets the sum.
__device__ __forceinline__ double block_sum_double_256(double v, double* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int w = 0; w < 4; ++w) s += red[w];
  __syncthreads();
  return s;
}

// Quantizes the 8 consecutive floats v of this thread, one quarter of a 32-element block whose
// other quarters sit in the 3 adjacent lanes (part = lane & 3), as quantize_row_q8_0 does: the
// thread's 8 quants go to blk + 2 + 8 * part, part 0 also writes the fp16 scale. active:
// whether this thread's elements exist (the shuffles still need every lane).
__device__ __forceinline__ void quantize8_store(const float (&v)[8], bool active, uint8_t* blk, uint32_t part) {
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  if (!active) return;
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint32_t q[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) q[k] = static_cast<uint32_t>(static_cast<int32_t>(roundf(v[k] * id))) & 0xffu;
  if (part == 0) *reinterpret_cast<uint16_t*>(blk) = static_cast<uint16_t>(float_to_half_bits(d));
  uint16_t* qs = reinterpret_cast<uint16_t*>(blk + 2 + 8 * part);
#pragma unroll
  for (int k = 0; k < 4; ++k) qs[k] = static_cast<uint16_t>(q[2 * k] | (q[2 * k + 1] << 8));
}

// rmsnorm (src/kernels/ref/rmsnorm.cpp:10-21) of one row of n <= 2048 floats (n % 32 == 0;
// x, w, y 16-byte aligned) by a 256-thread workgroup: thread t holds elements 8t..8t+7 in
// registers; y = x * inv * w (or not stored when y is null) and its Q8_0 blocks into yq (or
// not when null).
__device__ __forceinline__ void rmsnorm_row_256(const float* xr, const float* w, float* yr, uint8_t* yq, uint32_t n,
                                                float eps, double* red) {
  const uint32_t e0 = threadIdx.x * 8;
  const bool has = e0 < n;
  float xv[8], wv[8];
  if (has) {
    const float4 a = *reinterpret_cast<const float4*>(xr + e0);
    const float4 b = *reinterpret_cast<const float4*>(xr + e0 + 4);
    const float4 c = *reinterpret_cast<const float4*>(w + e0);
    const float4 d = *reinterpret_cast<const float4*>(w + e0 + 4);
    xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w; xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    wv[0] = c.x; wv[1] = c.y; wv[2] = c.z; wv[3] = c.w; wv[4] = d.x; wv[5] = d.y; wv[6] = d.z; wv[7] = d.w;
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) xv[k] = wv[k] = 0.0f;
  }
  double ss = 0.0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const double v = static_cast<double>(xv[k]);
    ss += v * v;
  }
  ss = block_sum_double_256(ss, red);
  const float inv = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(n) + static_cast<double>(eps)));
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = xv[k] * inv * wv[k];
  if (yr != nullptr && has) {
    *reinterpret_cast<float4*>(yr + e0) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(yr + e0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
  if (yq != nullptr) quantize8_store(v, has, yq + (e0 / kQK) * kBytesQ8_0, threadIdx.x & 3);
}

// ------------------------------------------------------------------------------------------
// LDS-DMA: global memory straight into LDS without passing through registers.

using LdsPtr = __attribute__((address_space(3))) void*;
// A generic pointer into a __shared__ object as an LDS address.
__device__ __forceinline__ LdsPtr as_lds(const void* p) { return (LdsPtr)(const_cast<void*>(p)); }
constexpr uint32_t kRawBufferWord3 = 0x00020000u;  // gfx9 raw buffer descriptor: 32-bit data

// Copies `bytes` from global src to LDS dst with buffer loads that write LDS directly: 16-byte
// units when src, dst and bytes are multiples of 16, else 4-byte units (all three must be
// multiples of 4). Threads [0, nthreads) of the block take part in whole waves (tid and
// nthreads multiples of 64 at wave starts). The copies complete asynchronously: s_waitcnt
// vmcnt(0) on every copying wave, then a barrier, before anyone reads dst.
__device__ __forceinline__ void dma_to_lds(const uint8_t* src, uint8_t* dst, uint32_t bytes, uint32_t tid,
                                           uint32_t nthreads) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(src), 0, static_cast<int>(bytes), static_cast<int>(kRawBufferWord3));
  const uint32_t lane = tid & 63u;
  const uint32_t wave0 = tid & ~63u;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | bytes) & 15u) == 0) {
    const uint32_t units = bytes >> 4;
    for (uint32_t base = wave0; base < units; base += nthreads) {
      if (base + lane < units) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, as_lds(dst + base * 16u), 16, (base + lane) * 16u, 0, 0, 0);
      }
    }
  } else {
    const uint32_t units = bytes >> 2;
    for (uint32_t base = wave0; base < units; base += nthreads) {
      if (base + lane < units) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, as_lds(dst + base * 4u), 4, (base + lane) * 4u, 0, 0, 0);
      }
    }
  }
}

// LDS-DMA from inline assembly. The compiler does not count these copies, so a kernel that
// uses them waits for them itself (wait_vm, wait_vm_upto): vmcnt drains in issue order, so a
// load issued before the copies can be waited for while the copies stay in flight, which the
// compiler's own counting (that sees the copies) cannot express.
typedef int RsrcWords __attribute__((ext_vector_type(4)));

// A raw buffer descriptor of `bytes` from base, in scalar registers (every lane holds the same
// words).
__device__ __forceinline__ RsrcWords raw_buffer_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  RsrcWords w;
  w.x = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  w.y = __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu));  // stride 0
  w.z = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  w.w = static_cast<int>(kRawBufferWord3);
  return w;
}

// 4 bytes per lane from rsrc + voffset to LDS at lds + 4 * lane (lds uniform).
__device__ __forceinline__ void lds_dma4(RsrcWords rsrc, uint32_t voffset, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds" : : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory");
}

// 16 bytes per lane from rsrc + voffset + soffset to LDS at lds + 16 * lane (soffset and lds
// uniform).
__device__ __forceinline__ void lds_dma16_so(RsrcWords rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
  soffset = __builtin_amdgcn_readfirstlane(soffset);
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               : : "v"(voffset), "s"(rsrc), "s"(soffset), "s"(lds) : "memory");
}

// 16 bytes per lane from rsrc + voffset to LDS at lds + 16 * lane (lds uniform).
__device__ __forceinline__ void lds_dma16(RsrcWords rsrc, uint32_t voffset, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
  // m0 is set and consumed inside the statement; the compiler reserves it and keeps nothing in
  // it across statements of this kernel.
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory");
}

// s_waitcnt vmcnt(N) as a statement the compiler does not move memory accesses across.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// s_waitcnt vmcnt(n) for a wave-uniform n; counts above 31 wait for 31 (a stricter wait).
__device__ __forceinline__ void wait_vm_upto(uint32_t n) {
  n = __builtin_amdgcn_readfirstlane(n);
#define AXON_WAIT_CASE(k) \
  case k: wait_vm<k>(); return;
  switch (n) {
    AXON_WAIT_CASE(0) AXON_WAIT_CASE(1) AXON_WAIT_CASE(2) AXON_WAIT_CASE(3) AXON_WAIT_CASE(4) AXON_WAIT_CASE(5)
    AXON_WAIT_CASE(6) AXON_WAIT_CASE(7) AXON_WAIT_CASE(8) AXON_WAIT_CASE(9) AXON_WAIT_CASE(10) AXON_WAIT_CASE(11)
    AXON_WAIT_CASE(12) AXON_WAIT_CASE(13) AXON_WAIT_CASE(14) AXON_WAIT_CASE(15) AXON_WAIT_CASE(16)
    AXON_WAIT_CASE(17) AXON_WAIT_CASE(18) AXON_WAIT_CASE(19) AXON_WAIT_CASE(20) AXON_WAIT_CASE(21)
    AXON_WAIT_CASE(22) AXON_WAIT_CASE(23) AXON_WAIT_CASE(24) AXON_WAIT_CASE(25) AXON_WAIT_CASE(26)
    AXON_WAIT_CASE(27) AXON_WAIT_CASE(28) AXON_WAIT_CASE(29) AXON_WAIT_CASE(30)
    default: wait_vm<31>(); return;
  }
#undef AXON_WAIT_CASE
}

// Waits for every outstanding memory operation of this wave, LDS-DMA copies included.
__device__ __forceinline__ void wait_memory() { __builtin_amdgcn_s_waitcnt(0); }

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4);  // LDS reads and writes of this wave done

// ------------------------------------------------------------------------------------------
// Host-side plumbing shared by the translation units.

hipStream_t stream();
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
inline size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }

// Kernel-time probe: hands out (and clears) the event pair armed by axon_hip_probe_next_launch.
void take_probe(hipEvent_t* start, hipEvent_t* stop);

// Launches on the library stream. When a probe is armed, the launch goes through
// hipExtLaunchKernel with the probe's events, which then carry the dispatch's own start and end
// timestamps (the kernel duration a profiler reports, without the event packets' overhead).
template <typename... Params, typename... Args>
inline void launch(void (*kernel)(Params...), dim3 grid, dim3 block, size_t lds, Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  take_probe(&start, &stop);
  if (start != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream(), start, stop, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, stream(), args...);
  }
}

}  // namespace axon_hip
