// Block dots and ordered chains of the decode matvecs, shared by the fused decode matvec
// (matvec_fused.hip) and the persistent decode-step kernel (decode_step.hip), so both compute
// the same bits: the integer-exact per-block sums of trickymind1324/axon-infer
// src/kernels/ref/quant.cpp:44-69, 161-181 and the left-to-right float accumulation over blocks.
#pragma once

#include "common.h"

namespace axon_hip {


template <int T>
constexpr int wbytes() {
  return T == Q8_0 ? kBytesQ8_0 : T == Q4_0 ? kBytesQ4_0 : kBytesQ4_1;
}

template <int T>
__device__ __forceinline__ int32_t fused_block_sumi(const uint8_t* tile, uint32_t off, const ActBlock& a, float& dw,
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
      return s - 8 * a.sum;
    } else {
      mw = half_bits_to_float(h[0] >> 16);
      return s;
    }
  }
}

template <int T>
__device__ __forceinline__ float fused_term(const uint8_t* tile, uint32_t off, const ActBlock& a) {
  float dw, mw;
  const int32_t sumi = fused_block_sumi<T>(tile, off, a, dw, mw);
  if constexpr (T == Q4_1) {
    return static_cast<float>(sumi) * dw * a.d + mw * a.d * static_cast<float>(a.sum);
  } else {
    return static_cast<float>(sumi) * dw * a.d;
  }
}

// Quantizes 8 consecutive elements held by this thread; the 4 adjacent lanes (part 0..3) hold
// one 32-element block. Writes the thread's 2 dwords of quants, and lane part 0 the scale (as
// the fp16 value the block would store) and the quant sum.
__device__ __forceinline__ void quantize8_to_act(const float (&v)[8], uint32_t part, ActBlock& blk) {
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint32_t q[8];
  int32_t s = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int32_t qi = static_cast<int32_t>(roundf(v[k] * id));
    s += qi;
    q[k] = static_cast<uint32_t>(qi) & 0xffu;
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  blk.qs[2 * part] = static_cast<int32_t>(q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24));
  blk.qs[2 * part + 1] = static_cast<int32_t>(q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24));
  if (part == 0) {
    blk.d = half_bits_to_float(float_to_half_bits(d));
    blk.sum = s;
  }
}

// Terms rows are 16-byte aligned (a multiple of 4 floats) so the chains read them four at a time.
__host__ __device__ constexpr uint32_t term_pitch(uint32_t nb) { return (nb + 3) & ~3u; }

// t[0] + t[1] + ... + t[n-1], left to right, from 16-byte aligned LDS: 64 terms at a time are
// read into registers and then added, so the dependent adds run back to back (a chain of adds
// whose operands come straight from LDS costs about twice as much per add). The tail goes in
// rounds of 16 reads that stay within the rows' padding; only the first n terms are added.
__device__ __forceinline__ float ordered_sum(const float* t, uint32_t n) {
  float acc = 0.0f;
  uint32_t i = 0;
  for (; i + 64 <= n; i += 64) {
    float4 v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = reinterpret_cast<const float4*>(t + i)[k];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      acc += v[k].x;
      acc += v[k].y;
      acc += v[k].z;
      acc += v[k].w;
    }
  }
  for (; i < n; i += 16) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 q = reinterpret_cast<const float4*>(t + i)[k];
      v[4 * k] = q.x;
      v[4 * k + 1] = q.y;
      v[4 * k + 2] = q.z;
      v[4 * k + 3] = q.w;
    }
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) {
      if (i + k < n) acc += v[k];
    }
  }
  return acc;
}


}  // namespace axon_hip
