// A whole decode step's transformer layers for one sequence as one persistent kernel: for every
// layer, q|k|v with RMSNorm, bias, RoPE and the KV write (src/model/llama.cpp:493-537), the
// attention of each head over the cache (llama.cpp:539-556, src/kernels/ref/attention.cpp:27-59),
// wo with the residual add (llama.cpp:594-595), gate|up with RMSNorm and SiLU (llama.cpp:598-620)
// and down with the residual add (llama.cpp:621-623), in the reference's order, bit for bit with
// the per-launch decode path (matvec_fused.hip, attention.hip).
//
// Why one kernel: a decode step of batch one is a chain of small dependent matvecs. As separate
// launches each costs a dispatch (2.4 us back to back on one stream) plus its own ramp-up
// (argument and activation loads, the prologue, the chain) before its weights stream; one step
// of the Llama-3.2-1B shape had 103 launches. Here one workgroup per CU runs every phase.
//
// Layout of a workgroup (512 threads): waves 0-3 compute, with the 256-thread reductions of the
// launch-per-kernel path; waves 4-7 copy weights into LDS with LDS-DMA. Each phase's slice of
// the next layer's weights (q|k|v rows, wo rows, 32 gate and 32 up rows, down rows) is issued
// when the phase after the one that used the slice starts, so the weights of a layer stream from
// HBM while the attention and the waits run, and issuing them overlaps the polls. The copying waves keep no other memory operation
// outstanding, so their waits (s_waitcnt vmcnt) count their own copies only, in issue order;
// they follow the compute waves' workgroup barriers until a phase-done flag in LDS is set.
//
// Phases hand data on without grid barriers: every value another workgroup reads (the residual
// stream x, q, the current K and V rows, the scores, the heads' outputs, the SiLU output's
// Q8_0 blocks) is stored as a 64-bit word whose high half is the number of the phase that wrote
// it (device-scope, sc1), and the reader polls exactly the words it needs until each carries
// that number. A workgroup that reads a buffer in a phase also writes something every later
// writer of that buffer waits for, so no word is overwritten before all its readers have it.
// Every poll is bounded: a workgroup that gives up writes the status word (pinned host memory)
// and leaves at its next phase; the workgroups waiting on it give up in turn, so the grid
// always drains.
#include "blockdot.h"
#include "common.h"
#include "decode_step.h"

#include <algorithm>
#include <mutex>

namespace axon_hip {

namespace {

constexpr uint32_t kStepThreads = 512;
constexpr uint32_t kCompute = 256;
constexpr uint32_t kGuRows = 32;         // gate rows (and up rows) per workgroup: one Q8_0 block of SiLU output
constexpr uint32_t kHeadDim = 64;
constexpr uint32_t kVRegs = 2;         // float4 of V slices each compute thread stages per chunk
constexpr uint32_t kVChunkF4 = kVRegs * 256;  // float4 per V chunk (8 KB)

// How long a wait polls: `limit` polls of a word before the workgroup gives up; with `never` set
// (a test hook) no word counts as written, so every wait gives up after its polls.
struct PollLimit {
  uint32_t limit;
  uint32_t never;
};

struct StepK {
  StepShape s;
  const StepLayer* layers;
  float eps, scale;
  const float* rope_table;
  float* x;
  float* cache;
  int64_t cache_off;
  int32_t pos;
  // Tagged words (phase tag << 32 | payload bits) passed between workgroups.
  uint64_t* xt;      // [d] the residual stream after wo and after down
  uint64_t* qt;      // [dq] q after bias and RoPE
  uint64_t* kvt;     // [2 * dkv] the current position's K and V rows
  uint64_t* attnt;   // [dq] the heads' outputs
  uint64_t* ht;      // [ff / 32][10] SiLU * up as Q8_0 blocks (the words of an ActBlock)
  uint64_t* scores;  // [n_head][max_ctx]
  uint32_t dsplit, dd, vchunk;  // mix: workgroups per head, dims per workgroup, positions per V chunk
  uint64_t epoch;
  uint32_t* status;
  PollLimit poll;
  uint64_t* stamps;                         // per-phase clock stamps, or null
  uint32_t stamp_stride;                    // workgroup slots per stamp point (one per CU)
  uint32_t r_qkv, r_o, r_d;                 // weight rows per workgroup
  uint32_t rb_d, rb_q, rb_ff;               // bytes per row of the d-, dq- and ff-wide matrices
  uint32_t rb_o, rb_down;
  uint32_t lds_layers, lds_qkv, lds_o, lds_gu, lds_dn, lds_scratch, scratch_bytes;
};

__device__ __forceinline__ uint64_t ld_dev(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Loads through pointers read from the LDS copy of the layer records, as global accesses (the
// compiler cannot tell their address space and would make them flat).
typedef const float __attribute__((address_space(1)))* GlobalF;
typedef float F4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 gload4(const float* p) {
  const F4v v = *reinterpret_cast<const F4v __attribute__((address_space(1)))*>(reinterpret_cast<uintptr_t>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float gload(const float* p) { return *reinterpret_cast<GlobalF>(reinterpret_cast<uintptr_t>(p)); }
typedef uint32_t U2v __attribute__((ext_vector_type(2)));
typedef uint32_t U4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t gload_u1(const void* p) {
  return *reinterpret_cast<const uint32_t __attribute__((address_space(1)))*>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ U2v gload_u2(const void* p) {
  return *reinterpret_cast<const U2v __attribute__((address_space(1)))*>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ U4v gload_u4(const void* p) {
  return *reinterpret_cast<const U4v __attribute__((address_space(1)))*>(reinterpret_cast<uintptr_t>(p));
}


// A workgroup barrier that waits for this wave's LDS accesses only (never for its copies).
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(n) for a wave-uniform n in 0..63.
__device__ __forceinline__ void wait_vm_n(uint32_t n) {
  n = __builtin_amdgcn_readfirstlane(n);
#define AXON_W(k) \
  case k: wait_vm<k>(); return;
  switch (n) {
    AXON_W(0) AXON_W(1) AXON_W(2) AXON_W(3) AXON_W(4) AXON_W(5) AXON_W(6) AXON_W(7) AXON_W(8) AXON_W(9)
    AXON_W(10) AXON_W(11) AXON_W(12) AXON_W(13) AXON_W(14) AXON_W(15) AXON_W(16) AXON_W(17) AXON_W(18)
    AXON_W(19) AXON_W(20) AXON_W(21) AXON_W(22) AXON_W(23) AXON_W(24) AXON_W(25) AXON_W(26) AXON_W(27)
    AXON_W(28) AXON_W(29) AXON_W(30) AXON_W(31) AXON_W(32) AXON_W(33) AXON_W(34) AXON_W(35) AXON_W(36)
    AXON_W(37) AXON_W(38) AXON_W(39) AXON_W(40) AXON_W(41) AXON_W(42) AXON_W(43) AXON_W(44) AXON_W(45)
    AXON_W(46) AXON_W(47) AXON_W(48) AXON_W(49) AXON_W(50) AXON_W(51) AXON_W(52) AXON_W(53) AXON_W(54)
    AXON_W(55) AXON_W(56) AXON_W(57) AXON_W(58) AXON_W(59) AXON_W(60) AXON_W(61) AXON_W(62)
    default: wait_vm<0>(); return;
  }
#undef AXON_W
}

// Copies `bytes` from src to LDS byte address lds, split over the four copying waves in 64-unit
// chunks (unit: 16 bytes when src, lds and bytes allow, else 4); returns the copies this wave
// issues (counted the same way with issue false).
__device__ __forceinline__ uint32_t dma_piece(const uint8_t* src, uint32_t lds, uint32_t bytes, uint32_t dw,
                                              uint32_t lane, bool issue) {
  if (bytes == 0) return 0;
  const bool wide = ((reinterpret_cast<uintptr_t>(src) | lds | bytes) & 15u) == 0;
  const uint32_t unit = wide ? 16u : 4u;
  const uint32_t units = bytes / unit;
  const RsrcWords rsrc = raw_buffer_words(src, bytes);
  uint32_t n = 0;
  for (uint32_t base = dw * 64; base < units; base += 256) {
    if (issue && base + lane < units) {
      if (wide) lds_dma16(rsrc, (base + lane) * 16u, lds + base * 16u);
      else lds_dma4(rsrc, (base + lane) * 4u, lds + base * 4u);
    }
    ++n;
  }
  return n;
}

enum Region : int { kQkv = 0, kWo = 1, kGu = 2, kDown = 3 };

// One layer's slice of a region for workgroup w: issue (or count) its copies.
__device__ uint32_t region_copies(const StepK& k, const StepLayer& L, int region, uint32_t w, uint32_t lds_base,
                                  uint32_t dw, uint32_t lane, bool issue) {
  const StepShape& s = k.s;
  uint32_t n = 0;
  if (region == kQkv) {
    const uint32_t r0 = w * k.r_qkv;
    const uint32_t r1 = min(r0 + k.r_qkv, s.dq + 2 * s.dkv);
    const uint8_t* bases[3] = {L.wq, L.wk, L.wv};
    const uint32_t lo_s[3] = {0, s.dq, s.dq + s.dkv};
    const uint32_t hi_s[3] = {s.dq, s.dq + s.dkv, s.dq + 2 * s.dkv};
    for (int seg = 0; seg < 3; ++seg) {
      const uint32_t lo = max(r0, lo_s[seg]), hi = min(r1, hi_s[seg]);
      if (lo < hi)
        n += dma_piece(bases[seg] + static_cast<size_t>(lo - lo_s[seg]) * k.rb_d,
                       lds_base + k.lds_qkv + (lo - r0) * k.rb_d, (hi - lo) * k.rb_d, dw, lane, issue);
    }
  } else if (region == kWo) {
    const uint32_t r0 = w * k.r_o;
    if (r0 < s.d)
      n += dma_piece(L.wo + static_cast<size_t>(r0) * k.rb_o, lds_base + k.lds_o, (min(r0 + k.r_o, s.d) - r0) * k.rb_o,
                     dw, lane, issue);
  } else if (region == kGu) {
    const uint32_t r0 = w * kGuRows;
    if (r0 < s.ff) {
      n += dma_piece(L.w_gate + static_cast<size_t>(r0) * k.rb_d, lds_base + k.lds_gu, kGuRows * k.rb_d, dw, lane, issue);
      n += dma_piece(L.w_up + static_cast<size_t>(r0) * k.rb_d, lds_base + k.lds_gu + kGuRows * k.rb_d,
                     kGuRows * k.rb_d, dw, lane, issue);
    }
  } else {
    const uint32_t r0 = w * k.r_d;
    if (r0 < s.d)
      n += dma_piece(L.w_down + static_cast<size_t>(r0) * k.rb_down, lds_base + k.lds_dn,
                     (min(r0 + k.r_d, s.d) - r0) * k.rb_down, dw, lane, issue);
  }
  return n;
}

// Block terms of nr weight rows (row pitch rb bytes in the LDS tile) against nb activation
// blocks, terms[r][b] with row pitch tp: the decomposition of the fused decode matvec.
template <int T>
__device__ __forceinline__ void terms_of(const uint8_t* tile, uint32_t rb, uint32_t nr, uint32_t nb,
                                         const ActBlock* act, float* terms, uint32_t tp, uint32_t t, uint32_t workers) {
  constexpr uint32_t bs = wbytes<T>();
  const uint32_t groups = nb <= workers ? workers / nb : 1;
  const uint32_t col0 = nb <= workers ? t % nb : t;
  const uint32_t rg = nb <= workers ? t / nb : 0;
  if (rg >= groups) return;
  for (uint32_t b = col0; b < nb; b += workers) {
    const ActBlock a = act[b];
    uint32_t r = rg;
    // Four rows at a time, so the LDS reads of all four are in flight together.
    for (; r + 3 * groups < nr; r += 4 * groups) {
      const float t0 = fused_term<T>(tile, r * rb + b * bs, a);
      const float t1 = fused_term<T>(tile, (r + groups) * rb + b * bs, a);
      const float t2 = fused_term<T>(tile, (r + 2 * groups) * rb + b * bs, a);
      const float t3 = fused_term<T>(tile, (r + 3 * groups) * rb + b * bs, a);
      terms[r * tp + b] = t0;
      terms[(r + groups) * tp + b] = t1;
      terms[(r + 2 * groups) * tp + b] = t2;
      terms[(r + 3 * groups) * tp + b] = t3;
    }
    for (; r < nr; r += groups) terms[r * tp + b] = fused_term<T>(tile, r * rb + b * bs, a);
  }
}

__device__ __forceinline__ void terms_any(int type, const uint8_t* tile, uint32_t rb, uint32_t nr, uint32_t nb,
                                          const ActBlock* act, float* terms, uint32_t tp, uint32_t t, uint32_t workers) {
  switch (type) {
  case Q8_0: terms_of<Q8_0>(tile, rb, nr, nb, act, terms, tp, t, workers); break;
  case Q4_0: terms_of<Q4_0>(tile, rb, nr, nb, act, terms, tp, t, workers); break;
  default: terms_of<Q4_1>(tile, rb, nr, nb, act, terms, tp, t, workers); break;
  }
}

// A block-terms job in LDS, published by the compute waves so the copying waves take half of
// it: the weight type, the LDS byte offsets of the weight tile, the activation blocks and the
// terms, and the shape.
struct TermsJob {
  int type;
  uint32_t tile, act, terms, rb, nr, nb, tp;
};

__device__ __forceinline__ void run_job(const TermsJob& j, uint8_t* smem, uint32_t worker) {
  terms_any(j.type, smem + j.tile, j.rb, j.nr, j.nb, reinterpret_cast<const ActBlock*>(smem + j.act),
            reinterpret_cast<float*>(smem + j.terms), j.tp, worker, kStepThreads);
}

// A tagged word: the phase's tag in the high half, 32 payload bits in the low half.
__device__ __forceinline__ void put(uint64_t* p, uint32_t tag, uint32_t bits) {
  st_dev(p, (static_cast<uint64_t>(tag) << 32) | bits);
}

// Polls n consecutive tagged words until every one carries `tag`, their payloads into out;
// false when the poll limit ran out first.
template <int N>
__device__ __forceinline__ bool take(const uint64_t* src, uint32_t tag, uint32_t (&out)[N], PollLimit poll) {
  uint64_t u[N];
  for (uint32_t spins = 0;; ++spins) {
    bool ok = poll.never == 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      u[i] = ld_dev(src + i);
      ok &= static_cast<uint32_t>(u[i] >> 32) == tag;
    }
    if (ok) break;
    if (spins >= poll.limit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = static_cast<uint32_t>(u[i]);
  return true;
}

// Polls the words p[i] with use[i] set, word i until it carries tag[i], all of them in flight
// together each round (one round trip when they are all there), payloads into out; false when
// the poll limit ran out first.
template <int N>
__device__ __forceinline__ bool take_words(const uint64_t* const (&p)[N], const bool (&use)[N],
                                           const uint32_t (&tag)[N], uint32_t (&out)[N], PollLimit poll) {
  uint64_t u[N];
  for (uint32_t spins = 0;; ++spins) {
    bool ok = poll.never == 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (use[i]) {
        u[i] = ld_dev(p[i]);
        ok &= static_cast<uint32_t>(u[i] >> 32) == tag[i];
      }
    }
    if (ok) break;
    if (spins >= poll.limit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = use[i] ? static_cast<uint32_t>(u[i]) : 0u;
  return true;
}


// RMSNorm'd and quantized activation blocks of x (d floats) into act, with rmsnorm_row_256's
// reduction (one 8-float chunk per thread, d <= 2048). x is the launch's input (xt null) or the
// tagged copy the previous phase wrote. False when the poll gave up.
// When stamping (at non-null, the same in every thread), the device clock goes to *at once every
// thread of the compute waves has passed this point (their polls done): one more barrier, which
// the copying waves' barrier loop absorbs.
__device__ __forceinline__ void stamp_at(uint64_t* at) {
  if (at == nullptr) return;
  bar();
  if (threadIdx.x == 0) *at = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ bool norm_quantize(const StepK& k, const float* gain, const uint64_t* xt, uint32_t tag,
                                              ActBlock* act, double* red, uint32_t t, uint64_t* stamp) {
  const uint32_t d = k.s.d;
  const bool has = t * 8 < d;
  float xv[8], wv[8];
  double ss = 0.0;
  bool ok = true;
  if (has) {
    // The gains first: their loads are in flight during the poll instead of after it.
    const float4 ga = gload4(gain + t * 8);
    const float4 gb = gload4(gain + t * 8 + 4);
    if (xt == nullptr) {
      const float4 a = gload4(k.x + t * 8);
      const float4 b = gload4(k.x + t * 8 + 4);
      xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w; xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    } else {
      uint32_t u[8];
      ok = take<8>(xt + t * 8, tag, u, k.poll);
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] = __uint_as_float(u[i]);
    }
    wv[0] = ga.x; wv[1] = ga.y; wv[2] = ga.z; wv[3] = ga.w; wv[4] = gb.x; wv[5] = gb.y; wv[6] = gb.z; wv[7] = gb.w;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const double v = static_cast<double>(xv[i]);
      ss += v * v;
    }
  }
  stamp_at(stamp);
  ss = block_sum_double_256(ss, red);
  const float inv = static_cast<float>(1.0 / sqrt(ss / static_cast<double>(d) + static_cast<double>(k.eps)));
  if (has) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = xv[i] * inv * wv[i];
    quantize8_to_act(v, t & 3u, act[t / 4]);
  }
  return ok;
}

// The Q8_0 block of 32 values held one per lane of a 32-lane half-wave (lane32 = 0..31), as
// quantize_block_lanes computes it, stored as 10 tagged words: the 8 quant words, the scale
// widened from its fp16 value, the quant sum (the fields of an ActBlock, in order).
__device__ __forceinline__ void put_act_block(float x, uint32_t lane32, uint64_t* dst, uint32_t tag) {
  float amax = fabsf(x);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const int32_t q = static_cast<int32_t>(roundf(x * id));
  int32_t sum = q;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 32);
  const uint32_t b = static_cast<uint32_t>(q) & 0xffu;
  const uint32_t word = b | (__shfl_down(b, 1, 32) << 8) | (__shfl_down(b, 2, 32) << 16) | (__shfl_down(b, 3, 32) << 24);
  if ((lane32 & 3u) == 0) put(dst + lane32 / 4, tag, word);
  if (lane32 == 0) {
    put(dst + 8, tag, __float_as_uint(half_bits_to_float(float_to_half_bits(d))));
    put(dst + 9, tag, static_cast<uint32_t>(sum));
  }
}

// The step's shared LDS state.
struct StepLds {
  double red[4];
  float redf[4];
  uint32_t abort, done;
  uint32_t job_seq;  // bumped when a new terms job is published
  TermsJob job;
  uint64_t exp_tab[32];  // kExp2Tab, for exp_libm_from
};

// The copying waves (4-7): the layer's weight slices into LDS, one region after the phase that
// used it, waits before the phase that needs it; between them, one barrier for each of the
// compute waves' until the phase-done flag. Its own loop, sharing no code after the split, so
// no wait the compiler places for the compute waves' loads runs here.
__device__ __forceinline__ void copier_main(const StepK& k, StepLds& sh, uint8_t* smem, const StepLayer* layers,
                                            uint32_t lds_base, uint32_t w, uint32_t dw, uint32_t lane) {
  const StepShape& s = k.s;
  uint32_t nq = region_copies(k, layers[0], kQkv, w, lds_base, dw, lane, true);
  uint32_t no = region_copies(k, layers[0], kWo, w, lds_base, dw, lane, true);
  uint32_t ng = region_copies(k, layers[0], kGu, w, lds_base, dw, lane, true);
  uint32_t nd = 0;
  // keep: copies that may stay in flight when the phase starts (63: no wait).
  auto begin = [&](uint32_t keep) -> bool {
    if (keep < 63) wait_vm_n(keep);
    bar();
    return sh.abort == 0;
  };
  uint32_t jobs_done = 0;
  auto follow = [&]() {
    for (;;) {
      bar();
      if (sh.job_seq != jobs_done) {  // this wave's half of the terms; the next barrier ends it
        jobs_done = sh.job_seq;
        run_job(sh.job, smem, threadIdx.x);
        continue;
      }
      if (sh.done != 0) break;
    }
    bar();
  };
  // Issue order per layer l, each right after the barrier that starts a phase (the region's
  // last reader finished before it), so the issue overlaps the compute waves' polls instead of
  // holding up that barrier: q|k|v of l+1 at B, down of l at C (its region holds the attention's
  // scores and value tiles during B), wo of l+1 at D, gate|up of l+1 at E. A phase's begin
  // leaves in flight only the copies issued after its own region's.
  for (uint32_t l = 0; l < s.n_layer; ++l) {
    const bool more = l + 1 < s.n_layer;
    const StepLayer& N = layers[more ? l + 1 : l];
    if (!begin(nd + no + ng)) break;  // A
    follow();
    if (!begin(63)) break;  // B
    nq = more ? region_copies(k, N, kQkv, w, lds_base, dw, lane, true) : 0;
    follow();
    if (!begin(ng + nq)) break;  // C
    nd = region_copies(k, layers[l], kDown, w, lds_base, dw, lane, true);
    follow();
    if (!begin(nq + nd)) break;  // D
    no = more ? region_copies(k, N, kWo, w, lds_base, dw, lane, true) : 0;
    follow();
    if (!begin(no)) break;  // E
    ng = more ? region_copies(k, N, kGu, w, lds_base, dw, lane, true) : 0;
    follow();
  }
  wait_vm<0>();  // no copy outlives the workgroup
}

// F16: the KV pool holds fp16 bit patterns (one instantiation per cache type, so the float
// cache's kernel carries no branch on it).
template <bool F16>
__global__ __launch_bounds__(kStepThreads) void decode_step_kernel(StepK k) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ StepLds sh;
  const StepShape& s = k.s;
  const uint32_t tid = threadIdx.x;
  const uint32_t t = tid;  // compute thread 0..255
  const uint32_t lane = tid & 63u;
  const uint32_t w = blockIdx.x;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(as_lds(smem)));
  StepLayer* layers = reinterpret_cast<StepLayer*>(smem + k.lds_layers);
  uint8_t* scratch = smem + k.lds_scratch;
  double* red = sh.red;
  // The layer records into LDS, so the copying waves read them without vector loads.
  if (tid < kCompute) {
    const uint32_t words = s.n_layer * sizeof(StepLayer) / 8;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(k.layers);
    uint64_t* dst = reinterpret_cast<uint64_t*>(layers);
    for (uint32_t i = t; i < words; i += kCompute) dst[i] = src[i];
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  if (tid == 0) {
    sh.abort = 0;
    sh.done = 0;
    sh.job_seq = 0;
  }
  if (tid < 32) sh.exp_tab[tid] = kExp2Tab[tid];
  bar();
  if (tid >= kCompute) {
    copier_main(k, sh, smem, layers, lds_base, w, (tid - kCompute) >> 6, lane);
    return;
  }

  const uint32_t kv_row = s.dkv;
  const uint32_t group = s.n_head / s.n_kv;
  constexpr bool f16 = F16;
  // A phase starts with a workgroup barrier, after which everyone knows whether to give up.
  // The flags are LDS words read right after a barrier, whose memory clobber makes the
  // compiler read them again (plain accesses keep them ds_read/ds_write; a generic or volatile
  // access would be a flat one).
  auto begin = [&]() -> bool {
    bar();
    return sh.abort == 0;
  };
  // The end of a phase: the copying waves see the phase-done flag after the first barrier, and
  // the flag is cleared after the second.
  auto lead_end = [&]() {
    if (tid == 0) sh.done = 1;
    bar();
    bar();
    if (tid == 0) sh.done = 0;
  };
  // Block terms over all eight waves: the job is published before the barrier that precedes
  // it, and the barrier after it ends the copying waves' half.
  auto terms = [&](int type, uint32_t tile, uint32_t rb, uint32_t nr, uint32_t nb, const ActBlock* act, float* out,
                   uint32_t tp) __attribute__((always_inline)) {
    if (tid == 0) {
      sh.job = TermsJob{type, tile, static_cast<uint32_t>(reinterpret_cast<const uint8_t*>(act) - smem),
                        static_cast<uint32_t>(reinterpret_cast<uint8_t*>(out) - smem), rb, nr, nb, tp};
      ++sh.job_seq;
    }
    bar();
    run_job(sh.job, smem, tid);
    bar();
  };
  auto give_up = [&]() {
    sh.abort = 1;
    __hip_atomic_store(k.status, kStepTimedOut, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  };
  // Measurement: the device clock at point pt of phase ph of layer l (stamp buffer words
  // ((l * 5 + ph) * 4 + pt) * workgroups + w); stamp_in first waits for every compute thread.
  auto slot_of = [&](uint32_t l, uint32_t ph, uint32_t pt) -> uint64_t* {
    return k.stamps == nullptr ? nullptr : k.stamps + (static_cast<size_t>(l * 5 + ph) * 4 + pt) * k.stamp_stride + w;
  };
  auto stamp = [&](uint32_t l, uint32_t ph, uint32_t pt) {
    if (k.stamps != nullptr && tid == 0) *slot_of(l, ph, pt) = __builtin_amdgcn_s_memrealtime();
  };
  auto stamp_in = [&](uint32_t l, uint32_t ph, uint32_t pt) { stamp_at(slot_of(l, ph, pt)); };
  // The rows of x this workgroup's wo and down rows update, held in registers across layers.
  const uint32_t r0x = w * k.r_o;
  const uint32_t nrx = r0x < s.d ? min(k.r_o, s.d - r0x) : 0;
  float xr = t < nrx ? gload(k.x + r0x + t) : 0.0f;
  // The attention's split, the same in every layer: KV group g = w % n_kv and this
  // workgroup's rank among the group's workgroups; the positions [p0, p1) it scores.
  const uint32_t n_vis = static_cast<uint32_t>(k.pos) + 1;
  const uint32_t last = n_vis - 1;
  const uint32_t g = w % s.n_kv, rank = w / s.n_kv;
  const uint32_t members = (gridDim.x - g + s.n_kv - 1) / s.n_kv;
  const uint32_t cs = (n_vis + members - 1) / members;
  const uint32_t p0 = min(n_vis, rank * cs), p1 = min(n_vis, p0 + cs);

  for (uint32_t l = 0; l < s.n_layer; ++l) {
    const StepLayer& L = layers[l];
    const bool more = l + 1 < s.n_layer;
    const uint32_t tag_a = static_cast<uint32_t>(k.epoch + 5ull * l + 1);
    const uint32_t tag_b = tag_a + 1, tag_c = tag_a + 2, tag_d = tag_a + 3, tag_e = tag_a + 4;

    // ---- A: RMSNorm, q|k|v, bias, RoPE, q and the KV row -----------------------------------
    if (!begin()) break;
    stamp(l, 0, 0);
    {
      const uint32_t r0 = w * k.r_qkv;
      const uint32_t nr = r0 < s.dq + 2 * s.dkv ? min(k.r_qkv, s.dq + 2 * s.dkv - r0) : 0;
      // One dword of each 128-byte line of the K and V rows this workgroup's group reads in
      // the attention (positions [p0, p1) before the current one), read while x arrives, so
      // the lines sit in this XCD's L2 by then; the values are discarded.
      float touch = 0.0f;
      const uint32_t p1t = min(p1, last);
      if constexpr (f16) {  // one 128-byte line per head row
        const uint16_t* c16 = reinterpret_cast<const uint16_t*>(k.cache) + k.cache_off + g * kHeadDim;
        for (uint32_t e = t; p0 < p1t && e < (p1t - p0) * 2; e += kCompute) {
          const int64_t layer = (e & 1u) ? L.v_layer_off : L.k_layer_off;
          touch += __uint_as_float(gload_u1(c16 + layer + static_cast<size_t>(p0 + e / 2) * kv_row));
        }
      } else {  // two per head row
        for (uint32_t e = t; p0 < p1t && e < (p1t - p0) * 4; e += kCompute) {
          const int64_t layer = (e & 2u) ? L.v_layer_off : L.k_layer_off;
          touch += gload(k.cache + k.cache_off + layer + g * kHeadDim + static_cast<size_t>(p0 + e / 4) * kv_row +
                         (e & 1u) * 32);
        }
      }
      if (nr == 0) asm volatile("" ::"v"(touch));
      if (nr > 0) {
        // This thread's output pair: its segment (q, k or v), bias and RoPE factors, loaded
        // before the norm so they are not on the path after x arrives.
        const uint32_t o = r0 + 2 * t;
        const bool pair = t < nr / 2;
        const int seg = o < s.dq ? 0 : o < s.dq + s.dkv ? 1 : 2;
        const uint32_t oo = seg == 0 ? o : seg == 1 ? o - s.dq : o - s.dq - s.dkv;
        const float* bias = seg == 0 ? L.bq : seg == 1 ? L.bk : L.bv;
        float b0 = 0.0f, b1 = 0.0f;
        if (pair && bias != nullptr) {
          b0 = gload(bias + oo);
          b1 = gload(bias + oo + 1);
        }
        const uint32_t ri = (oo % kHeadDim) / 2;
        const bool rot = seg < 2 && ri < s.rot_half;
        float2 rc = make_float2(1.0f, 0.0f);
        if (pair && rot) rc = reinterpret_cast<const float2*>(k.rope_table)[static_cast<size_t>(k.pos) * s.rot_half + ri];
        ActBlock* act = reinterpret_cast<ActBlock*>(scratch);
        const uint32_t nb = s.d / kQK;
        float* tv = reinterpret_cast<float*>(scratch + nb * sizeof(ActBlock));
        const uint32_t tp = term_pitch(nb);
        float* outv = tv + k.r_qkv * tp + 64;
        // x: the launch's input, or the previous layer's down phase.
        if (!norm_quantize(k, L.attn_norm, l == 0 ? nullptr : k.xt, tag_a - 1, act, red, t, slot_of(l, 0, 1))) give_up();
        stamp(l, 0, 2);
        asm volatile("" ::"v"(touch));  // the reads are complete: x came after them
        terms(s.t_qkv, k.lds_qkv, k.rb_d, nr, nb, act, tv, tp);
        if (t < nr) outv[t] = ordered_sum(tv + t * tp, nb);
        bar();
        if (pair) {
          float x0 = outv[2 * t], x1 = outv[2 * t + 1];
          if (bias != nullptr) {
            x0 = x0 + b0;
            x1 = x1 + b1;
          }
          if (rot) {
            const float a0 = x0, a1 = x1;
            x0 = a0 * rc.x - a1 * rc.y;
            x1 = a0 * rc.y + a1 * rc.x;
          }
          if (seg == 0) {
            put(k.qt + oo, tag_a, __float_as_uint(x0));
            put(k.qt + oo + 1, tag_a, __float_as_uint(x1));
          } else {
            // The cache row for later steps; the tagged copy for this step's attention.
            const int64_t at = k.cache_off + (seg == 1 ? L.k_layer_off : L.v_layer_off) +
                               static_cast<int64_t>(k.pos) * kv_row + oo;
            if constexpr (f16) {
              // Rounded once into the fp16 cache; this step's attention reads the rounded row,
              // as every later step does.
              const uint32_t h0 = float_to_half_bits(x0), h1 = float_to_half_bits(x1);
              *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(k.cache) + at) = h0 | (h1 << 16);
              x0 = half_value(h0);
              x1 = half_value(h1);
            } else {
              *reinterpret_cast<float2*>(k.cache + at) = make_float2(x0, x1);
            }
            uint64_t* kv = k.kvt + (seg == 1 ? 0 : s.dkv) + oo;
            put(kv, tag_a, __float_as_uint(x0));
            put(kv + 1, tag_a, __float_as_uint(x1));
          }
        }
      } else {
        stamp(l, 0, 1);
        stamp(l, 0, 2);
      }
      stamp(l, 0, 3);
      lead_end();
    }

    // ---- B: attention, the workgroups of KV group g = w % n_kv sharing its heads -----------
    // Scores: the group's positions split over its workgroups, one thread per (position, head),
    // each score stored tagged. Mix: each (head, slice of the head's dims) on one workgroup of
    // the group, which waits for the head's scores, softmaxes them itself and runs the
    // in-order chains of its dims over V slices staged in LDS.
    if (!begin()) break;
    stamp(l, 1, 0);
    {
      float* qs = reinterpret_cast<float*>(smem + k.lds_dn);  // the down region is copied only
      float* klast = qs + group * kHeadDim;                     // after this phase
      float* sc = klast + kHeadDim;
      float* vb = sc + ((s.max_ctx + 3) & ~3u);
      const float* kbase = k.cache + k.cache_off + L.k_layer_off + g * kHeadDim;
      const uint16_t* kbase16 = reinterpret_cast<const uint16_t*>(k.cache) + k.cache_off + L.k_layer_off + g * kHeadDim;
      // A K row's raw words (fp32: 16 float4; fp16: 8 x 8 halves) and q . k over them, the
      // products added in dimension order, as the reference's dot.
      auto kfetch = [&](uint32_t j, float4 (&f)[kHeadDim / 4], U4v (&hh)[kHeadDim / 8]) {
        if constexpr (f16) {
          const uint16_t* kb = kbase16 + static_cast<size_t>(j) * kv_row;
#pragma unroll
          for (uint32_t i = 0; i < kHeadDim / 8; ++i) hh[i] = gload_u4(kb + 8 * i);
        } else {
#pragma unroll
          for (uint32_t i = 0; i < kHeadDim / 4; ++i) f[i] = gload4(kbase + static_cast<size_t>(j) * kv_row + 4 * i);
        }
      };
      auto kdot = [&](const float* qh, const float4 (&f)[kHeadDim / 4], const U4v (&hh)[kHeadDim / 8]) -> float {
        float acc = 0.0f;
        if constexpr (f16) {
#pragma unroll
          for (uint32_t i = 0; i < kHeadDim / 8; ++i) {
#pragma unroll
            for (uint32_t c = 0; c < 4; ++c) {
              acc += mul_half_bits(qh[8 * i + 2 * c], hh[i][c]);
              acc += mul_half_bits_hi(qh[8 * i + 2 * c + 1], hh[i][c]);
            }
          }
        } else {
#pragma unroll
          for (uint32_t i = 0; i < kHeadDim / 4; ++i) {
            acc += qh[4 * i] * f[i].x;
            acc += qh[4 * i + 1] * f[i].y;
            acc += qh[4 * i + 2] * f[i].z;
            acc += qh[4 * i + 3] * f[i].w;
          }
        }
        return acc;
      };
      auto kdot_last = [&](const float* qh) -> float {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < kHeadDim; ++i) acc += qh[i] * klast[i];
        return acc;
      };
      if (p0 < p1) {
        const uint32_t pairs = (p1 - p0) * group;
        // The group's q and (on the workgroup that scores the current position) its K row, in
        // rounds of up to 4 q words and that K word per thread.
        bool ok = true;
        for (uint32_t i0 = 0; ok && i0 < group * kHeadDim; i0 += 4 * kCompute) {
          const uint64_t* p[5];
          bool use[5];
          uint32_t tg[5], got[5];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t i = i0 + t + u * kCompute;
            use[u] = i < group * kHeadDim;
            p[u] = k.qt + g * group * kHeadDim + (use[u] ? i : 0);
            tg[u] = tag_a;
          }
          use[4] = i0 == 0 && p1 == n_vis && t < kHeadDim;
          p[4] = k.kvt + g * kHeadDim + (t < kHeadDim ? t : 0);
          tg[4] = tag_a;
          ok = take_words<5>(p, use, tg, got, k.poll);
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u)
            if (use[u]) qs[i0 + t + u * kCompute] = __uint_as_float(got[u]);
          if (use[4]) klast[t] = __uint_as_float(got[4]);
        }
        if (!ok) give_up();
        bar();
        stamp(l, 1, 1);
        float4 kf[kHeadDim / 4];
        U4v kh[kHeadDim / 8];
        for (uint32_t e = t; e < pairs; e += kCompute) {
          const uint32_t j = p0 + e / group, hi = e % group;
          const float* qh = qs + hi * kHeadDim;
          float acc;
          if (j == last) {
            acc = kdot_last(qh);
          } else {
            kfetch(j, kf, kh);
            acc = kdot(qh, kf, kh);
          }
          put(k.scores + static_cast<size_t>(g * group + hi) * s.max_ctx + j, tag_b, __float_as_uint(k.scale * acc));
        }
      } else {
        stamp(l, 1, 1);
      }
      if (rank < group * k.dsplit) {
        const uint32_t h = g * group + rank / k.dsplit;
        const uint32_t dim0 = (rank % k.dsplit) * k.dd;
        const uint32_t per = k.dd / 4;  // float4 of a V row slice
        const float* vbase = k.cache + k.cache_off + L.v_layer_off + g * kHeadDim + dim0;
        const uint16_t* vbase16 =
            reinterpret_cast<const uint16_t*>(k.cache) + k.cache_off + L.v_layer_off + g * kHeadDim + dim0;
        // V slices of positions [0, last) in chunks of vchunk positions, kVRegs float4 per thread.
        float4 vr[kVRegs];  // float cache: the values
        U2v vh[kVRegs];     // fp16 cache: the values' bits (the products widen them)
        auto vload = [&](uint32_t c) {
#pragma unroll
          for (uint32_t u = 0; u < kVRegs; ++u) {
            const uint32_t unit = t + u * kCompute;
            const uint32_t j = c * k.vchunk + unit / per;
            if constexpr (f16) {
              if (j < last) {
                vh[u] = gload_u2(vbase16 + static_cast<size_t>(j) * kv_row + 4 * (unit % per));
              } else {
                vh[u][0] = 0u;
                vh[u][1] = 0u;
              }
            } else {
              vr[u] = j < last ? gload4(vbase + static_cast<size_t>(j) * kv_row + 4 * (unit % per))
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
          }
        };
        vload(0);
        bool ok = true;
        float vlast = 0.0f;
        // The head's scores, in rounds of up to 8 per thread (one round for up to 2048
        // positions), the first with this slice's word of the current V row.
        const uint64_t* src = k.scores + static_cast<size_t>(h) * s.max_ctx;
        for (uint32_t j0 = 0; ok && j0 < n_vis; j0 += 8 * kCompute) {
          const uint64_t* p[9];
          bool use[9];
          uint32_t tg[9], got[9];
#pragma unroll
          for (uint32_t u = 0; u < 8; ++u) {
            const uint32_t j = j0 + t + u * kCompute;
            use[u] = j < n_vis;
            p[u] = src + (use[u] ? j : 0);
            tg[u] = tag_b;
          }
          use[8] = j0 == 0 && t < k.dd;
          p[8] = k.kvt + s.dkv + g * kHeadDim + dim0 + (t < k.dd ? t : 0);
          tg[8] = tag_a;
          ok = take_words<9>(p, use, tg, got, k.poll);
#pragma unroll
          for (uint32_t u = 0; u < 8; ++u)
            if (use[u]) sc[j0 + t + u * kCompute] = __uint_as_float(got[u]);
          if (use[8]) vlast = __uint_as_float(got[8]);
        }
        if (!ok) give_up();
        bar();
        stamp(l, 1, 2);
        if (sh.abort == 0) {
          // Softmax: the maximum, e = exp(s - max), the double sum over the 256-thread tree,
          // p = e / sum.
          float m = -INFINITY;
          for (uint32_t j = t; j < n_vis; j += kCompute) m = fmaxf(m, sc[j]);
#pragma unroll
          for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
          if (lane == 0) sh.redf[t >> 6] = m;
          bar();
          m = fmaxf(fmaxf(sh.redf[0], sh.redf[1]), fmaxf(sh.redf[2], sh.redf[3]));
          double part = 0.0;
          for (uint32_t j = t; j < n_vis; j += kCompute) {
            const float e = exp_libm_from(sc[j] - m, sh.exp_tab);
            sc[j] = e;
            part += static_cast<double>(e);
          }
          const double sum = block_sum_double_256(part, red);
          const float inv = static_cast<float>(1.0 / sum);
          // Mix: lane d of wave 0 adds p[j] * v[j][dim0 + d] over j in ascending order, with
          // p[j] = e[j] * inv. Each chunk's V slices go, as the products p[j] * v[j][d], to one of
          // two LDS buffers laid out [d][position] (rows padded by 4 floats), while the next
          // chunk's loads fly; the chain then reads 4 positions per LDS read.
          float acc = 0.0f;
          const uint32_t pitch = k.vchunk + 4;
          const uint32_t chunks = (last + k.vchunk - 1) / k.vchunk;
          for (uint32_t c = 0; c < chunks; ++c) {
            float* buf = vb + (c & 1u) * k.dd * pitch;
            const uint32_t j0 = c * k.vchunk;
            const uint32_t cnt = min(k.vchunk, last - j0);
#pragma unroll
            for (uint32_t u = 0; u < kVRegs; ++u) {
              const uint32_t unit = t + u * kCompute;
              const uint32_t jj = unit / per, q = unit % per;
              if (jj < cnt) {
                const float p = sc[j0 + jj] * inv;
                float* dst = buf + 4 * q * pitch + jj;
                if constexpr (f16) {
                  dst[0] = mul_half_bits(p, vh[u][0]);
                  dst[pitch] = mul_half_bits_hi(p, vh[u][0]);
                  dst[2 * pitch] = mul_half_bits(p, vh[u][1]);
                  dst[3 * pitch] = mul_half_bits_hi(p, vh[u][1]);
                } else {
                  dst[0] = p * vr[u].x;
                  dst[pitch] = p * vr[u].y;
                  dst[2 * pitch] = p * vr[u].z;
                  dst[3 * pitch] = p * vr[u].w;
                }
              }
            }
            if (c + 1 < chunks) vload(c + 1);
            bar();
            if (t < k.dd) {
              const float4* row = reinterpret_cast<const float4*>(buf + t * pitch);
              uint32_t jj = 0;
              for (; jj + 64 <= cnt; jj += 64) {
                float4 v[16];
#pragma unroll
                for (uint32_t i = 0; i < 16; ++i) v[i] = row[jj / 4 + i];
#pragma unroll
                for (uint32_t i = 0; i < 16; ++i) {
                  acc += v[i].x;
                  acc += v[i].y;
                  acc += v[i].z;
                  acc += v[i].w;
                }
              }
              for (; jj + 4 <= cnt; jj += 4) {
                const float4 v = row[jj / 4];
                acc += v.x;
                acc += v.y;
                acc += v.z;
                acc += v.w;
              }
              const float* tail = buf + t * pitch;
              for (; jj < cnt; ++jj) acc += tail[jj];
            }
          }
          if (t < k.dd) {
            acc += (sc[last] * inv) * vlast;
            put(k.attnt + h * kHeadDim + dim0 + t, tag_b, __float_as_uint(acc));
          }
        }
      } else {
        stamp(l, 1, 2);
      }
      stamp(l, 1, 3);
      lead_end();
    }

    // ---- C: wo and the residual add ---------------------------------------------------------
    if (!begin()) break;
    stamp(l, 2, 0);
    if (nrx > 0) {
      const uint32_t nb = s.dq / kQK;
      ActBlock* act = reinterpret_cast<ActBlock*>(scratch);
      float* tv = reinterpret_cast<float*>(scratch + nb * sizeof(ActBlock));
      const uint32_t tp = term_pitch(nb);
      float* outv = tv + k.r_o * tp + 64;
      if (t * 8 < s.dq) {  // the heads' outputs as Q8_0 blocks, 8 values per thread
        uint32_t u[8];
        if (!take<8>(k.attnt + t * 8, tag_b, u, k.poll)) give_up();
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(u[i]);
        quantize8_to_act(v, t & 3u, act[t / 4]);
      }
      stamp_in(l, 2, 1);
      stamp(l, 2, 2);
      terms(s.t_o, k.lds_o, k.rb_o, nrx, nb, act, tv, tp);
      if (t < nrx) outv[t] = ordered_sum(tv + t * tp, nb);
      bar();
      if (t < nrx) {
        xr = xr + outv[t];
        put(k.xt + r0x + t, tag_c, __float_as_uint(xr));
      }
    } else {
      stamp(l, 2, 1);
      stamp(l, 2, 2);
    }
    stamp(l, 2, 3);
    lead_end();

    // ---- D: RMSNorm, gate|up, SiLU * up, its Q8_0 block ------------------------------------
    if (!begin()) break;
    stamp(l, 3, 0);
    if (w * kGuRows < s.ff) {
      const uint32_t nb = s.d / kQK;
      ActBlock* act = reinterpret_cast<ActBlock*>(scratch);
      float* tv = reinterpret_cast<float*>(scratch + nb * sizeof(ActBlock));
      const uint32_t tp = term_pitch(nb);
      float* outv = tv + 2 * kGuRows * tp + 64;
      if (!norm_quantize(k, L.ffn_norm, k.xt, tag_c, act, red, t, slot_of(l, 3, 1))) give_up();
      stamp(l, 3, 2);
      terms(s.t_gu, k.lds_gu, k.rb_d, 2 * kGuRows, nb, act, tv, tp);
      if (t < 2 * kGuRows) outv[t] = ordered_sum(tv + t * tp, nb);
      bar();
      if (t < kGuRows) {
        const float gt = outv[t];
        const float u = outv[kGuRows + t];
        const float hv = gt / (1.0f + exp_libm_from(-gt, sh.exp_tab)) * u;
        put_act_block(hv, t, k.ht + static_cast<size_t>(w) * 10, tag_d);
      }
    } else {
      stamp(l, 3, 1);
      stamp(l, 3, 2);
    }
    stamp(l, 3, 3);
    lead_end();

    // ---- E: down and the residual add -------------------------------------------------------
    if (!begin()) break;
    stamp(l, 4, 0);
    if (nrx > 0) {
      const uint32_t nb = s.ff / kQK;
      ActBlock* act = reinterpret_cast<ActBlock*>(scratch);
      float* tv = reinterpret_cast<float*>(scratch + nb * sizeof(ActBlock));
      const uint32_t tp = term_pitch(nb);
      float* outv = tv + k.r_d * tp + 64;
      if (t < nb) {
        uint32_t u[10];
        if (!take<10>(k.ht + static_cast<size_t>(t) * 10, tag_d, u, k.poll)) give_up();
        ActBlock& a = act[t];
#pragma unroll
        for (int i = 0; i < 8; ++i) a.qs[i] = static_cast<int32_t>(u[i]);
        a.d = __uint_as_float(u[8]);
        a.sum = static_cast<int32_t>(u[9]);
      }
      stamp_in(l, 4, 1);
      stamp(l, 4, 2);
      terms(s.t_down, k.lds_dn, k.rb_down, nrx, nb, act, tv, tp);
      if (t < nrx) outv[t] = ordered_sum(tv + t * tp, nb);
      bar();
      if (t < nrx) {
        xr = xr + outv[t];
        if (more) put(k.xt + r0x + t, tag_e, __float_as_uint(xr));
        else k.x[r0x + t] = xr;  // the step's output, read by the launches after this one
      }
    } else {
      stamp(l, 4, 1);
      stamp(l, 4, 2);
    }
    stamp(l, 4, 3);
    lead_end();
  }
}

// Row split and LDS layout for one shape on a grid of `wgs` workgroups.
bool step_geometry(const StepShape& s, uint32_t wgs, StepK& k, size_t* lds_out, const char** why) {
  auto bytes_of = [](int t, uint32_t n) -> uint32_t {
    return n / kQK * (t == Q8_0 ? kBytesQ8_0 : t == Q4_0 ? kBytesQ4_0 : kBytesQ4_1);
  };
  auto align16 = [](size_t v) { return (v + 15) & ~size_t(15); };
  const uint32_t n_qkv = s.dq + 2 * s.dkv;
  k.r_qkv = static_cast<uint32_t>(ceil_div(n_qkv, wgs));
  k.r_qkv += k.r_qkv & 1u;
  k.r_o = static_cast<uint32_t>(ceil_div(s.d, wgs));
  k.r_d = k.r_o;
  k.rb_d = bytes_of(s.t_qkv, s.d);
  k.rb_o = bytes_of(s.t_o, s.dq);
  k.rb_down = bytes_of(s.t_down, s.ff);
  const uint32_t rb_gu = bytes_of(s.t_gu, s.d);
  if (rb_gu != k.rb_d) {
    *why = "q|k|v and gate|up of different block types";
    return false;
  }
  if ((k.rb_d | k.rb_o | k.rb_down) % 4 != 0) {
    *why = "weight rows that are not whole dwords (LDS-DMA copies move dwords)";
    return false;
  }
  size_t off = 0;
  k.lds_qkv = static_cast<uint32_t>(off);
  off = align16(off + static_cast<size_t>(k.r_qkv) * k.rb_d);
  k.lds_o = static_cast<uint32_t>(off);
  off = align16(off + static_cast<size_t>(k.r_o) * k.rb_o);
  k.lds_gu = static_cast<uint32_t>(off);
  off = align16(off + static_cast<size_t>(2 * kGuRows) * k.rb_d);
  // Attention: the workgroups of a KV group (at least wgs / n_kv) give each of its heads
  // dsplit of them, a power of two up to 16, each mixing dd = 64 / dsplit dims.
  const uint32_t group = s.n_head / s.n_kv;
  const uint32_t per_head = wgs / s.n_kv / group;
  if (per_head == 0) {
    *why = "fewer workgroups per KV group than heads sharing it";
    return false;
  }
  k.dsplit = 1;
  while (k.dsplit * 2 <= std::min(per_head, 16u)) k.dsplit *= 2;
  k.dd = kHeadDim / k.dsplit;
  k.vchunk = kVChunkF4 * 4 / k.dd;
  k.lds_dn = static_cast<uint32_t>(off);
  const size_t attn =
      (static_cast<size_t>(group + 1) * kHeadDim + ((s.max_ctx + 3) & ~3u) + 2 * (kVChunkF4 * 4 + 4 * kHeadDim)) * 4;
  off = align16(off + std::max(static_cast<size_t>(k.r_d) * k.rb_down, attn));
  k.lds_layers = static_cast<uint32_t>(off);
  off = align16(off + static_cast<size_t>(s.n_layer) * sizeof(StepLayer));
  k.lds_scratch = static_cast<uint32_t>(off);
  // Scratch per matvec phase: activation blocks, terms (rows x pitch, +64 floats for the
  // chains' reads past a row), the chain results. The attention phase uses the down region:
  // the group's q rows, the current K row, the scores of max_ctx positions, two V chunks (as
  // products, rows padded by 4 floats).
  auto mv = [&](uint32_t n_in, uint32_t rows) {
    const uint32_t nb = n_in / kQK;
    return static_cast<size_t>(nb) * sizeof(ActBlock) + (static_cast<size_t>(rows) * term_pitch(nb) + 64 + rows) * 4;
  };
  const size_t scratch = std::max({mv(s.d, k.r_qkv), mv(s.dq, k.r_o), mv(s.d, 2 * kGuRows), mv(s.ff, k.r_d)});
  k.scratch_bytes = static_cast<uint32_t>(align16(scratch));
  *lds_out = off + k.scratch_bytes;
  return true;
}

uint32_t g_cus = 0;
size_t g_lds_granted = 0;
std::mutex g_step_mutex;

int step_device(uint32_t* cus, size_t* lds_max) {
  std::lock_guard<std::mutex> lock(g_step_mutex);
  if (g_cus == 0) {
    int dev = 0, n = 0, smem = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&smem, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      return fail(kHipError, "decode step: device attributes");
    const size_t want = static_cast<size_t>(smem) - 1024;  // the kernel's static LDS beside it
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(decode_step_kernel<false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(want)) != hipSuccess ||
        hipFuncSetAttribute(reinterpret_cast<const void*>(decode_step_kernel<true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(want)) != hipSuccess) {
      (void)hipGetLastError();
      return fail(kUnsupported, "decode step: %zu bytes of LDS not granted", want);
    }
    g_cus = static_cast<uint32_t>(n);
    g_lds_granted = want;
  }
  *cus = g_cus;
  *lds_max = g_lds_granted;
  return kOk;
}

// The copies one copying wave issues per region, as the kernel counts them (host mirror).
uint32_t copies_host(uint32_t bytes, bool wide, uint32_t dw) {
  const uint32_t units = bytes / (wide ? 16u : 4u);
  uint32_t n = 0;
  for (uint32_t base = dw * 64; base < units; base += 256) ++n;
  return n;
}

}  // namespace

namespace {
// Workspace layout (tagged words, each array 256-byte aligned): xt [d] | qt [dq] | kvt [2 dkv] |
// attnt [dq] | ht [ff / 32 * 10] | scores [n_head * max_ctx].
struct WorkLayout {
  size_t xt, qt, kvt, attnt, ht, scores, total;
};
WorkLayout work_layout(const StepShape& s) {
  auto words = [](size_t n) { return (n * 8 + 255) & ~size_t(255); };
  WorkLayout w{};
  w.xt = 0;
  w.qt = w.xt + words(s.d);
  w.kvt = w.qt + words(s.dq);
  w.attnt = w.kvt + words(2 * static_cast<size_t>(s.dkv));
  w.ht = w.attnt + words(s.dq);
  w.scores = w.ht + words(static_cast<size_t>(s.ff / kQK) * 10);
  w.total = w.scores + words(static_cast<size_t>(s.n_head) * s.max_ctx);
  return w;
}
// Why a grid of `wgs` workgroups cannot run the shape, or null.
const char* grid_unsupported(const StepShape& s, uint32_t wgs, size_t lds_max) {
  if (s.n_head > wgs || ceil_div(s.ff, kGuRows) > wgs) return "more heads or SiLU blocks than CUs";
  StepK k{};
  k.s = s;
  size_t lds = 0;
  const char* why = nullptr;
  if (!step_geometry(s, wgs, k, &lds, &why)) return why;
  if (lds > lds_max) return "the layer's weight slices and scratch exceed LDS";
  // Every copying wave keeps at most 63 copies in flight: one layer's four regions.
  for (uint32_t dw = 0; dw < 4; ++dw) {
    auto wide = [](uint32_t rb, uint32_t rows) { return (rb * rows) % 16 == 0 && rb % 16 == 0; };
    const uint32_t n = copies_host(k.r_qkv * k.rb_d, wide(k.rb_d, k.r_qkv), dw) * 3 +
                       copies_host(k.r_o * k.rb_o, wide(k.rb_o, k.r_o), dw) +
                       2 * copies_host(kGuRows * k.rb_d, wide(k.rb_d, kGuRows), dw) +
                       copies_host(k.r_d * k.rb_down, wide(k.rb_down, k.r_d), dw);
    if (n > 63) return "a layer's weight slices need more copies in flight than a wave can count";
  }
  return nullptr;
}

// Workgroups of the step grid: kSmallGrid when the shape runs on that many, else one per CU.
// Each phase's hand-off is an all-to-all of tagged words whose cost grows with the workgroups
// that write them (one round of 256 writers and readers takes about 2.6 us on MI355X, of 128
// about 1.7 us), so a model small enough to run on half the CUs does (C1, SmolLM2-135M: 1382
// against 1272 tokens/s); larger ones need every CU's LDS for their weight slices.
constexpr uint32_t kSmallGrid = 128;
uint32_t step_grid(const StepShape& s, uint32_t cus, size_t lds_max) {
  return cus > kSmallGrid && grid_unsupported(s, kSmallGrid, lds_max) == nullptr ? kSmallGrid : cus;
}

}  // namespace

size_t step_workspace_bytes(const StepShape& s) { return work_layout(s).total; }

size_t step_stamp_count(const StepShape& s) {
  uint32_t cus = 0;
  size_t lds_max = 0;
  if (step_device(&cus, &lds_max) != kOk) return 0;
  return static_cast<size_t>(s.n_layer) * 5 * 4 * cus;
}

uint64_t step_phases(const StepShape& s) { return 5ull * s.n_layer; }

const char* step_unsupported(const StepShape& s) {
  if (s.n_layer == 0) return "no layers";
  if (s.max_ctx == 0) return "no positions";
  for (int t : {s.t_qkv, s.t_o, s.t_gu, s.t_down})
    if (t != Q8_0 && t != Q4_0 && t != Q4_1) return "a layer matrix outside Q8_0 / Q4_0 / Q4_1";
  if (s.n_kv == 0 || s.n_head % s.n_kv != 0 || s.dq != s.n_head * kHeadDim || s.dkv != s.n_kv * kHeadDim)
    return "heads other than 64 wide";
  if (s.d % kQK != 0 || s.d > 2048 || s.dq > 2048 || s.ff % kQK != 0 || s.rot_half > kHeadDim / 2)
    return "a width outside the kernel's norm and block layout";
  uint32_t cus = 0;
  size_t lds_max = 0;
  if (step_device(&cus, &lds_max) != kOk) return "the device does not grant the kernel's LDS";
  return grid_unsupported(s, cus, lds_max);
}

int step_launch(const StepShape& s, const StepCall& c) {
  uint32_t cus = 0;
  size_t lds_max = 0;
  const int rc = step_device(&cus, &lds_max);
  if (rc != kOk) return rc;
  if (c.pos < 0 || static_cast<uint32_t>(c.pos) >= s.max_ctx)
    return fail(kInvalidArgument, "decode step: position %d outside [0, %u)", c.pos, s.max_ctx);
  const char* why = step_unsupported(s);
  if (why != nullptr) return fail(kUnsupported, "decode step: %s", why);
  const uint32_t wgs = step_grid(s, cus, lds_max);
  StepK k{};
  k.s = s;
  size_t lds = 0;
  if (!step_geometry(s, wgs, k, &lds, &why)) return fail(kUnsupported, "decode step: %s", why);
  k.layers = c.layers;
  k.eps = c.eps;
  k.scale = c.scale;
  k.rope_table = c.rope_table;
  k.x = c.x;
  k.cache = c.cache;
  k.cache_off = c.cache_off;
  k.pos = c.pos;
  uint8_t* work = static_cast<uint8_t*>(c.work);
  const WorkLayout wl = work_layout(s);
  k.xt = reinterpret_cast<uint64_t*>(work + wl.xt);
  k.qt = reinterpret_cast<uint64_t*>(work + wl.qt);
  k.kvt = reinterpret_cast<uint64_t*>(work + wl.kvt);
  k.attnt = reinterpret_cast<uint64_t*>(work + wl.attnt);
  k.ht = reinterpret_cast<uint64_t*>(work + wl.ht);
  k.scores = reinterpret_cast<uint64_t*>(work + wl.scores);
  k.epoch = c.epoch;
  k.status = c.status;
  k.poll = PollLimit{c.spin_limit, c.fail_waits};
  k.stamps = c.stamps;
  k.stamp_stride = cus;
  void* args[] = {&k};
  const void* kernel = s.cache_f16 ? reinterpret_cast<const void*>(decode_step_kernel<true>)
                                   : reinterpret_cast<const void*>(decode_step_kernel<false>);
  // A probed launch is bracketed by events on the stream.
  hipEvent_t start = nullptr, stop = nullptr;
  take_probe(&start, &stop);
  if (start != nullptr && hipEventRecord(start, stream()) != hipSuccess)
    return fail(kHipError, "decode step: probe start event");
  // An ordinary launch of one workgroup per CU (the most a CU holds at this LDS size): on a
  // device with nothing else running, the stream's previous kernel done, every workgroup is
  // resident. The kernel needs no more than that (its hand-offs are its own tagged words, not
  // a grid barrier), and every wait is bounded: a workgroup that never became resident makes
  // the call give up (status word), not hang. The cooperative launch API, which checks
  // residency at the launch, cost about 15 us per launch on this runtime and profilers lose
  // their results for processes that use it, so it is not used.
  const hipError_t e = hipLaunchKernel(kernel, dim3(wgs), dim3(kStepThreads), args, static_cast<unsigned>(lds), stream());
  if (e != hipSuccess) return fail(kHipError, "decode step: launch: %s", hipGetErrorString(e));
  if (stop != nullptr && hipEventRecord(stop, stream()) != hipSuccess)
    return fail(kHipError, "decode step: probe stop event");
  return kOk;
}

}  // namespace axon_hip
