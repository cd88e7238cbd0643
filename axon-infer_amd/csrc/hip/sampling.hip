// Greedy token selection on the device, as the reference's sampler takes it at temperature zero
// (trickymind1324/axon-infer src/sampling/sampler.cpp:67-102): the repetition penalty over each
// row's recent tokens, then the index of the first maximum (std::ranges::max_element). Only the
// chosen ids cross to the host instead of [rows][n_vocab] floats.
//
// Penalty (sampler.cpp:73-97): one workgroup per row; each distinct in-range id of the row's
// window is rescaled once, by the thread holding its first occurrence, so no two threads write
// one logit. The window is short (repeat_last_n, 64 by default), so the quadratic first-occurrence
// scan costs less than a launch.
//
// Argmax, two launches: kParts workgroups per row each reduce a contiguous slice to one key, then one
// wave per row reduces the keys. A key orders (value, index) as max_element does: a larger
// value wins, and between equal values the smaller index. Values map to an unsigned order that
// matches float comparison for every non-NaN value (negative zero and zero compare equal, as
// they do with `<`). NaN follows max_element's scan with `<`: a NaN never replaces the running
// maximum and is skipped, except that a NaN in the first element is never replaced, so such a
// row selects index 0.
//
// Top-k (the candidates of the stochastic stages, sampler.cpp:104-118): one workgroup per row
// returns the row's k largest logits in descending order, equal logits by ascending id (the
// reference's std::partial_sort leaves their order unspecified; ascending id is the oracle's
// choice), NaN skipped. A candidate is the (value, index) key above, so every key is distinct.
// Rounds: each thread keeps the four largest keys below a bound among its strided elements;
// the 4096 kept keys are sorted in LDS (bitonic). Let M be the largest fourth key over the
// threads that kept four. Every key above M is then among the kept ones (a thread's dropped keys
// lie below its fourth), so the sorted keys above M are the row's next keys in order and are
// taken. The thread that holds M kept three keys above it, so a round takes at least three,
// and on a row of random logits the first round takes all k.
#include "common.h"
#include "elementwise.h"

#include <mutex>

namespace axon_hip {

namespace {

constexpr uint32_t kParts = 64;
constexpr uint32_t kThreads = 256;

__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float* __restrict__ x, uint32_t n,
                                                                  size_t stride, uint64_t* __restrict__ part) {
  __shared__ uint64_t red[kThreads / 64];
  const uint32_t r = blockIdx.y;
  const uint32_t chunk = (n + kParts - 1) / kParts;
  const uint32_t j0 = blockIdx.x * chunk;
  const uint32_t j1 = min(n, j0 + chunk);
  const float* row = x + static_cast<size_t>(r) * stride;
  uint64_t best = 0;
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kThreads) {
    const float v = row[j];
    if (v == v) {  // NaN never compares greater under max_element's `<`
      const uint64_t k = argmax_key(v, j);
      best = k > best ? k : best;
    }
  }
  best = max_key_wave(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t k = red[0];
    for (uint32_t w = 1; w < kThreads / 64; ++w) k = red[w] > k ? red[w] : k;
    part[static_cast<size_t>(r) * kParts + blockIdx.x] = k;
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ x, size_t stride,
                                                          const uint64_t* __restrict__ part, int32_t* __restrict__ out) {
  const uint32_t r = blockIdx.x;
  const uint64_t k = max_key_wave(part[static_cast<size_t>(r) * kParts + threadIdx.x]);
  if (threadIdx.x == 0) {
    const float first = x[static_cast<size_t>(r) * stride];
    // A NaN first element, or no key at all (every value NaN): index 0.
    out[r] = (first != first || k == 0) ? 0 : static_cast<int32_t>(~static_cast<uint32_t>(k & 0xffffffffu));
  }
}

__global__ __launch_bounds__(256) void repeat_penalty_kernel(float* __restrict__ x, uint32_t n, size_t stride,
                                                             const int32_t* __restrict__ recent,
                                                             const uint32_t* __restrict__ recent_len,
                                                             size_t recent_stride, float penalty) {
  const uint32_t r = blockIdx.x;
  const int32_t* ids = recent + static_cast<size_t>(r) * recent_stride;
  const uint32_t m = static_cast<uint32_t>(min(static_cast<size_t>(recent_len[r]), recent_stride));
  float* row = x + static_cast<size_t>(r) * stride;
  for (uint32_t i = threadIdx.x; i < m; i += blockDim.x) {
    const int32_t id = ids[i];
    if (id < 0 || static_cast<uint32_t>(id) >= n) continue;
    bool first = true;
    for (uint32_t j = 0; j < i && first; ++j) first = ids[j] != id;
    if (!first) continue;
    const float v = row[id];
    row[id] = v > 0.0f ? v / penalty : v * penalty;  // correctly rounded division, as on the host
  }
}

constexpr uint32_t kTopKThreads = 1024;
constexpr uint32_t kTopKKeep = 4;
constexpr uint32_t kTopKKeys = kTopKThreads * kTopKKeep;

__global__ __launch_bounds__(kTopKThreads) void topk_rows_kernel(const float* __restrict__ x, uint32_t n, size_t stride,
                                                                 uint32_t k, float* __restrict__ out_logit,
                                                                 int32_t* __restrict__ out_id) {
  __shared__ uint64_t keys[kTopKKeys];
  __shared__ uint64_t red[kTopKThreads / 64];
  __shared__ uint32_t taken;
  const uint32_t r = blockIdx.x;
  const uint32_t t = threadIdx.x;
  const float* row = x + static_cast<size_t>(r) * stride;
  float* ol = out_logit + static_cast<size_t>(r) * k;
  int32_t* oi = out_id + static_cast<size_t>(r) * k;
  uint32_t got = 0;
  uint64_t bound = ~0ull;  // above every key
  for (;;) {
    uint64_t c0 = 0, c1 = 0, c2 = 0, c3 = 0;  // descending; 0 is below every key
    for (uint32_t j = t; j < n; j += kTopKThreads) {
      const float v = row[j];
      if (v != v) continue;
      const uint64_t key = argmax_key(v, j);
      if (key >= bound || key <= c3) continue;
      if (key > c2) {
        c3 = c2;
        if (key > c1) {
          c2 = c1;
          if (key > c0) {
            c1 = c0;
            c0 = key;
          } else {
            c1 = key;
          }
        } else {
          c2 = key;
        }
      } else {
        c3 = key;
      }
    }
    const uint64_t m = max_key_wave(c3);
    if ((t & 63) == 0) red[t >> 6] = m;
    keys[kTopKKeep * t] = c0;
    keys[kTopKKeep * t + 1] = c1;
    keys[kTopKKeep * t + 2] = c2;
    keys[kTopKKeep * t + 3] = c3;
    if (t == 0) taken = 0;
    __syncthreads();
    // Bitonic sort, descending: 2048 compare-exchanges per stage, two per thread.
    for (uint32_t size = 2; size <= kTopKKeys; size <<= 1) {
      for (uint32_t half = size >> 1; half > 0; half >>= 1) {
#pragma unroll
        for (uint32_t p = 0; p < 2; ++p) {
          const uint32_t q = t + p * kTopKThreads;  // pair index
          const uint32_t i = 2 * q - (q & (half - 1));
          const uint32_t j = i + half;
          const uint64_t a = keys[i], b = keys[j];
          const bool desc = (i & size) == 0;
          if (desc ? a < b : a > b) {
            keys[i] = b;
            keys[j] = a;
          }
        }
        __syncthreads();
      }
    }
    uint64_t big_m = red[0];
    for (uint32_t w = 1; w < kTopKThreads / 64; ++w) big_m = red[w] > big_m ? red[w] : big_m;
    // g = the number of sorted keys above M (keys at or below M, zeros included, follow them).
#pragma unroll
    for (uint32_t p = 0; p < kTopKKeep; ++p) {
      const uint32_t i = kTopKKeep * t + p;
      if (keys[i] > big_m && (i + 1 == kTopKKeys || keys[i + 1] <= big_m)) taken = i + 1;
    }
    __syncthreads();
    const uint32_t g = taken;
    const uint32_t take = min(g, k - got);
    for (uint32_t i = t; i < take; i += kTopKThreads) {
      const uint64_t key = keys[i];
      const uint32_t id = ~static_cast<uint32_t>(key & 0xffffffffu);
      ol[got + i] = row[id];
      oi[got + i] = static_cast<int32_t>(id);
    }
    got += take;
    // Done at k keys, or when no thread kept four (every remaining key was taken).
    if (got == k || big_m == 0) break;
    bound = keys[take - 1];
    __syncthreads();
  }
  for (uint32_t i = got + t; i < k; i += kTopKThreads) {  // fewer than k non-NaN values
    ol[i] = 0.0f;
    oi[i] = -1;
  }
}

// ---- Whole-row sort (top_k 0, or more than kMaxTopK candidates) -------------------------------
// sampler.cpp:105-118 sorts every id by logit when top_k keeps them all. One workgroup per row
// runs a stable LSD radix sort of 32-bit keys, four passes of 8-bit digits, in the order the
// top-k kernel keeps: larger values first, equal values (-0 equal to +0) by ascending index,
// NaN last with id -1. The key is the complement of the order-preserving map of argmax_key, so
// an ascending sort of keys is a descending sort of values; the input order is ascending index
// and every pass is stable, so ties keep it.
//
// The four digit histograms come from one sweep (the keys are the same in every pass). A pass
// takes the row 1024 keys at a time in index order: lanes of a wave that share a digit find each
// other with eight ballots, a lane's rank among them is the popcount of the lower ones, the
// first of them writes the group's count into a [wave][digit] table, and 256 threads turn each
// digit's column into offsets (the digit's running base plus the earlier waves' counts). Two
// tables alternate, so the one the next group of keys counts into is cleared while this one is
// read. Passes ping-pong between the workspace and the output arrays: row -> work -> out ->
// work -> out, the last pass writing the original values (signed zeros kept) and ids.

constexpr uint32_t kSortThreads = 1024;
constexpr uint32_t kSortWaves = kSortThreads / 64;
constexpr uint32_t kSortNaN = 0xffffffffu;

__device__ __forceinline__ uint32_t sort_key(float v) {
  if (v != v) return kSortNaN;  // no other value maps there: only a NaN has order 0
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0;
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ~ord;
}

// The valid lanes of this wave whose digit equals this lane's.
__device__ __forceinline__ uint64_t same_digit_lanes(uint32_t d, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (uint32_t b = 0; b < 8; ++b) {
    const bool bit = ((d >> b) & 1u) != 0;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

__global__ __launch_bounds__(kSortThreads) void sort_rows_kernel(const float* __restrict__ x, uint32_t n,
                                                                 size_t stride, uint32_t* __restrict__ work_key,
                                                                 int32_t* __restrict__ work_id,
                                                                 float* __restrict__ out_logit,
                                                                 int32_t* __restrict__ out_id) {
  __shared__ uint32_t hist[4][256];
  __shared__ uint32_t offs[2][kSortWaves][256];
  const uint32_t r = blockIdx.x;
  const uint32_t t = threadIdx.x;
  const uint32_t w = t >> 6;
  const uint64_t below = (1ull << (t & 63)) - 1;
  const float* row = x + static_cast<size_t>(r) * stride;
  uint32_t* ak = work_key + static_cast<size_t>(r) * n;
  int32_t* ai = work_id + static_cast<size_t>(r) * n;
  // The output arrays hold keys between passes; every access inside the kernel is as uint32.
  uint32_t* bk = reinterpret_cast<uint32_t*>(out_logit) + static_cast<size_t>(r) * n;
  int32_t* bi = out_id + static_cast<size_t>(r) * n;

  for (uint32_t i = t; i < 4 * 256; i += kSortThreads) (&hist[0][0])[i] = 0;
  for (uint32_t i = t; i < 2 * kSortWaves * 256; i += kSortThreads) (&offs[0][0][0])[i] = 0;
  __syncthreads();
  for (uint32_t j0 = 0; j0 < n; j0 += kSortThreads) {
    const uint32_t j = j0 + t;
    const bool valid = j < n;
    const uint32_t k = valid ? sort_key(row[j]) : 0;
#pragma unroll
    for (uint32_t p = 0; p < 4; ++p) {
      const uint32_t d = (k >> (8 * p)) & 255u;
      const uint64_t peers = same_digit_lanes(d, valid);
      if (valid && (peers & below) == 0) atomicAdd(&hist[p][d], static_cast<uint32_t>(__popcll(peers)));
    }
  }
  __syncthreads();
  if (w < 4) {  // exclusive scan of pass w's histogram, four bins a lane
    const uint32_t lane = t & 63;
    uint32_t c[4];
    uint32_t s = 0;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      c[i] = hist[w][4 * lane + i];
      s += c[i];
    }
    uint32_t inc = s;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(inc, off, 64);
      if (lane >= off) inc += o;
    }
    uint32_t e = inc - s;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      hist[w][4 * lane + i] = e;
      e += c[i];
    }
  }
  __syncthreads();

  uint32_t buf = 0;  // offs[buf] is clear when a group of keys starts
  for (uint32_t pass = 0; pass < 4; ++pass) {
    const uint32_t shift = 8 * pass;
    const uint32_t* sk = pass == 2 ? bk : ak;
    const int32_t* si = pass == 2 ? bi : ai;
    uint32_t* dk = (pass & 1u) ? bk : ak;
    int32_t* di = (pass & 1u) ? bi : ai;
    uint32_t base = t < 256 ? hist[pass][t] : 0;  // digit t's next free slot
    for (uint32_t j0 = 0; j0 < n; j0 += kSortThreads, buf ^= 1u) {
      const uint32_t j = j0 + t;
      const bool valid = j < n;
      uint32_t k = kSortNaN;
      int32_t id = -1;
      if (valid) {
        if (pass == 0) {
          k = sort_key(row[j]);
          id = static_cast<int32_t>(j);
        } else {
          k = sk[j];
          id = si[j];
        }
      }
      const uint32_t d = (k >> shift) & 255u;
      const uint64_t peers = same_digit_lanes(d, valid);
      const uint32_t rank = static_cast<uint32_t>(__popcll(peers & below));
      if (valid && rank == 0) offs[buf][w][d] = static_cast<uint32_t>(__popcll(peers));
      __syncthreads();
      if (t < 256) {
        uint32_t c[kSortWaves];
#pragma unroll
        for (uint32_t v = 0; v < kSortWaves; ++v) c[v] = offs[buf][v][t];
        uint32_t s = base;
#pragma unroll
        for (uint32_t v = 0; v < kSortWaves; ++v) {
          offs[buf][v][t] = s;
          s += c[v];
          offs[buf ^ 1u][v][t] = 0;  // read by the previous group, which every thread has finished
        }
        base = s;
      }
      __syncthreads();
      if (valid) {
        const uint32_t at = offs[buf][w][d] + rank;
        if (pass == 3) {
          const bool nan = k == kSortNaN;
          dk[at] = nan ? 0u : __float_as_uint(row[id]);
          di[at] = nan ? -1 : id;
        } else {
          dk[at] = k;
          di[at] = id;
        }
      }
    }
    __syncthreads();  // this pass's stores before the next pass's loads (one workgroup)
  }
}

}  // namespace

int sort_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, void* work, float* out_logit,
                     int32_t* out_id) {
  if (n_rows == 0) return kOk;
  if (n == 0) return fail(kInvalidArgument, "sort_rows: empty rows");
  if (n_rows > 65535) return fail(kInvalidArgument, "sort_rows: %u rows exceed one launch's 65535", n_rows);
  auto* key = static_cast<uint32_t*>(work);
  auto* id = reinterpret_cast<int32_t*>(key + static_cast<size_t>(n_rows) * n);
  hipLaunchKernelGGL(sort_rows_kernel, dim3(n_rows), dim3(kSortThreads), 0, stream(), x, n, stride, key, id, out_logit,
                     out_id);
  return check_launch("sort_rows");
}

int topk_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, uint32_t k, float* out_logit,
                     int32_t* out_id) {
  if (n_rows == 0) return kOk;
  if (n == 0 || k == 0 || k > kMaxTopK) return fail(kInvalidArgument, "topk: k %u of %u values (k in 1..%u)", k, n, kMaxTopK);
  if (n_rows > 65535) return fail(kInvalidArgument, "topk: %u rows exceed one launch's 65535", n_rows);
  hipLaunchKernelGGL(topk_rows_kernel, dim3(n_rows), dim3(kTopKThreads), 0, stream(), x, n, stride, k, out_logit,
                     out_id);
  return check_launch("topk");
}

int repeat_penalty_launch(float* x, uint32_t n, uint32_t n_rows, size_t stride, const int32_t* recent,
                          const uint32_t* recent_len, size_t recent_stride, float penalty) {
  if (n_rows == 0 || recent_stride == 0) return kOk;
  hipLaunchKernelGGL(repeat_penalty_kernel, dim3(n_rows), dim3(256), 0, stream(), x, n, stride, recent, recent_len,
                     recent_stride, penalty);
  return check_launch("repeat_penalty");
}

size_t argmax_scratch_words(uint32_t n_rows) { return static_cast<size_t>(n_rows) * kParts; }

int argmax_rows_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, uint64_t* scratch, int32_t* out) {
  if (n_rows == 0) return kOk;
  if (n == 0) return fail(kInvalidArgument, "argmax: empty rows");
  if (n_rows > 65535) return fail(kInvalidArgument, "argmax: %u rows exceed one launch's 65535", n_rows);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(kParts, n_rows), dim3(kThreads), 0, stream(), x, n, stride, scratch);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(n_rows), dim3(64), 0, stream(), x, stride, scratch, out);
  return check_launch("argmax");
}

// ---- The allocation-free greedy choice -------------------------------------------------------
// The partial keys of argmax_rows_launch in a fixed device array instead of a caller workspace,
// for callers that cannot allocate. Each GPU holds its own copy for the life of the process;
// host code never passes the array's name to a kernel (in host code it is only a stand-in for
// the symbol): it passes the address hipGetSymbolAddress returned for the current device. Every
// slot a call reads is written earlier in the same call, so nothing needs clearing; two calls
// that overlap on one GPU share the array and race.
static __device__ __align__(256) uint64_t scratch[kArgmaxNoAllocRows * kParts];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint64_t* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int argmax_noalloc_setup() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(kHipError, "argmax (no allocation): hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(kInvalidArgument, "argmax (no allocation): device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] != nullptr) return kOk;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return fail(kHipError, "argmax (no allocation): hipGetSymbolAddress: %s", hipGetErrorString(e));
  g_scratch_ptr[dev] = static_cast<uint64_t*>(p);
  return kOk;
}

int argmax_rows_noalloc_launch(const float* x, uint32_t n, uint32_t n_rows, size_t stride, int32_t* out) {
  if (n_rows > kArgmaxNoAllocRows)
    return fail(kInvalidArgument, "argmax (no allocation): %u rows exceed the fixed scratch's %u", n_rows,
                kArgmaxNoAllocRows);
  const int rc = argmax_noalloc_setup();  // a lookup after the first call on this device
  if (rc != kOk) return rc;
  int dev = 0;
  (void)hipGetDevice(&dev);
  return argmax_rows_launch(x, n, n_rows, stride, g_scratch_ptr[dev], out);
}

}  // namespace axon_hip
