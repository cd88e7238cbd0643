// Measurements behind the decode-step kernel's design, as a program of its own (not part of the
// libraries): what a hand-off between workgroups costs on this GPU, how that cost grows with
// the number of workgroups whose words a reader waits for, how long a chain of dependent adds
// takes per step, and what LDS-DMA pulls per workgroup. Every wait is bounded: a wait that runs
// out stops its workgroup and the others' waits then run out too, so every grid drains.
//
//   fabric_probe            prints one line per measurement
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                  \
  do {                                                                            \
    const hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "fabric_probe: %s: %s\n", #x, hipGetErrorString(e_)); \
      std::exit(1);                                                               \
    }                                                                             \
  } while (0)

namespace {

constexpr unsigned kSpins = 1u << 14;  // polls of one word before a wait gives up

__device__ __forceinline__ uint64_t ld_dev(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ping-pong of one tagged word each way between workgroups a and b (one lane each).
__global__ void ping_pong(uint64_t* w, int a, int b, int n, unsigned* xcc, long long* out) {
  unsigned id;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(id));
  if (threadIdx.x == 0) xcc[blockIdx.x] = id & 0xfu;
  if ((static_cast<int>(blockIdx.x) != a && static_cast<int>(blockIdx.x) != b) || threadIdx.x != 0) return;
  uint64_t* to_b = w;
  uint64_t* to_a = w + 32;  // another 256-byte line
  uint64_t* dead = w + 64;
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  int i = 0;
  for (; i < n; ++i) {
    const bool is_a = static_cast<int>(blockIdx.x) == a;
    if (is_a) st_dev(to_b, 2ull * i + 1);
    const uint64_t* src = is_a ? to_a : to_b;
    const uint64_t want = is_a ? 2ull * i + 2 : 2ull * i + 1;
    unsigned s = 0;
    while (ld_dev(src) != want) {
      if (++s > kSpins || ld_dev(dead) != 0) {
        st_dev(dead, 1);
        i = n + 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!is_a && i <= n) st_dev(to_a, 2ull * i + 2);
  }
  const long long t1 = __builtin_amdgcn_s_memrealtime();
  if (static_cast<int>(blockIdx.x) == a) {
    out[0] = t1 - t0;
    out[1] = i;
  }
}

// All-to-all rounds: workgroups w < writers write 8 tagged words (the decode step's x rows of one
// workgroup), then every workgroup's 256 threads poll them, thread t the 8 words of writer t (as
// the step kernel's norm reads x). Two buffers alternate by round.
__global__ __launch_bounds__(256) void all_to_all(uint64_t* buf, int rounds, int writers, int* fails,
                                                  long long* out) {
  __shared__ int bad;
  const int w = blockIdx.x, t = threadIdx.x;
  if (t == 0) bad = 0;
  __syncthreads();
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  float acc = 0.0f;
  for (int r = 0; r < rounds; ++r) {
    uint64_t* b = buf + (r & 1) * 2048;
    const uint32_t tag = r + 1;
    if (w < writers && t < 8) st_dev(b + w * 8 + t, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(1.0f));
    bool ok = true;
    if (t < writers) {
      uint64_t u[8];
      for (unsigned s = 0;; ++s) {
        bool all = true;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          u[i] = ld_dev(b + t * 8 + i);
          all &= static_cast<uint32_t>(u[i] >> 32) == tag;
        }
        if (all) break;
        if (s > kSpins) {
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += __uint_as_float(static_cast<uint32_t>(u[i]));
    }
    if (!ok) bad = 1;
    __syncthreads();
    if (bad) break;
  }
  const long long t1 = __builtin_amdgcn_s_memrealtime();
  if (t == 0) {
    out[w] = t1 - t0;
    if (bad) atomicAdd(fails, 1);
  }
  if (acc == -1.0f) out[0] = 0;  // keeps the reads
}

// Dependent adds: from registers, and fed by 16-byte LDS reads (16 reads, then 64 adds).
__global__ void chain_registers(const float* in, float* out, int n, long long* t) {
  float v[16];
  for (int i = 0; i < 16; ++i) v[i] = in[threadIdx.x + 64 * i];
  float acc = 0.0f;
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int j = 0; j < n; j += 16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += v[i];
    asm volatile("" : "+v"(v[0]));
  }
  const long long t1 = __builtin_amdgcn_s_memrealtime();
  out[threadIdx.x] = acc;
  if (threadIdx.x == 0) *t = t1 - t0;
}
__global__ void chain_lds(const float* in, float* out, int n, long long* t) {
  __shared__ float pr[64 * 516];
  for (int i = threadIdx.x; i < 64 * 516; i += blockDim.x) pr[i] = in[i % 1024];
  __syncthreads();
  const int c = threadIdx.x % 64;
  float acc = 0.0f;
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int j = 0; j < n; j += 64) {
    float4 q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i] = *reinterpret_cast<const float4*>(&pr[c * 516 + ((j + 4 * i) & 511)]);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc += q[i].x;
      acc += q[i].y;
      acc += q[i].z;
      acc += q[i].w;
    }
  }
  const long long t1 = __builtin_amdgcn_s_memrealtime();
  out[threadIdx.x] = acc;
  if (threadIdx.x == 0) *t = t1 - t0;
}

// LDS-DMA: four waves per workgroup pull `per_wg` bytes into a 64 KB LDS ring, 1 KB per copy,
// each wave keeping up to 16 copies in flight.
typedef int I4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void dma_pull(const uint8_t* src, uint32_t per_wg, long long* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
  const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint64_t a = reinterpret_cast<uint64_t>(src + static_cast<size_t>(blockIdx.x) * per_wg);
  const I4 rsrc = {__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)),
                   __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu)),
                   __builtin_amdgcn_readfirstlane(static_cast<int>(per_wg)), 0x00020000};
  const uint32_t ring_lds = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)ring));
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t k = 0;
  for (uint32_t c = wv; c < per_wg / 1024; c += 4, ++k) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(ring_lds + (c % 64) * 1024);
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 : : "v"(c * 1024 + lane * 16), "s"(rsrc), "s"(lds) : "memory");
    if (k >= 15) asm volatile("s_waitcnt vmcnt(15)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const long long t1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) out[blockIdx.x] = t1 - t0;
}

double ns_of(long long ticks, double hz) { return static_cast<double>(ticks) * 1e9 / hz; }

}  // namespace

int main() {
  int dev = 0, khz = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const double hz = khz * 1e3;  // s_memrealtime's rate
  const int grid = cus < 256 ? cus : 256;
  uint64_t* words = nullptr;
  unsigned* xcc = nullptr;
  long long* out = nullptr;
  int* fails = nullptr;
  CHECK(hipMalloc(&words, 4096 * 8));
  CHECK(hipMalloc(&xcc, 256 * 4));
  CHECK(hipMalloc(&out, 512 * 8));
  CHECK(hipMalloc(&fails, 4));

  // 1. Ping-pong.
  const int n_pp = 2000;
  for (const auto& pr : std::vector<std::pair<int, int>>{{0, 1}, {0, 8}, {0, 4}, {3, 11}}) {
    if (pr.second >= grid) continue;
    CHECK(hipMemset(words, 0, 4096 * 8));
    CHECK(hipMemset(out, 0, 16));
    hipLaunchKernelGGL(ping_pong, dim3(grid), dim3(64), 0, 0, words, pr.first, pr.second, n_pp, xcc, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    long long h[2];
    std::vector<unsigned> x(grid);
    CHECK(hipMemcpy(h, out, 16, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(x.data(), xcc, grid * 4, hipMemcpyDeviceToHost));
    std::printf("ping-pong wg %d (XCD %u) <-> wg %d (XCD %u): round trip %.0f ns%s\n", pr.first, x[pr.first], pr.second,
                x[pr.second], ns_of(h[0], hz) / n_pp, h[1] == n_pp ? "" : " (a wait ran out)");
  }

  // 2. All-to-all rounds against the number of writers, every workgroup polling.
  const int rounds = 200;
  for (int writers : {32, 64, 128, 256}) {
    if (writers > grid) continue;
    CHECK(hipMemset(words, 0, 4096 * 8));
    CHECK(hipMemset(fails, 0, 4));
    hipLaunchKernelGGL(all_to_all, dim3(grid), dim3(256), 0, 0, words, rounds, writers, fails, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    std::vector<long long> h(grid);
    int f = 0;
    CHECK(hipMemcpy(h.data(), out, grid * 8, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(&f, fails, 4, hipMemcpyDeviceToHost));
    long long mx = 0;
    for (long long v : h) mx = v > mx ? v : mx;
    std::printf("all-to-all: %3d writers x 8 words, %d readers: %.0f ns per round%s\n", writers, grid,
                ns_of(mx, hz) / rounds, f ? " (a wait ran out)" : "");
  }

  // 3. Dependent adds.
  float *fin = nullptr, *fout = nullptr;
  CHECK(hipMalloc(&fin, 1 << 20));
  CHECK(hipMalloc(&fout, 1 << 20));
  std::vector<float> ones(1 << 18, 1.0f);
  CHECK(hipMemcpy(fin, ones.data(), 1 << 20, hipMemcpyHostToDevice));
  const int n_chain = 4096;
  for (int which = 0; which < 2; ++which) {
    long long tt = 0;
    for (int r = 0; r < 3; ++r) {
      if (which == 0) hipLaunchKernelGGL(chain_registers, dim3(1), dim3(64), 0, 0, fin, fout, n_chain, out);
      else hipLaunchKernelGGL(chain_lds, dim3(1), dim3(64), 0, 0, fin, fout, n_chain, out);
      CHECK(hipGetLastError());
      CHECK(hipDeviceSynchronize());
    }
    CHECK(hipMemcpy(&tt, out, 8, hipMemcpyDeviceToHost));
    std::printf("dependent adds (%s): %.2f ns per add\n", which == 0 ? "registers" : "16-byte LDS reads",
                ns_of(tt, hz) / n_chain);
  }

  // 4. LDS-DMA pull per workgroup.
  const uint32_t per_wg = 4u << 20;
  uint8_t* src = nullptr;
  CHECK(hipMalloc(&src, static_cast<size_t>(per_wg) * grid));
  CHECK(hipMemset(src, 1, static_cast<size_t>(per_wg) * grid));
  CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(dma_pull), hipFuncAttributeMaxDynamicSharedMemorySize, 65536));
  for (int wgs : {1, 64, grid}) {
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(dma_pull, dim3(wgs), dim3(256), 65536, 0, src, per_wg, out);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipDeviceSynchronize());
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::vector<long long> h(wgs);
    CHECK(hipMemcpy(h.data(), out, wgs * 8, hipMemcpyDeviceToHost));
    long long mx = 0;
    for (long long v : h) mx = v > mx ? v : mx;
    std::printf("LDS-DMA pull, %3d workgroups (64 KB in flight each): %.1f GB/s per workgroup, %.0f GB/s in all\n", wgs,
                per_wg / (ns_of(mx, hz) * 1e-9) / 1e9, static_cast<double>(per_wg) * wgs / (ms * 1e-3) / 1e9);
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
  }
  CHECK(hipFree(src));
  CHECK(hipFree(fin));
  CHECK(hipFree(fout));
  CHECK(hipFree(words));
  CHECK(hipFree(xcc));
  CHECK(hipFree(out));
  CHECK(hipFree(fails));
  return 0;
}
