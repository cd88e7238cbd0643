// Allocation counters of this library's host code, for tests that pin the reference's "a forward
// pass performs no heap allocation" (tests/unit/alloc_counter.cpp:33-46,
// tests/unit/test_model_forward.cpp:119-128). The library's own global operator new and delete
// count each allocation and forward to malloc and free; the link's version script keeps them
// local to the library (alloc_count.map), so they serve its code only and the HIP runtime and
// the rest of the process keep theirs. Device allocations (axon_hip_malloc, axon_hip_host_malloc,
// axon_hip_event_create) are counted where they are made, in capi.hip.
#include "axon_hip.h"

#include <atomic>
#include <cstdlib>
#include <new>

namespace axon_hip {
std::atomic<size_t> g_host_allocations{0};
std::atomic<size_t> g_device_allocations{0};
}  // namespace axon_hip

namespace {
void* counted(size_t size) {
  axon_hip::g_host_allocations.fetch_add(1, std::memory_order_relaxed);
  return std::malloc(size == 0 ? 1 : size);
}
}  // namespace

void* operator new(size_t size) {
  void* p = counted(size);
  if (p == nullptr) throw std::bad_alloc();
  return p;
}
void* operator new[](size_t size) {
  void* p = counted(size);
  if (p == nullptr) throw std::bad_alloc();
  return p;
}
void* operator new(size_t size, const std::nothrow_t&) noexcept { return counted(size); }
void* operator new[](size_t size, const std::nothrow_t&) noexcept { return counted(size); }
void operator delete(void* p) noexcept { std::free(p); }
void operator delete[](void* p) noexcept { std::free(p); }
void operator delete(void* p, size_t) noexcept { std::free(p); }
void operator delete[](void* p, size_t) noexcept { std::free(p); }

extern "C" void axon_hip_allocation_counts(size_t* host_new, size_t* device) {
  if (host_new != nullptr) *host_new = axon_hip::g_host_allocations.load(std::memory_order_relaxed);
  if (device != nullptr) *device = axon_hip::g_device_allocations.load(std::memory_order_relaxed);
}
