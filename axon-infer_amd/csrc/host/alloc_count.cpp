// Allocation counter of the host library (libaxon_host.so): its own global operator new and
// delete count each allocation and forward to malloc and free, kept local to the library by the
// link's version script (alloc_count.map), as libaxon_hip.so does for its own code
// (hip/alloc_count.hip). Tests use it to pin the reference's "a forward pass performs no heap
// allocation" (tests/unit/alloc_counter.cpp:33-46, tests/unit/test_model_forward.cpp:119-128).
#include "axon_model.h"

#include <atomic>
#include <cstdlib>
#include <new>

namespace {
std::atomic<size_t> g_allocations{0};
void* counted(size_t size) {
  g_allocations.fetch_add(1, std::memory_order_relaxed);
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

extern "C" size_t axon_model_host_allocations(void) { return g_allocations.load(std::memory_order_relaxed); }
