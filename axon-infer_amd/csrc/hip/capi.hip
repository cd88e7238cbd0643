// The C ABI of the hip table (include/axon_hip.h): device detection and lifecycle, and one
// thin adapter per entry that validates sizes on the host, then launches the kernels of this
// library on the library stream. No entry falls back to the CPU.
#include "common.h"
#include "decode_step.h"
#include "elementwise.h"
#include "matmul_float.h"
#include "matvec.h"

#include "../../../include/axon_hip.h"

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

namespace axon_hip {

extern std::atomic<size_t> g_device_allocations;  // alloc_count.hip

namespace {

thread_local char g_error[512] = "";
hipStream_t g_stream = nullptr;
int g_device = -1;
std::mutex g_init_mutex;

int hip_fail(hipError_t e, const char* what) {
  return fail(kHipError, "%s: %s", what, hipGetErrorString(e));
}

int init_device(int device) {
  std::lock_guard<std::mutex> lock(g_init_mutex);
  if (g_device == device && g_stream != nullptr) return kOk;
  if (g_stream != nullptr) return fail(kInvalidArgument, "axon_hip_init: already bound to device %d", g_device);
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    (void)hipGetLastError();
    return fail(kNoDevice, "hip: no GPU visible to this process");
  }
  if (device < 0 || device >= count) return fail(kInvalidArgument, "hip: device %d of %d", device, count);
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(kNoDevice, "hip: device %d is %s; this table is built for gfx950 (MI355X) only", device,
                prop.gcnArchName);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
  g_device = device;
  // The fixed scratch of the allocation-free entry, looked up once with this device current. It
  // serves that one optional entry only: a failed lookup is reported by the entry itself (which
  // retries it), not by the library's initialisation.
  if (argmax_noalloc_setup() != kOk) (void)hipGetLastError();
  return kOk;
}

int ready() {
  if (g_stream != nullptr) return kOk;
  return init_device(0);
}

#define AXON_READY()                 \
  do {                               \
    const int rc_ = ready();         \
    if (rc_ != kOk) return rc_;      \
  } while (0)

bool fits_u32(size_t v) { return v <= 0xffffffffull; }

// The Q8_0-activation path: one or two rows on the decode matvec or the dot4 matvec, the
// few-rows MFMA kernel (every segment in one launch) up to 64 rows (from 3 rows where the dot4
// kernel holds them poorly), the tile MFMA kernel (every segment in one launch, 64-row tiles)
// beyond, and from 33 rows on matrices wide enough for 128 of its tiles (their weights read
// once, not up to four times); rows whose bases or lengths do not suit their dword loads take
// the staged 64 x 64 MFMA tiles or the dot4 groups. All of them give the same bits for a row.
int q8_matmul(int type, const void* xq, size_t n_rows, size_t n_in, size_t n_seg, const void* const* w,
              float* const* y, const size_t* n_out, const size_t* y_stride, int accumulate) {
  if (n_in % kQK != 0) return fail(kInvalidArgument, "quantized matmul: n_in %zu is not a multiple of 32", n_in);
  if (type != Q8_0 && type != Q4_0 && type != Q4_1) return fail(kUnsupported, "matmul_q8: weight type %d", type);
  if (n_seg < 1 || n_seg > 3) return fail(kInvalidArgument, "matmul_q8: %zu segments", n_seg);
  if (!fits_u32(n_rows) || !fits_u32(n_in)) return fail(kInvalidArgument, "matmul_q8: sizes too large");
  for (size_t s = 0; s < n_seg; ++s) {
    if (!fits_u32(n_out[s]) || !fits_u32(y_stride[s])) return fail(kInvalidArgument, "matmul_q8: sizes too large");
    if (n_rows > 1 && y_stride[s] < n_out[s]) return fail(kInvalidArgument, "matmul_q8: y_stride %zu < n_out %zu", y_stride[s], n_out[s]);
  }
  if (n_rows == 0) return kOk;
  const uint32_t nb = static_cast<uint32_t>(n_in / kQK);
  const size_t xrow = static_cast<size_t>(nb) * kBytesQ8_0;
  // Fewer rows also take the MFMA kernels where the dot4 kernel below holds them poorly:
  // three or four rows of 8192 inputs and more (C4 down 2048 x 8192: 25 / 34 us at 3 / 4 rows
  // on the dot4 kernel, 17 us on the rows kernel) or of a matrix wide enough for the decode
  // tile (16384 x 2048 at 4 rows 14.4 -> 11.5 us, 128256 x 2048 at 3 / 4 rows 59 / 65 ->
  // 53 / 46 us), and rows beyond what one dot4 launch holds, each further launch reading the
  // matrix again (4096 x 14336 at 2 rows: 54 us).
  size_t wg64 = 0;
  for (size_t s = 0; s < n_seg; ++s) wg64 += (n_out[s] + 63) / 64;
  if (n_rows >= 5 || (n_rows >= 3 && (nb >= 256 || wg64 >= 256)) || n_rows > matvec_q8_max_rows(type, nb)) {
    MatvecArgs a{};
    for (size_t s = 0; s < n_seg; ++s) {
      a.seg[s] = MatvecSeg{static_cast<const uint8_t*>(w[s]), y[s], static_cast<uint32_t>(n_out[s]),
                           static_cast<uint32_t>(y_stride[s]), 0};
    }
    a.n_seg = static_cast<int>(n_seg);
    a.xq = static_cast<const uint8_t*>(xq);
    a.nb = nb;
    a.m = static_cast<uint32_t>(n_rows);
    a.accumulate = accumulate;
    if (n_rows > kRowsMaxM || matmul_q8_tile_fills(a)) {
      if (matmul_q8_rows_fits(type, a, true)) return matmul_q8_tile_launch(type, a);
    } else if (matmul_q8_rows_fits(type, a)) {
      return matmul_q8_rows_launch(type, a);
    }
  }
  if (n_rows >= 16) {
    for (size_t s = 0; s < n_seg; ++s) {
      MatvecArgs a{};
      a.seg[0] = MatvecSeg{static_cast<const uint8_t*>(w[s]), y[s], static_cast<uint32_t>(n_out[s]),
                           static_cast<uint32_t>(y_stride[s]), 0};
      a.n_seg = 1;
      a.xq = static_cast<const uint8_t*>(xq);
      a.nb = nb;
      a.m = static_cast<uint32_t>(n_rows);
      a.accumulate = accumulate;
      const int rc = matmul_q8_mfma_launch(type, a);
      if (rc != kOk) return rc;
    }
    return kOk;
  }
  // One or two rows of a matrix narrower than that: the decode matvec (weights streamed through
  // LDS by DMA), where LDS holds the rows' blocks; the same bits as the dot4 kernel (2048 x 8192
  // at 1 / 2 rows 8.6 / 10.1 -> 6.6 / 8.1 us, 2048 x 2048 4.3 -> 3.9 us).
  if (n_rows <= 2 && wg64 < 256 && matvec_fused_fits(type, kInQ8, static_cast<uint32_t>(n_rows), nb, false)) {
    FusedArgs f{};
    f.n_seg = static_cast<int>(n_seg);
    for (size_t s = 0; s < n_seg; ++s) {
      f.w[s] = static_cast<const uint8_t*>(w[s]);
      f.n_out[s] = static_cast<uint32_t>(n_out[s]);
      f.y[s] = y[s];
      f.y_stride[s] = static_cast<uint32_t>(y_stride[s]);
    }
    f.nb = nb;
    f.m = static_cast<uint32_t>(n_rows);
    f.in_mode = kInQ8;
    f.xq = static_cast<const uint8_t*>(xq);
    f.out_mode = accumulate ? kOutAdd : kOutStore;
    const int rc = matvec_fused_launch(type, f);
    if (rc != kUnsupported) return rc;
  }
  const uint32_t group = matvec_q8_max_rows(type, nb);
  for (size_t m0 = 0; m0 < n_rows; m0 += group) {
    const uint32_t mm = static_cast<uint32_t>(std::min<size_t>(group, n_rows - m0));
    MatvecArgs a{};
    for (size_t s = 0; s < n_seg; ++s) {
      a.seg[s] = MatvecSeg{static_cast<const uint8_t*>(w[s]), y[s] + m0 * y_stride[s], static_cast<uint32_t>(n_out[s]),
                           static_cast<uint32_t>(y_stride[s]), 0};
    }
    a.n_seg = static_cast<int>(n_seg);
    a.xq = static_cast<const uint8_t*>(xq) + m0 * xrow;
    a.nb = nb;
    a.m = mm;
    a.accumulate = accumulate;
    const int rc = matvec_q8_launch(type, a);
    if (rc != kOk) return rc;
  }
  return kOk;
}

int q8_rows(int type, const void* w, const void* xq, float* y, size_t n_rows, size_t n_out, size_t n_in,
            size_t y_stride) {
  AXON_READY();
  const void* ws[1] = {w};
  float* ys[1] = {y};
  const size_t no[1] = {n_out};
  const size_t st[1] = {y_stride};
  return q8_matmul(type, xq, n_rows, n_in, 1, ws, ys, no, st, 0);
}

int float_rows(int type, const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
               size_t y_stride) {
  AXON_READY();
  if (!fits_u32(n_rows) || !fits_u32(n_out) || !fits_u32(n_in) || !fits_u32(y_stride))
    return fail(kInvalidArgument, "matmul: sizes too large");
  if (n_rows > 1 && y_stride < n_out) return fail(kInvalidArgument, "matmul: y_stride %zu < n_out %zu", y_stride, n_out);
  return matmul_float_launch(type, w, x, y, static_cast<uint32_t>(n_rows), static_cast<uint32_t>(n_out),
                             static_cast<uint32_t>(n_in), static_cast<uint32_t>(y_stride));
}

int q6k_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in, size_t y_stride) {
  AXON_READY();
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k: n_in %zu is not a multiple of 256", n_in);
  if (!fits_u32(n_rows) || !fits_u32(n_out) || !fits_u32(n_in) || !fits_u32(y_stride))
    return fail(kInvalidArgument, "matmul_q6_k: sizes too large");
  if (n_rows > 1 && y_stride < n_out) return fail(kInvalidArgument, "matmul_q6_k: y_stride %zu < n_out %zu", y_stride, n_out);
  MatvecArgs a{};
  a.seg[0] = MatvecSeg{static_cast<const uint8_t*>(w), y, static_cast<uint32_t>(n_out), static_cast<uint32_t>(y_stride), 0};
  a.n_seg = 1;
  a.xq = reinterpret_cast<const uint8_t*>(x);
  a.nb = static_cast<uint32_t>(n_in / kQKK);
  a.m = static_cast<uint32_t>(n_rows);
  return matvec_q6k_launch(a, static_cast<uint32_t>(n_in));
}

int attention_heads(const float* q, const void* k, const void* v, float* out, float* scores, size_t n_q,
                    size_t n_past, size_t n_head, size_t n_kv, size_t head_dim, float scale, size_t hb, size_t he,
                    int f16) {
  AXON_READY();
  if (!fits_u32(n_q) || !fits_u32(n_past + n_q) || !fits_u32(n_head) || !fits_u32(head_dim))
    return fail(kInvalidArgument, "attention: sizes too large");
  // One cache for all rows; K and V are separate arrays, so address both from the K base.
  AttnArgs a{};
  a.q = q;
  a.out = out;
  a.q_stride = static_cast<uint32_t>(n_head * head_dim);
  a.out_stride = a.q_stride;
  a.kv = k;
  const ptrdiff_t elem = f16 ? 2 : 4;
  a.k_off_c = 0;
  a.v_off_c = (static_cast<const char*>(v) - static_cast<const char*>(k)) / elem;
  if ((static_cast<const char*>(v) - static_cast<const char*>(k)) % elem != 0)
    return fail(kInvalidArgument, "attention: v_cache is not element-aligned with k_cache");
  a.n_past = static_cast<int32_t>(n_past);
  a.n_head = static_cast<uint32_t>(n_head);
  a.n_kv = static_cast<uint32_t>(n_kv);
  a.head_dim = static_cast<uint32_t>(head_dim);
  a.head_begin = static_cast<uint32_t>(hb);
  a.head_end = static_cast<uint32_t>(he);
  a.scale = scale;
  a.f16 = f16;
  a.scratch = scores;
  a.max_vis = static_cast<uint32_t>(n_past + n_q);
  return attention_launch(a, static_cast<uint32_t>(n_q));
}

}  // namespace

hipStream_t stream() { return g_stream; }

namespace {
thread_local hipEvent_t g_probe_start = nullptr;
thread_local hipEvent_t g_probe_stop = nullptr;
}  // namespace

void take_probe(hipEvent_t* start, hipEvent_t* stop) {
  *start = g_probe_start;
  *stop = g_probe_stop;
  g_probe_start = g_probe_stop = nullptr;
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  return kOk;
}

}  // namespace axon_hip

using namespace axon_hip;

extern "C" {

// ---- lifecycle ------------------------------------------------------------------------------

int axon_hip_device_count(int* count) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  *count = n;
  return kOk;
}

int axon_hip_init(int device) { return init_device(device); }

int axon_hip_device_arch(char* buf, size_t len) {
  AXON_READY();
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, g_device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  std::snprintf(buf, len, "%s", prop.gcnArchName);
  return kOk;
}

const char* axon_hip_last_error(void) { return g_error; }

int axon_hip_malloc(void** ptr, size_t bytes) {
  AXON_READY();
  *ptr = nullptr;
  if (bytes == 0) return kOk;
  const hipError_t e = hipMalloc(ptr, bytes);
  if (e == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    return fail(kOutOfMemory, "hipMalloc: %zu bytes: out of device memory", bytes);
  }
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  g_device_allocations.fetch_add(1, std::memory_order_relaxed);
  return kOk;
}

int axon_hip_free(void* ptr) {
  if (ptr == nullptr) return kOk;
  const hipError_t e = hipFree(ptr);
  return e == hipSuccess ? kOk : hip_fail(e, "hipFree");
}

int axon_hip_host_malloc(void** ptr, size_t bytes) {
  AXON_READY();
  const hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
  if (e != hipSuccess) return hip_fail(e, "hipHostMalloc");
  g_device_allocations.fetch_add(1, std::memory_order_relaxed);
  return kOk;
}

int axon_hip_host_free(void* ptr) {
  const hipError_t e = hipHostFree(ptr);
  return e == hipSuccess ? kOk : hip_fail(e, "hipHostFree");
}

static int copy_sync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, const char* what) {
  AXON_READY();
  if (bytes == 0) return kOk;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  return e == hipSuccess ? kOk : hip_fail(e, what);
}

int axon_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyHostToDevice, "memcpy_h2d");
}
int axon_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToHost, "memcpy_d2h");
}
int axon_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToDevice, "memcpy_d2d");
}

int axon_hip_memcpy_h2d_async(void* dst, const void* src, size_t bytes) {
  AXON_READY();
  if (bytes == 0) return kOk;
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream);
  return e == hipSuccess ? kOk : hip_fail(e, "memcpy_h2d_async");
}

int axon_hip_memset(void* dst, int value, size_t bytes) {
  AXON_READY();
  if (bytes == 0) return kOk;
  // A memset node in a captured graph is not replayed reliably on this platform, and the
  // synchronize below is illegal under capture: refuse while axon_hip_graph_begin is open.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(g_stream, &cap);
  if (e != hipSuccess) return hip_fail(e, "memset: hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(kInvalidArgument, "memset: refused while a graph capture is open on the library stream");
  e = hipMemsetAsync(dst, value, bytes, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  return e == hipSuccess ? kOk : hip_fail(e, "memset");
}

int axon_hip_synchronize(void) {
  AXON_READY();
  const hipError_t e = hipStreamSynchronize(g_stream);
  return e == hipSuccess ? kOk : hip_fail(e, "hipStreamSynchronize");
}

int axon_hip_event_create(void** event) {
  AXON_READY();
  hipEvent_t ev;
  const hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
  g_device_allocations.fetch_add(1, std::memory_order_relaxed);
  *event = ev;
  return kOk;
}

int axon_hip_event_record(void* event) {
  AXON_READY();
  const hipError_t e = hipEventRecord(static_cast<hipEvent_t>(event), g_stream);
  return e == hipSuccess ? kOk : hip_fail(e, "hipEventRecord");
}

int axon_hip_probe_next_launch(void* start, void* stop) {
  AXON_READY();
  if ((start == nullptr) != (stop == nullptr)) return fail(kInvalidArgument, "probe: both events or neither");
  g_probe_start = static_cast<hipEvent_t>(start);
  g_probe_stop = static_cast<hipEvent_t>(stop);
  return kOk;
}

int axon_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(stop));
  if (e == hipSuccess) e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
  return e == hipSuccess ? kOk : hip_fail(e, "hipEventElapsedTime");
}

int axon_hip_event_destroy(void* event) {
  const hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
  return e == hipSuccess ? kOk : hip_fail(e, "hipEventDestroy");
}

int axon_hip_graph_begin(void) {
  AXON_READY();
  const hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal);
  return e == hipSuccess ? kOk : hip_fail(e, "hipStreamBeginCapture");
}

int axon_hip_graph_end(void** graph) {
  AXON_READY();
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g);
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *graph = exec;
  return kOk;
}

int axon_hip_graph_launch(void* graph) {
  AXON_READY();
  const hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph), g_stream);
  return e == hipSuccess ? kOk : hip_fail(e, "hipGraphLaunch");
}

int axon_hip_graph_destroy(void* graph) {
  const hipError_t e = hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph));
  return e == hipSuccess ? kOk : hip_fail(e, "hipGraphExecDestroy");
}

// ---- KernelTable entries -----------------------------------------------------------------

int axon_hip_matmul_f32(const float* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return float_rows(F32, w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_f16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return float_rows(F16, w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_bf16(const uint16_t* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return float_rows(BF16, w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_f32_rows(const float* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                             size_t y_stride) {
  return float_rows(F32, w, x, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_f16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                             size_t y_stride) {
  return float_rows(F16, w, x, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_bf16_rows(const uint16_t* w, const float* x, float* y, size_t n_rows, size_t n_out,
                              size_t n_in, size_t y_stride) {
  return float_rows(BF16, w, x, y, n_rows, n_out, n_in, y_stride);
}

int axon_hip_rmsnorm(const float* x, const float* weight, float* y, size_t n, float eps) {
  AXON_READY();
  if (n == 0) return fail(kInvalidArgument, "rmsnorm: n is 0");
  if (!fits_u32(n)) return fail(kInvalidArgument, "rmsnorm: n too large");
  return rmsnorm_launch(x, weight, y, nullptr, static_cast<uint32_t>(n), 1, eps);
}

int axon_hip_rope(float* x, size_t n_heads, size_t pos, size_t head_dim, size_t rotary_dim, float theta, int style,
                  const float* freq_factors) {
  AXON_READY();
  if (!fits_u32(n_heads) || !fits_u32(head_dim) || pos > 0x7fffffffull) return fail(kInvalidArgument, "rope: sizes too large");
  RopeRowsArgs a{};
  a.q = x;
  a.pos0 = static_cast<int32_t>(pos);
  a.q_stride = static_cast<uint32_t>(n_heads * head_dim);
  a.n_head = static_cast<uint32_t>(n_heads);
  a.head_dim = static_cast<uint32_t>(head_dim);
  a.rotary_dim = static_cast<uint32_t>(rotary_dim);
  a.neox = style;
  a.theta = theta;
  a.freq_factors = freq_factors;
  return rope_rows_launch(a, 1);
}

int axon_hip_softmax(float* x, size_t n) {
  AXON_READY();
  if (n == 0) return fail(kInvalidArgument, "softmax: n is 0");
  if (!fits_u32(n)) return fail(kInvalidArgument, "softmax: n too large");
  return softmax_launch(x, static_cast<uint32_t>(n));
}

int axon_hip_silu_mul(const float* gate, const float* up, float* out, size_t n) {
  AXON_READY();
  if (!fits_u32(n)) return fail(kInvalidArgument, "silu_mul: n too large");
  return silu_mul_launch(gate, up, out, nullptr, static_cast<uint32_t>(n), 1);
}

int axon_hip_embedding_row(int type, const void* table, size_t n, int64_t index, float* out) {
  AXON_READY();
  if (index < 0) return fail(kInvalidArgument, "embedding_row: index %lld", static_cast<long long>(index));
  if (!fits_u32(n)) return fail(kInvalidArgument, "embedding_row: n too large");
  return embedding_launch(type, static_cast<const uint8_t*>(table), static_cast<uint32_t>(n), nullptr, index, 1, out);
}

int axon_hip_attention(const float* q, const float* k, const float* v, float* out, float* scores, size_t seq,
                       size_t n_head, size_t n_head_kv, size_t head_dim, float scale) {
  return attention_heads(q, k, v, out, scores, seq, 0, n_head, n_head_kv, head_dim, scale, 0, n_head, 0);
}

int axon_hip_attention_kv(const float* q, const float* k_cache, const float* v_cache, float* out, float* scores,
                          size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv, size_t head_dim, float scale) {
  return attention_heads(q, k_cache, v_cache, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale, 0,
                         n_head, 0);
}

int axon_hip_attention_kv_heads(const float* q, const float* k_cache, const float* v_cache, float* out,
                                float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                                size_t head_dim, float scale, size_t head_begin, size_t head_end) {
  return attention_heads(q, k_cache, v_cache, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale,
                         head_begin, head_end, 0);
}

int axon_hip_attention_kv_heads_f16(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                                    float* scores, size_t n_q, size_t n_past, size_t n_head, size_t n_head_kv,
                                    size_t head_dim, float scale, size_t head_begin, size_t head_end) {
  return attention_heads(q, k_cache, v_cache, out, scores, n_q, n_past, n_head, n_head_kv, head_dim, scale,
                         head_begin, head_end, 1);
}

int axon_hip_matmul_q8_0(const void* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return float_rows(Q8_0, w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q4_0(const void* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return float_rows(Q4_0, w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q8_0_q8(const void* w, const void* xq, float* y, size_t n_out, size_t n_in) {
  return q8_rows(Q8_0, w, xq, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q4_0_q8(const void* w, const void* xq, float* y, size_t n_out, size_t n_in) {
  return q8_rows(Q4_0, w, xq, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q8_0_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride) {
  return float_rows(Q8_0, w, x, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_q4_0_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride) {
  return float_rows(Q4_0, w, x, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_q8_0_q8_rows(const void* w, const void* xq, float* y, size_t n_rows, size_t n_out, size_t n_in,
                                 size_t y_stride) {
  return q8_rows(Q8_0, w, xq, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_q4_0_q8_rows(const void* w, const void* xq, float* y, size_t n_rows, size_t n_out, size_t n_in,
                                 size_t y_stride) {
  return q8_rows(Q4_0, w, xq, y, n_rows, n_out, n_in, y_stride);
}

int axon_hip_quantize_row_q8_0(const float* x, void* out, size_t n) {
  AXON_READY();
  if (!fits_u32(n)) return fail(kInvalidArgument, "quantize_row_q8_0: n too large");
  return quantize_rows_launch(x, static_cast<uint8_t*>(out), static_cast<uint32_t>(n), 1, static_cast<uint32_t>(n));
}

int axon_hip_matmul_q4_1(const void* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return float_rows(Q4_1, w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q4_1_q8(const void* w, const void* xq, float* y, size_t n_out, size_t n_in) {
  return q8_rows(Q4_1, w, xq, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q4_1_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride) {
  return float_rows(Q4_1, w, x, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_q4_1_q8_rows(const void* w, const void* xq, float* y, size_t n_rows, size_t n_out, size_t n_in,
                                 size_t y_stride) {
  return q8_rows(Q4_1, w, xq, y, n_rows, n_out, n_in, y_stride);
}
int axon_hip_matmul_q6_k(const void* w, const float* x, float* y, size_t n_out, size_t n_in) {
  return q6k_rows(w, x, y, 1, n_out, n_in, n_out);
}
int axon_hip_matmul_q6_k_rows(const void* w, const float* x, float* y, size_t n_rows, size_t n_out, size_t n_in,
                              size_t y_stride) {
  return q6k_rows(w, x, y, n_rows, n_out, n_in, y_stride);
}

// ---- coarse entries ---------------------------------------------------------------------

size_t axon_hip_q6k_planar_bytes(size_t n_out, size_t n_in) {
  if (!fits_u32(n_out) || n_in % kQKK != 0) return 0;
  return q6k_planar_column_bytes(static_cast<uint32_t>(n_out)) * (n_in / kQKK);
}

int axon_hip_q6k_repack(const void* w, size_t n_out, size_t n_in, void* planar) {
  AXON_READY();
  if (n_in % kQKK != 0 || !fits_u32(n_out) || !fits_u32(n_in / kQKK))
    return fail(kInvalidArgument, "q6k_repack: %zu x %zu (n_in a multiple of 256)", n_out, n_in);
  if (w == nullptr || planar == nullptr) return fail(kInvalidArgument, "q6k_repack: null pointer");
  return q6k_repack_launch(static_cast<const uint8_t*>(w), static_cast<uint8_t*>(planar), static_cast<uint32_t>(n_out),
                           static_cast<uint32_t>(n_in / kQKK));
}

int axon_hip_matmul_q6_k_planar(const void* planar, const float* x, float* y, size_t n_rows, size_t n_out,
                                size_t n_in, size_t y_stride) {
  AXON_READY();
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k_planar: n_in %zu is not a multiple of 256", n_in);
  if (!fits_u32(n_rows) || !fits_u32(n_out) || !fits_u32(n_in) || !fits_u32(y_stride))
    return fail(kInvalidArgument, "matmul_q6_k_planar: sizes too large");
  if (n_rows > 1 && y_stride < n_out)
    return fail(kInvalidArgument, "matmul_q6_k_planar: y_stride %zu < n_out %zu", y_stride, n_out);
  MatvecArgs a{};
  a.seg[0] = MatvecSeg{static_cast<const uint8_t*>(planar), y, static_cast<uint32_t>(n_out),
                       static_cast<uint32_t>(y_stride), 0};
  a.n_seg = 1;
  a.xq = reinterpret_cast<const uint8_t*>(x);
  a.nb = static_cast<uint32_t>(n_in / kQKK);
  a.m = static_cast<uint32_t>(n_rows);
  return matvec_q6k_planar_launch(a, static_cast<uint32_t>(n_in));
}

size_t axon_hip_q6k_argmax_parts(size_t n_out) {
  return n_out == 0 || !fits_u32(n_out) ? 0 : q6k_planar_argmax_parts(static_cast<uint32_t>(n_out));
}

int axon_hip_matmul_q6_k_planar_argmax(const void* planar, const float* x, float* y, size_t n_out, size_t n_in,
                                       uint64_t* keys, size_t key_words) {
  AXON_READY();
  if (n_in % kQKK != 0) return fail(kInvalidArgument, "matmul_q6_k_planar_argmax: n_in %zu is not a multiple of 256", n_in);
  if (n_out == 0 || !fits_u32(n_out) || !fits_u32(n_in)) return fail(kInvalidArgument, "matmul_q6_k_planar_argmax: %zu outputs", n_out);
  if (keys == nullptr || key_words < axon_hip_q6k_argmax_parts(n_out))
    return fail(kInvalidArgument, "matmul_q6_k_planar_argmax: %zu key words for %zu outputs", key_words, n_out);
  MatvecArgs a{};
  a.seg[0] = MatvecSeg{static_cast<const uint8_t*>(planar), y, static_cast<uint32_t>(n_out), static_cast<uint32_t>(n_out), 0};
  a.n_seg = 1;
  a.xq = reinterpret_cast<const uint8_t*>(x);
  a.nb = static_cast<uint32_t>(n_in / kQKK);
  a.m = 1;
  a.argmax_part = keys;
  return matvec_q6k_planar_launch(a, static_cast<uint32_t>(n_in));
}

int axon_hip_argmax_embed(const float* x, const uint64_t* keys, size_t n_keys, int32_t* out, int type,
                          const void* table, size_t table_rows, size_t n, float* emb) {
  AXON_READY();
  if (!fits_u32(n_keys) || !fits_u32(n) || !fits_u32(table_rows)) return fail(kInvalidArgument, "argmax_embed: sizes too large");
  if (x == nullptr || keys == nullptr || out == nullptr || table == nullptr || emb == nullptr)
    return fail(kInvalidArgument, "argmax_embed: null pointer");
  return argmax_embed_launch(x, keys, static_cast<uint32_t>(n_keys), out, type, static_cast<const uint8_t*>(table),
                             static_cast<uint32_t>(table_rows), static_cast<uint32_t>(n), emb);
}

int axon_hip_q6k_force_path(int path) {
  if (path < 0 || path > 3) return fail(kInvalidArgument, "q6k_force_path: path %d (0-3)", path);
  matvec_q6k_force_path(path);
  return kOk;
}

int axon_hip_rmsnorm_rows(const float* x, const float* weight, float* y, void* yq, size_t n, size_t n_rows,
                          float eps) {
  AXON_READY();
  if (n == 0) return fail(kInvalidArgument, "rmsnorm: n is 0");
  if (!fits_u32(n) || !fits_u32(n_rows)) return fail(kInvalidArgument, "rmsnorm: sizes too large");
  if (y == nullptr && yq == nullptr) return fail(kInvalidArgument, "rmsnorm_rows: no output");
  return rmsnorm_launch(x, weight, y, static_cast<uint8_t*>(yq), static_cast<uint32_t>(n),
                        static_cast<uint32_t>(n_rows), eps);
}

int axon_hip_quantize_rows_q8_0(const float* x, void* out, size_t n, size_t n_rows, size_t x_stride) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows) || !fits_u32(x_stride)) return fail(kInvalidArgument, "quantize_rows: sizes too large");
  return quantize_rows_launch(x, static_cast<uint8_t*>(out), static_cast<uint32_t>(n), static_cast<uint32_t>(n_rows),
                              static_cast<uint32_t>(x_stride));
}

int axon_hip_silu_mul_rows(const float* gate, const float* up, float* out, void* outq, size_t n, size_t n_rows) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows)) return fail(kInvalidArgument, "silu_mul_rows: sizes too large");
  return silu_mul_launch(gate, up, out, static_cast<uint8_t*>(outq), static_cast<uint32_t>(n),
                         static_cast<uint32_t>(n_rows));
}

int axon_hip_add(float* x, const float* y, size_t n) {
  AXON_READY();
  return add_launch(x, y, n);
}

int axon_hip_repeat_penalty_rows(float* x, size_t n, size_t n_rows, size_t stride, const int32_t* recent,
                                 const uint32_t* recent_len, size_t recent_stride, float penalty) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows) || stride < n)
    return fail(kInvalidArgument, "repeat_penalty: %zu x %zu, stride %zu", n_rows, n, stride);
  if (n_rows != 0 && recent_stride != 0 && (recent == nullptr || recent_len == nullptr))
    return fail(kInvalidArgument, "repeat_penalty: recent ids and lengths are required");
  return repeat_penalty_launch(x, static_cast<uint32_t>(n), static_cast<uint32_t>(n_rows), stride, recent, recent_len,
                               recent_stride, penalty);
}

size_t axon_hip_argmax_scratch_words(size_t n_rows) { return argmax_scratch_words(static_cast<uint32_t>(n_rows)); }

int axon_hip_argmax_rows(const float* x, size_t n, size_t n_rows, size_t stride, uint64_t* scratch, int32_t* out) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows) || stride < n) return fail(kInvalidArgument, "argmax: %zu x %zu, stride %zu", n_rows, n, stride);
  if (scratch == nullptr || out == nullptr) return fail(kInvalidArgument, "argmax: scratch and output are required");
  return argmax_rows_launch(x, static_cast<uint32_t>(n), static_cast<uint32_t>(n_rows), stride, scratch, out);
}

int axon_hip_argmax_rows_noalloc(const float* x, size_t n, size_t n_rows, size_t stride, int32_t* out) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows) || stride < n) return fail(kInvalidArgument, "argmax: %zu x %zu, stride %zu", n_rows, n, stride);
  if (out == nullptr) return fail(kInvalidArgument, "argmax: the output is required");
  return argmax_rows_noalloc_launch(x, static_cast<uint32_t>(n), static_cast<uint32_t>(n_rows), stride, out);
}

static_assert(kMaxTopK == AXON_HIP_MAX_TOPK, "one top-k bound");
static_assert(kArgmaxNoAllocRows == AXON_HIP_ARGMAX_NOALLOC_MAX_ROWS, "one no-allocation row bound");

int axon_hip_matmul_q8_swiglu(int type, const void* xq, size_t n_rows, size_t n_in, const void* w_gate,
                              const void* w_up, size_t n_ff, float* out, void* outq) {
  AXON_READY();
  if (n_in % kQK != 0 || n_ff % kQK != 0 || !fits_u32(n_rows) || !fits_u32(n_in) || !fits_u32(n_ff))
    return fail(kInvalidArgument, "matmul_q8_swiglu: %zu x %zu -> %zu", n_rows, n_in, n_ff);
  if (xq == nullptr || w_gate == nullptr || w_up == nullptr || outq == nullptr)
    return fail(kInvalidArgument, "matmul_q8_swiglu: null pointer");
  MatvecArgs a{};
  a.seg[0] = MatvecSeg{static_cast<const uint8_t*>(w_gate), out, static_cast<uint32_t>(n_ff), static_cast<uint32_t>(n_ff), 0};
  a.seg[1] = MatvecSeg{static_cast<const uint8_t*>(w_up), nullptr, static_cast<uint32_t>(n_ff), static_cast<uint32_t>(n_ff), 0};
  a.n_seg = 2;
  a.xq = static_cast<const uint8_t*>(xq);
  a.nb = static_cast<uint32_t>(n_in / kQK);
  a.m = static_cast<uint32_t>(n_rows);
  a.outq = static_cast<uint8_t*>(outq);
  return matmul_q8_swiglu_launch(type, a);
}

int axon_hip_topk_rows(const float* x, size_t n, size_t n_rows, size_t stride, size_t k, float* out_logit,
                       int32_t* out_id) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows) || stride < n) return fail(kInvalidArgument, "topk: %zu x %zu, stride %zu", n_rows, n, stride);
  if (k == 0 || k > kMaxTopK || k > n) return fail(kInvalidArgument, "topk: k %zu of %zu values (k in 1..%u)", k, n, kMaxTopK);
  if (out_logit == nullptr || out_id == nullptr) return fail(kInvalidArgument, "topk: outputs are required");
  return topk_rows_launch(x, static_cast<uint32_t>(n), static_cast<uint32_t>(n_rows), stride, static_cast<uint32_t>(k),
                          out_logit, out_id);
}

size_t axon_hip_sort_rows_work_bytes(size_t n, size_t n_rows) { return 8 * n * n_rows; }

int axon_hip_sort_rows(const float* x, size_t n, size_t n_rows, size_t stride, void* work, float* out_logit,
                       int32_t* out_id) {
  AXON_READY();
  if (n == 0 || !fits_u32(n) || !fits_u32(n_rows) || stride < n)
    return fail(kInvalidArgument, "sort_rows: %zu x %zu, stride %zu", n_rows, n, stride);
  if (work == nullptr || out_logit == nullptr || out_id == nullptr)
    return fail(kInvalidArgument, "sort_rows: the workspace and outputs are required");
  return sort_rows_launch(x, static_cast<uint32_t>(n), static_cast<uint32_t>(n_rows), stride, work, out_logit, out_id);
}

int axon_hip_matmul_q8_fused(int type, const void* xq, size_t n_rows, size_t n_in, size_t n_seg,
                             const void* const* w, float* const* y, const size_t* n_out, const size_t* y_stride,
                             int accumulate) {
  AXON_READY();
  return q8_matmul(type, xq, n_rows, n_in, n_seg, w, y, n_out, y_stride, accumulate);
}

int axon_hip_rope_rows(const axon_hip_rope_rows_args* args, size_t n_rows) {
  AXON_READY();
  if (!fits_u32(n_rows)) return fail(kInvalidArgument, "rope_rows: too many rows");
  static_assert(sizeof(axon_hip_rope_rows_args) == sizeof(RopeRowsArgs), "rope args layout");
  RopeRowsArgs a;
  std::memcpy(&a, args, sizeof(a));
  if ((a.bq == nullptr) != (a.bk == nullptr)) return fail(kInvalidArgument, "rope_rows: bq and bk go together");
  return rope_rows_launch(a, static_cast<uint32_t>(n_rows));
}

static AttnArgs attn_from(const axon_hip_attention_rows_args* args) {
  AttnArgs a{};
  a.q = args->q;
  a.out = args->out;
  a.q_stride = args->q_stride;
  a.out_stride = args->out_stride;
  a.kv = args->kv;
  a.k_off = args->k_off;
  a.v_off = args->v_off;
  a.n_vis = args->n_vis;
  a.k_off_c = args->k_layer_off;
  a.v_off_c = args->v_layer_off;
  a.n_past = args->n_past;
  a.n_head = args->n_head;
  a.n_kv = args->n_kv;
  a.head_dim = args->head_dim;
  a.head_begin = 0;
  a.head_end = args->n_head;
  a.scale = args->scale;
  a.f16 = args->f16;
  a.scratch = args->scratch;
  a.max_vis = args->max_vis;
  a.split = 1;
  a.outq = static_cast<uint8_t*>(args->outq);
  return a;
}

int axon_hip_attention_rows(const axon_hip_attention_rows_args* args, size_t n_rows) {
  AXON_READY();
  if (!fits_u32(n_rows)) return fail(kInvalidArgument, "attention_rows: too many rows");
  return attention_launch(attn_from(args), static_cast<uint32_t>(n_rows));
}

size_t axon_hip_attention_scratch_floats(const axon_hip_attention_rows_args* args, size_t n_rows) {
  return attention_scratch_floats(attn_from(args), static_cast<uint32_t>(n_rows));
}

int axon_hip_matvec_fused_supported(int type, int in_mode, size_t n_rows, size_t n_in, int silu) {
  if ((type != Q8_0 && type != Q4_0 && type != Q4_1) || n_in % kQK != 0 || n_rows > 4 || n_in > (1u << 24)) return 0;
  if (in_mode < kInQ8 || in_mode > kInNorm) return 0;
  return matvec_fused_fits(type, in_mode, static_cast<uint32_t>(n_rows), static_cast<uint32_t>(n_in / kQK), silu != 0)
             ? 1
             : 0;
}

int axon_hip_matvec_fused(const axon_hip_matvec_fused_args* p) {
  AXON_READY();
  if (p->n_seg < 1 || p->n_seg > 3) return fail(kInvalidArgument, "matvec_fused: %zu segments", p->n_seg);
  if (p->n_in % kQK != 0) return fail(kInvalidArgument, "matvec_fused: n_in %zu is not a multiple of 32", p->n_in);
  if (p->out_mode < kOutStore || p->out_mode > kOutRope) return fail(kInvalidArgument, "matvec_fused: out_mode %d", p->out_mode);
  if (p->in_mode < kInQ8 || p->in_mode > kInNorm) return fail(kInvalidArgument, "matvec_fused: in_mode %d", p->in_mode);
  if (p->out_mode == kOutRope && (p->pos == nullptr || p->cache == nullptr || p->cache_off == nullptr ||
                                  p->rope_table == nullptr || p->head_dim == 0 || p->rot_half * 2 > p->head_dim))
    return fail(kInvalidArgument, "matvec_fused: the rope epilogue needs positions, a cache and a cos/sin table");
  if (!fits_u32(p->n_rows) || !fits_u32(p->n_in) || !fits_u32(p->x_stride)) return fail(kInvalidArgument, "matvec_fused: sizes too large");
  FusedArgs a{};
  a.n_seg = static_cast<int>(p->n_seg);
  for (size_t s = 0; s < p->n_seg; ++s) {
    if (!fits_u32(p->n_out[s]) || !fits_u32(p->y_stride[s])) return fail(kInvalidArgument, "matvec_fused: sizes too large");
    a.w[s] = static_cast<const uint8_t*>(p->w[s]);
    a.n_out[s] = static_cast<uint32_t>(p->n_out[s]);
    a.y[s] = p->y[s];
    a.y_stride[s] = static_cast<uint32_t>(p->y_stride[s]);
    a.bias[s] = p->bias[s];
  }
  a.nb = static_cast<uint32_t>(p->n_in / kQK);
  a.m = static_cast<uint32_t>(p->n_rows);
  a.in_mode = p->in_mode;
  a.xq = static_cast<const uint8_t*>(p->xq);
  a.x = p->x;
  a.x_stride = static_cast<uint32_t>(p->x_stride);
  a.norm_w = p->norm_w;
  a.eps = p->eps;
  a.out_mode = p->out_mode;
  a.rope_table = p->rope_table;
  a.rot_half = p->rot_half;
  a.head_dim = p->head_dim;
  a.pos = p->pos;
  a.cache_off = p->cache_off;
  a.cache = p->cache;
  a.cache_f16 = p->cache_f16 != 0;
  a.k_layer_off = p->k_layer_off;
  a.v_layer_off = p->v_layer_off;
  a.outq = static_cast<uint8_t*>(p->outq);
  if (a.outq != nullptr && (a.out_mode != kOutSilu || a.n_out[0] % kQK != 0))
    return fail(kInvalidArgument, "matvec_fused: Q8_0 output needs the SiLU epilogue and outputs in whole blocks");
  return matvec_fused_launch(p->type, a);
}

int axon_hip_matmul_q8_qkv_rope(const axon_hip_matvec_fused_args* p) {
  AXON_READY();
  if (p->n_seg != 3 || p->in_mode != kInQ8 || p->out_mode != kOutRope)
    return fail(kInvalidArgument, "matmul_q8_qkv_rope: three segments, in_mode 0 and out_mode 3");
  if (p->n_in % kQK != 0 || p->n_in == 0) return fail(kInvalidArgument, "matmul_q8_qkv_rope: n_in %zu is not a positive multiple of 32", p->n_in);
  if (p->xq == nullptr || p->y[0] == nullptr || p->pos == nullptr || p->cache == nullptr || p->cache_off == nullptr ||
      p->rope_table == nullptr)
    return fail(kInvalidArgument, "matmul_q8_qkv_rope: needs the blocks, q's buffer, positions, a cache and a cos/sin table");
  if (p->head_dim == 0 || (p->head_dim & 1) != 0 || p->rot_half * 2 > p->head_dim || p->n_out[1] != p->n_out[2] ||
      ((p->n_out[0] | p->n_out[1]) & 1) != 0 || p->y_stride[0] < p->n_out[0])
    return fail(kInvalidArgument, "matmul_q8_qkv_rope: q|k|v shapes");
  if (p->n_rows == 0) return kOk;
  if (p->n_rows > kRowsMaxM) return fail(kUnsupported, "matmul_q8_qkv_rope: %zu rows (at most %u)", p->n_rows, kRowsMaxM);
  if (!fits_u32(p->n_in) || !fits_u32(p->n_out[0]) || !fits_u32(p->n_out[1]) || !fits_u32(p->y_stride[0]))
    return fail(kInvalidArgument, "matmul_q8_qkv_rope: sizes too large");
  MatvecArgs a{};
  for (int s = 0; s < 3; ++s)
    a.seg[s] = MatvecSeg{static_cast<const uint8_t*>(p->w[s]), s == 0 ? p->y[0] : nullptr,
                         static_cast<uint32_t>(p->n_out[s]), s == 0 ? static_cast<uint32_t>(p->y_stride[0]) : 0u, 0};
  a.n_seg = 3;
  a.xq = static_cast<const uint8_t*>(p->xq);
  a.nb = static_cast<uint32_t>(p->n_in / kQK);
  a.m = static_cast<uint32_t>(p->n_rows);
  RowsRope rp{};
  for (int s = 0; s < 3; ++s) rp.bias[s] = p->bias[s];
  rp.table = p->rope_table;
  rp.pos = p->pos;
  rp.cache_off = p->cache_off;
  rp.cache = p->cache;
  rp.k_layer_off = p->k_layer_off;
  rp.v_layer_off = p->v_layer_off;
  rp.rot_half = p->rot_half;
  rp.head_dim = p->head_dim;
  rp.kv_row = static_cast<uint32_t>(p->n_out[1]);
  rp.cache_f16 = p->cache_f16 != 0;
  return matmul_q8_rows_rope_launch(p->type, a, rp);
}

namespace {
axon_hip::StepShape step_shape_of(const axon_hip_decode_shape* sh) {
  axon_hip::StepShape s{};
  s.n_layer = sh->n_layer;
  s.d = sh->n_embd;
  s.dq = sh->n_head * 64;
  s.dkv = sh->n_head_kv * 64;
  s.ff = sh->n_ff;
  s.n_head = sh->n_head;
  s.n_kv = sh->n_head_kv;
  s.rot_half = sh->rotary_dim / 2;
  s.t_qkv = sh->type_qkv;
  s.t_o = sh->type_o;
  s.t_gu = sh->type_gate_up;
  s.t_down = sh->type_down;
  s.max_ctx = sh->max_ctx;
  s.cache_f16 = sh->cache_f16 != 0;
  return s;
}
constexpr uint32_t kStepSpinLimit = 1u << 20;  // polls of one barrier (about a second) before giving up
std::atomic<uint32_t> g_step_spin_limit{kStepSpinLimit};
std::atomic<uint32_t> g_step_fail_waits{0};
std::atomic<uint64_t*> g_step_stamps{nullptr};
static_assert(sizeof(axon_hip_decode_layer) == sizeof(axon_hip::StepLayer), "one layer record layout");
}  // namespace

int axon_hip_decode_layers_set_spin_limit(uint32_t polls) {
  g_step_spin_limit.store(polls == 0 ? kStepSpinLimit : polls, std::memory_order_relaxed);
  return kOk;
}

int axon_hip_decode_layers_set_fail_waits(int on) {
  g_step_fail_waits.store(on != 0 ? 1u : 0u, std::memory_order_relaxed);
  return kOk;
}

int axon_hip_decode_layers_set_stamps(uint64_t* stamps) {
  g_step_stamps.store(stamps, std::memory_order_relaxed);
  return kOk;
}

size_t axon_hip_decode_layers_stamp_count(const axon_hip_decode_shape* shape, double* ticks_per_second) {
  if (shape == nullptr || ready() != kOk) return 0;
  if (ticks_per_second != nullptr) {
    int khz = 0;
    *ticks_per_second = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, g_device) == hipSuccess
                            ? 1e3 * khz
                            : 0.0;
  }
  return step_stamp_count(step_shape_of(shape));
}

size_t axon_hip_decode_layers_workspace_bytes(const axon_hip_decode_shape* shape) {
  return shape == nullptr ? 0 : step_workspace_bytes(step_shape_of(shape));
}

const char* axon_hip_decode_layers_unsupported(const axon_hip_decode_shape* shape) {
  if (shape == nullptr) return "no shape";
  if (ready() != kOk) return "no device";
  if (shape->rotary_dim == 0 || shape->rotary_dim % 2 != 0 || shape->rotary_dim > 64) return "a rotary width outside the head";
  return step_unsupported(step_shape_of(shape));
}

int axon_hip_decode_layers(const axon_hip_decode_shape* shape, const axon_hip_decode_layers_args* a) {
  AXON_READY();
  if (shape == nullptr || a == nullptr || a->layers == nullptr || a->x == nullptr || a->cache == nullptr ||
      a->work == nullptr || a->epoch == nullptr || a->status == nullptr || a->rope_table == nullptr)
    return fail(kInvalidArgument, "decode_layers: missing argument");
  if (*reinterpret_cast<volatile uint32_t*>(a->status) != 0)
    return fail(kHipError, "decode_layers: an earlier call gave up at a device-wide barrier (status %u); "
                           "zero the workspace and reset epoch and status", *a->status);
  const StepShape s = step_shape_of(shape);
  // Phase tags are the low 32 bits of epoch + phase: the phases of this call must not wrap, or
  // a tag could match a word written 2^32 phases earlier (or a zeroed word, tag 0).
  if (*a->epoch + step_phases(s) > 0xffffffffull)
    return fail(kInvalidArgument, "decode_layers: epoch %llu + %llu phases passes 2^32; zero the workspace and reset epoch",
                static_cast<unsigned long long>(*a->epoch), static_cast<unsigned long long>(step_phases(s)));
  StepCall c{};
  c.layers = reinterpret_cast<const StepLayer*>(a->layers);
  c.eps = a->eps;
  c.scale = a->scale;
  c.rope_table = a->rope_table;
  c.x = a->x;
  c.cache = a->cache;
  c.cache_off = a->cache_off;
  c.pos = a->pos;
  c.work = a->work;
  c.epoch = *a->epoch;
  c.status = a->status;
  c.spin_limit = g_step_spin_limit.load(std::memory_order_relaxed);
  c.fail_waits = g_step_fail_waits.load(std::memory_order_relaxed);
  c.stamps = g_step_stamps.load(std::memory_order_relaxed);
  const int rc = step_launch(s, c);
  if (rc != kOk) return rc;
  *a->epoch += step_phases(s);
  return check_launch("decode_layers");
}

int axon_hip_embedding_rows(int type, const void* table, size_t n, const int32_t* ids, size_t n_rows, float* out) {
  AXON_READY();
  if (!fits_u32(n) || !fits_u32(n_rows)) return fail(kInvalidArgument, "embedding_rows: sizes too large");
  if (ids == nullptr) return fail(kInvalidArgument, "embedding_rows: ids is NULL");
  return embedding_launch(type, static_cast<const uint8_t*>(table), static_cast<uint32_t>(n), ids, 0,
                          static_cast<uint32_t>(n_rows), out);
}

int axon_hip_block_sums(int type, const void* w_row, const void* xq, size_t n_blocks, int32_t* sumi,
                        int32_t* sumx) {
  AXON_READY();
  if (!fits_u32(n_blocks)) return fail(kInvalidArgument, "block_sums: too many blocks");
  return block_sums_launch(type, w_row, xq, static_cast<uint32_t>(n_blocks), sumi, sumx);
}

}  // extern "C"
