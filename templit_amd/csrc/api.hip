// Device, memory, stream, event and graph entry points of the C-ABI.
//
// These stand in for what the Metal backend gets from metal-cpp:
//   metal::init/shutdown            src/my_metal/metal.cpp:18-38
//   MTLBuffer alloc/read/write/fill include/my_metal/storage.h:11-63
//   command queue / buffer / wait   src/my_metal/runtime.cpp:238,290-317
// The host runtime (hip::Runtime, Storage<hip::HIP,T>) reaches HIP only
// through these functions, so it builds with any C++20 compiler.
#include "common.h"
#include "gemm.h"

#include <rocprofiler-sdk-roctx/roctx.h>

#include <mutex>

using namespace tlh;

namespace {
std::once_flag g_init_once;
int g_init_status = 0;
int g_device = -1;

__global__ void fill_u32_kernel(uint32_t *dst, uint32_t value, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    dst[i] = value;
}

__global__ void increment_u32_kernel(uint32_t *c, size_t n, uint32_t delta) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    c[i] += delta;
}

// SplitMix64 output number i+1 of the stream seeded with `seed`.
__device__ inline uint64_t splitmix_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(float *dst, size_t n, uint64_t seed, float mean, float std) {
  const size_t pairs = (n + 1) / 2;
  for (size_t p = size_t(blockIdx.x) * blockDim.x + threadIdx.x; p < pairs;
       p += size_t(gridDim.x) * blockDim.x) {
    const double u1 = double((splitmix_at(seed, 2 * p) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = double((splitmix_at(seed, 2 * p + 1) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586 * u2;
    dst[2 * p] = float(mean + std * r * cos(t));
    if (2 * p + 1 < n) dst[2 * p + 1] = float(mean + std * r * sin(t));
  }
}

__global__ void fill_uniform_u32_kernel(uint32_t *dst, size_t n, uint64_t seed, uint32_t bound) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    dst[i] = uint32_t(splitmix_at(seed, i) % bound);
}

__global__ void compare_kernel(const uint32_t *a, const uint32_t *b, size_t n,
                               int *differs) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    if (a[i] != b[i]) {
      *differs = 1; // benign race: every writer stores the same value
      return;
    }
}

__global__ void compare_tail_kernel(const uint8_t *a, const uint8_t *b, size_t n,
                                    int *differs) {
  const size_t i = threadIdx.x;
  if (i < n && a[i] != b[i]) *differs = 1;
}
} // namespace

TLH_API int tlh_init(int device) {
  std::call_once(g_init_once, [&] {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e == hipSuccess && (device < 0 || device >= count)) e = hipErrorInvalidDevice;
    if (e == hipSuccess) e = hipSetDevice(device);
    // the allocation-free entry point's scratch address on this device
    if (e == hipSuccess) e = hipError_t(tlh::noalloc_scratch(nullptr));
    if (e == hipSuccess) g_device = device;
    g_init_status = int(e);
  });
  if (g_init_status == 0 && g_device != device) return int(hipErrorInvalidDevice);
  return g_init_status;
}

TLH_API int tlh_device_count(int *count) { return int(hipGetDeviceCount(count)); }

TLH_API int tlh_device_cu_count(int *count) {
  int device = 0;
  const hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return int(st);
  return int(hipDeviceGetAttribute(count, hipDeviceAttributeMultiprocessorCount, device));
}

TLH_API const char *tlh_error_string(int code) {
  return hipGetErrorString(static_cast<hipError_t>(code));
}

TLH_API int tlh_device_synchronize(void) { return int(hipDeviceSynchronize()); }

TLH_API int tlh_stream_create(void **stream) {
  hipStream_t s = nullptr;
  // Default priority on purpose: one in-order queue, like the Metal command
  // queue of the reference runtime.
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  *stream = s;
  return int(e);
}

TLH_API int tlh_stream_destroy(void *stream) {
  return int(hipStreamDestroy(as_stream(stream)));
}

TLH_API int tlh_stream_synchronize(void *stream) {
  return int(hipStreamSynchronize(as_stream(stream)));
}

TLH_API int tlh_malloc(void **ptr, size_t bytes) {
  *ptr = nullptr;
  if (bytes == 0) return 0;
  return int(hipMalloc(ptr, bytes));
}

TLH_API int tlh_free(void *ptr) { return ptr ? int(hipFree(ptr)) : 0; }

TLH_API int tlh_host_alloc(void **ptr, size_t bytes) {
  *ptr = nullptr;
  if (bytes == 0) return 0;
  return int(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}

TLH_API int tlh_host_free(void *ptr) { return ptr ? int(hipHostFree(ptr)) : 0; }

TLH_API int tlh_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
  if (bytes == 0) return 0;
  return int(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
}

TLH_API int tlh_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
  if (bytes == 0) return 0;
  return int(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
}

TLH_API int tlh_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream) {
  if (bytes == 0 || dst == src) return 0;
  return int(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
}

// Fills use kernels (never hipMemsetAsync) so they stay valid inside a
// captured graph that is replayed many times.
TLH_API int tlh_fill_u32(uint32_t *dst, uint32_t value, size_t n, void *stream) {
  if (n == 0) return 0;
  fill_u32_kernel<<<stride_grid(n, 256), 256, 0, as_stream(stream)>>>(dst, value, n);
  return launch_status();
}

TLH_API int tlh_increment_u32(uint32_t *counters, size_t n, uint32_t delta, void *stream) {
  if (n == 0) return 0;
  increment_u32_kernel<<<stride_grid(n, 256), 256, 0, as_stream(stream)>>>(counters, n, delta);
  return launch_status();
}

TLH_API int tlh_fill_normal(float *dst, size_t n, uint64_t seed, float mean, float std,
                            void *stream) {
  if (n == 0) return 0;
  fill_normal_kernel<<<stride_grid((n + 1) / 2, 256), 256, 0, as_stream(stream)>>>(dst, n, seed,
                                                                                  mean, std);
  return launch_status();
}

TLH_API int tlh_fill_uniform_u32(uint32_t *dst, size_t n, uint64_t seed, uint32_t bound,
                                 void *stream) {
  if (n == 0) return 0;
  if (bound == 0) return int(hipErrorInvalidValue);
  fill_uniform_u32_kernel<<<stride_grid(n, 256), 256, 0, as_stream(stream)>>>(dst, n, seed,
                                                                              bound);
  return launch_status();
}

TLH_API int tlh_fill_f32(float *dst, float value, size_t n, void *stream) {
  uint32_t bits;
  __builtin_memcpy(&bits, &value, 4);
  return tlh_fill_u32(reinterpret_cast<uint32_t *>(dst), bits, n, stream);
}

// Byte-wise equality of two device buffers; `scratch` is a device int.
// Synchronous: `*equal` is valid on return.
TLH_API int tlh_compare(const void *a, const void *b, size_t bytes, int *equal,
                        int *scratch, void *stream) {
  *equal = 1;
  if (bytes == 0 || a == b) return 0;
  hipStream_t s = as_stream(stream);
  int st = tlh_fill_u32(reinterpret_cast<uint32_t *>(scratch), 0, 1, stream);
  if (st) return st;
  const size_t words = bytes / 4;
  if (words) {
    compare_kernel<<<stride_grid(words, 256), 256, 0, s>>>(
        static_cast<const uint32_t *>(a), static_cast<const uint32_t *>(b), words, scratch);
    if ((st = launch_status())) return st;
  }
  if (bytes % 4) {
    compare_tail_kernel<<<1, 64, 0, s>>>(static_cast<const uint8_t *>(a) + words * 4,
                                         static_cast<const uint8_t *>(b) + words * 4,
                                         bytes % 4, scratch);
    if ((st = launch_status())) return st;
  }
  int differs = 0;
  st = int(hipMemcpyAsync(&differs, scratch, sizeof(int), hipMemcpyDeviceToHost, s));
  if (st) return st;
  st = int(hipStreamSynchronize(s));
  *equal = differs ? 0 : 1;
  return st;
}

TLH_API int tlh_event_create(void **event) {
  hipEvent_t e = nullptr;
  const hipError_t st = hipEventCreate(&e);
  *event = e;
  return int(st);
}

TLH_API int tlh_event_record(void *event, void *stream) {
  return int(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)));
}

TLH_API int tlh_stream_wait_event(void *stream, void *event) {
  return int(hipStreamWaitEvent(as_stream(stream), static_cast<hipEvent_t>(event), 0));
}

TLH_API int tlh_event_synchronize(void *event) {
  return int(hipEventSynchronize(static_cast<hipEvent_t>(event)));
}

TLH_API int tlh_event_elapsed_ms(void *start, void *end, float *ms) {
  return int(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                 static_cast<hipEvent_t>(end)));
}

TLH_API int tlh_event_destroy(void *event) {
  return event ? int(hipEventDestroy(static_cast<hipEvent_t>(event))) : 0;
}

// hipGraph capture/replay: stands in for recording a Metal command buffer
// once and committing it again (src/my_metal/runtime.cpp:290-317).
TLH_API int tlh_graph_begin_capture(void *stream) {
  return int(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
}

TLH_API int tlh_graph_end_capture(void *stream, void **exec) {
  *exec = nullptr;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(as_stream(stream), &graph);
  if (e != hipSuccess) return int(e);
  hipGraphExec_t ge = nullptr;
  e = hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  *exec = ge;
  return int(e);
}

TLH_API int tlh_graph_begin_capture_relaxed(void *stream) {
  return int(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeRelaxed));
}

TLH_API int tlh_graph_end_capture_graph(void *stream, void **graph) {
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(as_stream(stream), &g);
  *graph = g;
  return int(e);
}

TLH_API int tlh_graph_instantiate(void *graph, void **exec) {
  hipGraphExec_t ge = nullptr;
  const hipError_t e = hipGraphInstantiate(&ge, static_cast<hipGraph_t>(graph), nullptr, nullptr, 0);
  *exec = ge;
  return int(e);
}

// Rewrites the parameters of `exec` from `graph` when both have the same
// topology; *updated = 0 (and return 0) when they do not.
TLH_API int tlh_graph_exec_update(void *exec, void *graph, int *updated) {
  hipGraphNode_t error_node = nullptr;
  hipGraphExecUpdateResult result = hipGraphExecUpdateSuccess;
  const hipError_t e = hipGraphExecUpdate(static_cast<hipGraphExec_t>(exec),
                                          static_cast<hipGraph_t>(graph), &error_node, &result);
  *updated = (e == hipSuccess && result == hipGraphExecUpdateSuccess) ? 1 : 0;
  if (e != hipSuccess) (void)hipGetLastError(); // a refused update is not an error here
  return 0;
}

TLH_API int tlh_graph_free(void *graph) {
  return graph ? int(hipGraphDestroy(static_cast<hipGraph_t>(graph))) : 0;
}

TLH_API int tlh_stream_is_capturing(void *stream, int *capturing) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(as_stream(stream), &st);
  *capturing = st == hipStreamCaptureStatusActive ? 1 : 0;
  return int(e);
}

// Named ranges for rocprofv3 (--marker-trace) around host-side spans:
// Runtime::start_profile / end_profile (Metal: a GPU-trace capture,
// src/my_metal/runtime.cpp:42-63).
TLH_API int tlh_range_push(const char *name) { return roctxRangePushA(name) < 0 ? 1 : 0; }
TLH_API int tlh_range_pop(void) { return roctxRangePop() < 0 ? 1 : 0; }

TLH_API int tlh_graph_launch(void *exec, void *stream) {
  return int(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), as_stream(stream)));
}

TLH_API int tlh_graph_destroy(void *exec) {
  return exec ? int(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec))) : 0;
}
