// Process-wide device context of the HIP backend: device selection, the one
// in-order stream, a caching device-memory pool and host transfers.
//
// Reference counterpart: metal::init/shutdown/device (src/my_metal/
// metal.cpp:18-38) plus the shared-mode MTLBuffer allocation and memcpy of
// Storage<metal::Metal,T> (include/my_metal/storage.h:11-63). The Metal
// backend allocates a fresh buffer for every tensor; executor temporaries
// make that hundreds of allocations per training step, so here device
// memory comes from a pool that parks freed blocks by size and hands them
// back in LIFO order (a repeated step sees the same addresses again, which
// is what lets a recorded graph be refreshed rather than rebuilt).
//
// Host code only: all device access goes through include/templit_hip.h.
#include "my_hip/hip.h"

#include "templit_hip.h"

#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace hip {
namespace {

// Pool size classes: 512-byte granules up to 1 MiB, 64 KiB granules above
// (every block starts 256-byte aligned, as hipMalloc returns it).
size_t size_class(size_t bytes) {
  if (bytes <= (size_t(1) << 20)) return (bytes + 511) & ~size_t(511);
  return (bytes + 65535) & ~size_t(65535);
}

// Pinned staging for small host->device writes: the host data is copied
// into pinned memory and the device copy is queued without waiting. A slot
// is reused once the event recorded after its copy has completed.
constexpr size_t kStageSlot = 64 * 1024;
constexpr int kStageSlots = 64;

struct Context {
  int device = 0;
  void *stream = nullptr;
  void *side = nullptr; // transfers made while `stream` is being captured
  int *compare_scratch = nullptr;
  std::mutex mu;
  std::unordered_map<size_t, std::vector<void *>> free_blocks;
  // Blocks released while the stream is being captured, with their size
  // class. They rejoin free_blocks only once the captured graph has been
  // launched (or the capture dropped): a record-time host write into a
  // block handed out again within the same capture would otherwise be
  // overwritten when the graph runs the kernels that used it first.
  bool defer = false;
  std::vector<std::pair<size_t, void *>> deferred;
  MemoryStats stats;
  std::vector<void *> stage_host;
  std::vector<void *> stage_event;
  int stage_next = 0;
};

std::unique_ptr<Context> g_ctx;
std::mutex g_init_mu;

Context &ctx() {
  if (!g_ctx) throw std::logic_error("hip::init() must be called before using the HIP backend");
  return *g_ctx;
}

void free_cached(Context &c) {
  for (auto &[bytes, blocks] : c.free_blocks) {
    for (void *p : blocks) tlh_free(p);
    c.stats.cached_bytes -= bytes * blocks.size();
  }
  c.free_blocks.clear();
}

void pool_deferred(Context &c) {
  for (auto &[cls, p] : c.deferred) c.free_blocks[cls].push_back(p);
  c.deferred.clear();
}

// The stream a host transfer goes on: the main stream, or the side stream
// (then synchronously) while the main stream is being recorded.
void *transfer_stream(Context &c, bool &sync_side) {
  int capturing = 0;
  detail::check(tlh_stream_is_capturing(c.stream, &capturing), "hipStreamIsCapturing");
  sync_side = capturing != 0;
  return capturing ? c.side : c.stream;
}

} // namespace

void init(int device) {
  std::lock_guard<std::mutex> lock(g_init_mu);
  if (g_ctx) {
    if (g_ctx->device != device)
      throw std::logic_error("hip::init: the backend is already bound to another device");
    return;
  }
  int count = 0;
  if (tlh_device_count(&count) != 0 || count == 0)
    throw std::runtime_error("hip::init: no HIP device is visible");
  detail::check(tlh_init(device), "hip::init");
  auto c = std::make_unique<Context>();
  c->device = device;
  detail::check(tlh_stream_create(&c->stream), "hipStreamCreate");
  detail::check(tlh_stream_create(&c->side), "hipStreamCreate");
  void *scratch = nullptr;
  detail::check(tlh_malloc(&scratch, 256), "hipMalloc");
  c->compare_scratch = static_cast<int *>(scratch);
  c->stage_host.assign(kStageSlots, nullptr);
  c->stage_event.assign(kStageSlots, nullptr);
  for (int i = 0; i < kStageSlots; ++i) {
    detail::check(tlh_host_alloc(&c->stage_host[i], kStageSlot), "hipHostMalloc");
    detail::check(tlh_event_create(&c->stage_event[i]), "hipEventCreate");
  }
  g_ctx = std::move(c);
}

void shutdown() {
  detail::drop_deferred_views(); // their tensors release blocks into the pool
  std::lock_guard<std::mutex> lock(g_init_mu);
  if (!g_ctx) return;
  Context &c = *g_ctx;
  tlh_stream_synchronize(c.stream);
  tlh_stream_synchronize(c.side);
  {
    std::lock_guard<std::mutex> pool_lock(c.mu);
    pool_deferred(c);
    free_cached(c);
  }
  for (int i = 0; i < kStageSlots; ++i) {
    tlh_event_destroy(c.stage_event[i]);
    tlh_host_free(c.stage_host[i]);
  }
  tlh_free(c.compare_scratch);
  tlh_stream_destroy(c.side);
  tlh_stream_destroy(c.stream);
  g_ctx.reset();
}

bool initialised() { return g_ctx != nullptr; }
int device() { return ctx().device; }
void *stream() { return ctx().stream; }

void empty_cache() {
  Context &c = ctx();
  detail::check(tlh_stream_synchronize(c.stream), "hipStreamSynchronize");
  std::lock_guard<std::mutex> lock(c.mu);
  free_cached(c);
}

MemoryStats memory_stats() {
  Context &c = ctx();
  std::lock_guard<std::mutex> lock(c.mu);
  return c.stats;
}

namespace detail {

void check(int code, const char *what) {
  if (code != 0)
    throw std::runtime_error(std::string(what) + " failed: " + tlh_error_string(code) + " (" +
                             std::to_string(code) + ")");
}

namespace {
AccessHook g_access_hook = nullptr;
} // namespace

void set_access_hook(AccessHook hook) noexcept { g_access_hook = hook; }

void before_access(const void *base, int kind) {
  if (g_access_hook && base) g_access_hook(base, kind);
}

void drop_deferred_views() {
  if (g_access_hook) g_access_hook(nullptr, kAccessShutdown);
}

bool capturing() {
  if (!g_ctx) return false;
  int cap = 0;
  check(tlh_stream_is_capturing(g_ctx->stream, &cap), "hipStreamIsCapturing");
  return cap != 0;
}

void *allocate(size_t bytes) {
  if (bytes == 0) return nullptr;
  Context &c = ctx();
  const size_t cls = size_class(bytes);
  std::lock_guard<std::mutex> lock(c.mu);
  auto it = c.free_blocks.find(cls);
  void *p = nullptr;
  if (it != c.free_blocks.end() && !it->second.empty()) {
    p = it->second.back();
    it->second.pop_back();
    c.stats.cached_bytes -= cls;
  } else {
    int st = tlh_malloc(&p, cls);
    if (st != 0) {
      // Out of memory with blocks parked: return them and try once more.
      // Only safe when nothing queued can still touch them.
      tlh_stream_synchronize(c.stream);
      free_cached(c);
      st = tlh_malloc(&p, cls);
    }
    check(st, "hipMalloc");
    c.stats.device_allocations += 1;
  }
  c.stats.in_use_bytes += cls;
  if (c.stats.in_use_bytes > c.stats.peak_bytes) c.stats.peak_bytes = c.stats.in_use_bytes;
  return p;
}

void release(void *ptr, size_t bytes) noexcept {
  if (!ptr) return;
  if (!g_ctx) { // storage outliving hip::shutdown(): hand it straight back
    tlh_free(ptr);
    return;
  }
  Context &c = *g_ctx;
  const size_t cls = size_class(bytes);
  std::lock_guard<std::mutex> lock(c.mu);
  try {
    if (c.defer)
      c.deferred.emplace_back(cls, ptr);
    else
      c.free_blocks[cls].push_back(ptr);
    c.stats.cached_bytes += cls;
  } catch (...) {
    tlh_free(ptr);
  }
  c.stats.in_use_bytes -= cls;
}

void defer_releases(bool on) noexcept {
  if (!g_ctx) return;
  Context &c = *g_ctx;
  std::lock_guard<std::mutex> lock(c.mu);
  c.defer = on;
  if (!on) {
    try {
      pool_deferred(c);
    } catch (...) { // out of host memory: hand the blocks back to HIP instead
      for (auto &[cls, p] : c.deferred) {
        tlh_free(p);
        c.stats.cached_bytes -= cls;
      }
      c.deferred.clear();
    }
  }
}

void write(void *dst, const void *src, size_t bytes) {
  Context &c = ctx();
  bool sync_side = false;
  void *s = transfer_stream(c, sync_side);
  if (!sync_side && bytes <= kStageSlot) {
    std::lock_guard<std::mutex> lock(c.mu);
    const int slot = c.stage_next;
    c.stage_next = (c.stage_next + 1) % kStageSlots;
    check(tlh_event_synchronize(c.stage_event[slot]), "hipEventSynchronize");
    std::memcpy(c.stage_host[slot], src, bytes);
    check(tlh_memcpy_h2d(dst, c.stage_host[slot], bytes, s), "hipMemcpyAsync");
    check(tlh_event_record(c.stage_event[slot], s), "hipEventRecord");
    return;
  }
  check(tlh_memcpy_h2d(dst, src, bytes, s), "hipMemcpyAsync");
  check(tlh_stream_synchronize(s), "hipStreamSynchronize");
}

void read(void *dst, const void *src, size_t bytes) {
  Context &c = ctx();
  bool sync_side = false;
  void *s = transfer_stream(c, sync_side);
  check(tlh_memcpy_d2h(dst, src, bytes, s), "hipMemcpyAsync");
  check(tlh_stream_synchronize(s), "hipStreamSynchronize");
}

void fill32(void *dst, uint32_t pattern, size_t count) {
  Context &c = ctx();
  bool sync_side = false;
  void *s = transfer_stream(c, sync_side);
  check(tlh_fill_u32(static_cast<uint32_t *>(dst), pattern, count, s), "fill");
  if (sync_side) check(tlh_stream_synchronize(s), "hipStreamSynchronize");
}

void copy(void *dst, const void *src, size_t bytes) {
  Context &c = ctx();
  bool sync_side = false;
  void *s = transfer_stream(c, sync_side);
  check(tlh_memcpy_d2d(dst, src, bytes, s), "hipMemcpyAsync");
  if (sync_side) check(tlh_stream_synchronize(s), "hipStreamSynchronize");
}

bool equal(const void *a, const void *b, size_t bytes) {
  Context &c = ctx();
  bool sync_side = false;
  void *s = transfer_stream(c, sync_side);
  int eq = 0;
  check(tlh_compare(a, b, bytes, &eq, c.compare_scratch, s), "compare");
  return eq != 0;
}

} // namespace detail
} // namespace hip
