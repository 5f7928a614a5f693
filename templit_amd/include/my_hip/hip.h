// hip::HIP -- the device tag of the MI355X backend, and the process-wide
// device context every Storage<hip::HIP, T> and hip::Runtime shares.
//
// Stands in for metal::Metal / metal::init / metal::shutdown / metal::device
// (include/my_metal/metal.h:5-15, src/my_metal/metal.cpp:18-38):
//   - kernel_type = float and index_type = uint32_t as on Metal;
//   - init(device) selects the GPU once and creates the context: one
//     in-order HIP stream that all device work of the process is enqueued
//     on (the Metal backend's single serial command queue), a caching
//     device-memory pool and a side stream for host transfers made while
//     the main stream is being recorded into a graph;
//   - init is idempotent; a second init naming another device throws
//     std::logic_error; shutdown releases the pool and streams and may be
//     followed by init again.
// All device access goes through the C-ABI of include/templit_hip.h.
#pragma once

#include <cstddef>
#include <cstdint>

namespace hip {

struct HIP {};
using kernel_type = float;
using index_type = uint32_t;

void init(int device = 0);
void shutdown();
bool initialised();
int device();

// The stream (hipStream_t) all runtimes and storages enqueue on.
void *stream();

// Releases every cached, unused device block (hipFree).
void empty_cache();

struct MemoryStats {
  size_t in_use_bytes = 0;    // bytes held by live storages
  size_t cached_bytes = 0;    // bytes parked in the pool, free for reuse
  size_t peak_bytes = 0;      // high-water mark of in_use_bytes
  size_t device_allocations = 0; // hipMalloc calls made by the pool
};
MemoryStats memory_stats();

namespace detail {
// Device memory from the caching pool. Blocks are reused only in stream
// order: every kernel, fill and transfer runs on the one context stream, so
// a block freed while queued work still reads it is not written before that
// work has finished.
void *allocate(size_t bytes);
void release(void *ptr, size_t bytes) noexcept;
// While on (hip::Runtime turns it on for a graph capture), released blocks
// are held back from reuse; turning it off returns them to the pool. A
// captured graph runs after record-time host writes, so a block that one
// captured kernel used and a later tensor of the same capture received
// would have that tensor's recorded contents overwritten at launch.
void defer_releases(bool on) noexcept;

// Host <-> device transfers, synchronous for the host (the host buffer may
// be reused on return) and ordered after the work already on the stream.
// While the stream is being captured into a graph they run immediately on
// the side stream instead, i.e. at record time, like a write into a Metal
// shared buffer while a command buffer is being encoded.
void write(void *dst, const void *src, size_t bytes);
void read(void *dst, const void *src, size_t bytes);
// dst[i] = pattern for `count` 32-bit words; device copy; byte equality.
void fill32(void *dst, uint32_t pattern, size_t count);
void copy(void *dst, const void *src, size_t bytes);
bool equal(const void *a, const void *b, size_t bytes);

bool capturing();
// Throws std::runtime_error naming `what` when `code` (a hipError_t) != 0.
void check(int code, const char *what);

// Deferred device work on a storage block: hip::Runtime keeps some results
// as views to be materialised later (a transpose or copy that only a matrix
// product or broadcast op reads). Storage calls the installed hook with the
// block's base pointer before host access -- kAccessRead, kAccessWrite --
// and before releasing it (kAccessRelease, which must not throw); shutdown()
// calls it with kAccessShutdown (and no block) before the context goes.
enum AccessKind : int { kAccessRead = 0, kAccessWrite = 1, kAccessRelease = 2, kAccessShutdown = 3 };
using AccessHook = void (*)(const void *base, int kind);
void set_access_hook(AccessHook hook) noexcept;
void before_access(const void *base, int kind);
void drop_deferred_views();
} // namespace detail

} // namespace hip
