// Shared device/host helpers for the gfx950 kernels of libtemplit_hip.
//
// Every kernel in this library is written for CDNA4 (gfx950): 64-lane
// wavefronts, fp32 MFMA, 160 KiB LDS per CU, 256 CUs in 8 XCDs.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#define TLH_API extern "C" __attribute__((visibility("default")))

namespace tlh {

constexpr int kWave = 64;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));

// Return code of every entry point: hipError_t as int (0 = success).
inline int launch_status() { return static_cast<int>(hipGetLastError()); }

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned ceil_div(size_t a, size_t b) {
  return static_cast<unsigned>((a + b - 1) / b);
}

// Grid size for a grid-stride elementwise kernel: enough blocks to fill all
// 256 CUs several times over, never more than the work needs.
inline unsigned stride_grid(size_t n, unsigned block, unsigned per_thread = 1) {
  size_t need = (n + size_t(block) * per_thread - 1) / (size_t(block) * per_thread);
  if (need < 1) need = 1;
  const size_t cap = 256 * 16;
  return static_cast<unsigned>(need < cap ? need : cap);
}

// ---- wavefront reductions (64 lanes, DPP/permute via __shfl_xor) ----------
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `scratch` needs
// blockDim.x/64 floats of LDS. Result is broadcast to every thread.
__device__ inline float block_sum(float v, float *scratch) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += scratch[i];
  return t;
}

__device__ inline float block_max(float v, float *scratch) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) t = fmaxf(t, scratch[i]);
  return t;
}

// tanh-approximation GELU with the constants of the reference kernels
// (include/my_metal/math.metal:821-855). The forward kernel evaluates
// sqrt(2.0f / 3.14159265f) in fp32 (= 0x1.988452p-1) while the derivative
// kernel uses the literal 0.7978845608f (= 0x1.988454p-1); both are kept.
constexpr float kGeluFwdA = 0x1.988452p-1f; // sqrtf(2.0f / 3.14159265f)
constexpr float kGeluA = 0.7978845608f;     // derivative's sqrt(2/pi)
constexpr float kGeluB = 0.044715f;

__device__ inline float gelu_fwd(float x) {
  const float u = kGeluFwdA * (x + kGeluB * x * x * x);
  return 0.5f * x * (1.0f + tanhf(u));
}

__device__ inline float gelu_grad(float x) {
  const float x2 = x * x;
  const float t = tanhf(kGeluA * (x + kGeluB * x2 * x));
  return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * kGeluA * (1.0f + 3.0f * kGeluB * x2);
}

// ---- multi-tensor chunk maps -----------------------------------------------
// The tensors of a multi-tensor launch are cut into chunks numbered across
// all tensors; first[t] is tensor t's first chunk and first[count] the total.
// A block builds the map in LDS (256 threads, count <= kMaxMultiTensors) from
// chunks_of(t), so that chunk c's tensor is a binary search away instead of
// a walk over the device-side tensor table.
constexpr uint32_t kMaxMultiTensors = 2048;

template <typename ChunksOf>
__device__ inline uint32_t build_chunk_map(uint32_t *first, uint32_t count, ChunksOf chunks_of) {
  __shared__ uint32_t wave_total[4];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t per = (count + 255) / 256;
  const uint32_t b = min(count, tid * per), e = min(count, b + per);
  uint32_t sum = 0;
  for (uint32_t t = b; t < e; ++t) sum += chunks_of(t);
  uint32_t incl = sum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t x = __shfl_up(incl, o, 64);
    if (int(lane) >= o) incl += x;
  }
  if (lane == 63) wave_total[wave] = incl;
  __syncthreads();
  uint32_t acc = incl - sum, total = 0;
#pragma unroll
  for (uint32_t w = 0; w < 4; ++w) {
    if (w < wave) acc += wave_total[w];
    total += wave_total[w];
  }
  for (uint32_t t = b; t < e; ++t) { // (chunks_of again: a few table reads)
    first[t] = acc;
    acc += chunks_of(t);
  }
  if (tid == 0) first[count] = total;
  __syncthreads();
  return total;
}

// The tensor holding chunk c: the last t with first[t] <= c (skips empty tensors).
__device__ inline uint32_t chunk_owner(const uint32_t *first, uint32_t count, uint32_t c) {
  uint32_t lo = 0, hi = count; // first[lo] <= c < first[hi]
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (first[mid] <= c) lo = mid;
    else hi = mid;
  }
  return lo;
}

} // namespace tlh
