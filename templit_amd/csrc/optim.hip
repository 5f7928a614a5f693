// Gradient clipping and AdamW.
//
// Reference: clip_gradient (math.metal:985-1006) and adamW (1008-1043),
// launched once per gradient tensor from Compiled::step(max_norm)
// (include/passes/compile.h:236-258) and Optimiser::AdamW::update
// (include/optimiser/AdamW.h:73-82): 52 clip + 52 AdamW launches per GPT
// step, each re-reading the gradient.
// tlh_adamw_multi does clip + AdamW for every tensor in one launch, reading
// param, grad, m, v once and writing param, m, v once (28 bytes/param).
#include "common.h"

#include "../../include/templit_hip.h"

using namespace tlh;

namespace {

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__device__ inline float clip_scale(float squared_norm, float max_norm) {
  return fminf(1.0f, max_norm * rsqrtf(fmaxf(squared_norm, 1e-12f)));
}

__global__ __launch_bounds__(256) void clip_kernel(const float *__restrict__ g,
                                                   const float *__restrict__ squared_norm,
                                                   float max_norm, float *out, size_t n) {
  const float scale = clip_scale(*squared_norm, max_norm);
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    out[i] = g[i] * scale;
}

constexpr uint32_t kClipChunk = 4096; // elements per work item (multiple of 4)

// Multi-tensor clip: work items are (tensor, 4096-element chunk) pairs
// numbered across all tensors (a chunk map in LDS); block b takes items b,
// b+G, ... . Each element is src * scale, as in clip_kernel; dst may be src.
__global__ __launch_bounds__(256) void clip_multi_kernel(const float *const *__restrict__ srcs,
                                                         float *const *__restrict__ dsts,
                                                         const uint64_t *__restrict__ sizes,
                                                         uint32_t count,
                                                         const float *__restrict__ squared_norm,
                                                         float max_norm) {
  __shared__ uint32_t first[kMaxMultiTensors + 1];
  const uint32_t total = build_chunk_map(first, count, [&](uint32_t t) {
    return uint32_t((sizes[t] + kClipChunk - 1) / kClipChunk);
  });
  const float scale = clip_scale(*squared_norm, max_norm);
  for (uint32_t it = blockIdx.x; it < total; it += gridDim.x) {
    const uint32_t t = chunk_owner(first, count, it);
    const uint64_t n = sizes[t];
    const float *src = srcs[t];
    float *dst = dsts[t];
    const uint64_t begin = uint64_t(it - first[t]) * kClipChunk;
    const uint64_t end = begin + kClipChunk < n ? begin + kClipChunk : n;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    if (vec && end - begin == kClipChunk) {
      for (uint64_t i = begin + threadIdx.x * 4; i < end; i += blockDim.x * 4) {
        f4 v = *reinterpret_cast<const f4 *>(src + i);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = v[q] * scale;
        *reinterpret_cast<f4 *>(dst + i) = v;
      }
    } else {
      for (uint64_t i = begin + threadIdx.x; i < end; i += blockDim.x) dst[i] = src[i] * scale;
    }
  }
}

// One AdamW element update, in the operation order of math.metal:1008-1043.
__device__ inline float adamw_update(float p, float g, float &m, float &v, float b1, float b2,
                                     float decay, float lr, float eps, float c1, float c2) {
  m = b1 * m + (1.0f - b1) * g;
  v = b2 * v + (1.0f - b2) * g * g;
  return p * decay - lr * (m / c1) / (sqrtf(v / c2) + eps);
}

__global__ __launch_bounds__(256) void adamw_kernel(const float *param, const float *grad,
                                                    float *out, float *m1, float *m2,
                                                    const float *__restrict__ beta1,
                                                    const float *__restrict__ beta2,
                                                    const float *__restrict__ decay,
                                                    const float *__restrict__ lr, float eps,
                                                    uint32_t step, size_t n) {
  const float b1 = *beta1, b2 = *beta2, dc = *decay, l = *lr;
  const float c1 = 1.0f - powf(b1, float(step));
  const float c2 = 1.0f - powf(b2, float(step));
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    float m = m1[i], v = m2[i];
    const float p = adamw_update(param[i], grad[i], m, v, b1, b2, dc, l, eps, c1, c2);
    m1[i] = m;
    m2[i] = v;
    out[i] = p;
  }
}

constexpr uint32_t kChunk = 4096; // elements per work item (multiple of 4)

// Multi-tensor clip + AdamW. Work items are (tensor, 4096-element chunk)
// pairs numbered across all tensors (a chunk map in LDS); block b takes
// items b, b+G, ... .
__global__ __launch_bounds__(256) void adamw_multi_kernel(
    float *const *__restrict__ params, const float *const *__restrict__ grads,
    float *const *__restrict__ m1s, float *const *__restrict__ m2s,
    const uint64_t *__restrict__ sizes, const uint32_t *__restrict__ steps, uint32_t count,
    const float *__restrict__ beta1, const float *__restrict__ beta2,
    const float *__restrict__ decay, const float *__restrict__ lr, float eps,
    const float *__restrict__ squared_norm, float max_norm) {
  __shared__ uint32_t first[kMaxMultiTensors + 1];
  const uint32_t total = build_chunk_map(
      first, count, [&](uint32_t t) { return uint32_t((sizes[t] + kChunk - 1) / kChunk); });
  const float b1 = *beta1, b2 = *beta2, dc = *decay, l = *lr;
  const float scale = squared_norm ? clip_scale(*squared_norm, max_norm) : 1.0f;
  for (uint32_t it = blockIdx.x; it < total; it += gridDim.x) {
    const uint32_t t = chunk_owner(first, count, it);
    const uint64_t n = sizes[t];
    float *p = params[t];
    const float *g = grads[t];
    float *m1 = m1s[t];
    float *m2 = m2s[t];
    const float step = float(steps[t]);
    const float c1 = 1.0f - powf(b1, step);
    const float c2 = 1.0f - powf(b2, step);
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) |
                       reinterpret_cast<uintptr_t>(m1) | reinterpret_cast<uintptr_t>(m2)) &
                      15) == 0;
    const uint64_t begin = uint64_t(it - first[t]) * kChunk;
    const uint64_t end = begin + kChunk < n ? begin + kChunk : n;
    if (vec && end - begin == kChunk) {
      for (uint64_t i = begin + threadIdx.x * 4; i < end; i += blockDim.x * 4) {
        f4 pv = *reinterpret_cast<const f4 *>(p + i);
        const f4 gv = *reinterpret_cast<const f4 *>(g + i);
        f4 mv = *reinterpret_cast<const f4 *>(m1 + i);
        f4 vv = *reinterpret_cast<const f4 *>(m2 + i);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float m = mv[q], vq = vv[q];
          pv[q] = adamw_update(pv[q], gv[q] * scale, m, vq, b1, b2, dc, l, eps, c1, c2);
          mv[q] = m;
          vv[q] = vq;
        }
        *reinterpret_cast<f4 *>(p + i) = pv;
        *reinterpret_cast<f4 *>(m1 + i) = mv;
        *reinterpret_cast<f4 *>(m2 + i) = vv;
      }
    } else {
      for (uint64_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        float m = m1[i], v = m2[i];
        p[i] = adamw_update(p[i], g[i] * scale, m, v, b1, b2, dc, l, eps, c1, c2);
        m1[i] = m;
        m2[i] = v;
      }
    }
  }
}

} // namespace

TLH_API int tlh_clip_gradient(const float *g, const float *squared_norm, float max_norm,
                              float *out, size_t n, void *stream) {
  if (n == 0) return 0;
  clip_kernel<<<stride_grid(n, 256), 256, 0, as_stream(stream)>>>(g, squared_norm, max_norm, out,
                                                                  n);
  return launch_status();
}

TLH_API int tlh_clip_multi(const float *const *srcs, float *const *dsts, const uint64_t *sizes,
                           uint32_t count, const float *squared_norm, float max_norm,
                           void *stream) {
  if (count == 0) return 0;
  if (count > kMaxMultiTensors || !squared_norm) return int(hipErrorInvalidValue);
  clip_multi_kernel<<<1024, 256, 0, as_stream(stream)>>>(srcs, dsts, sizes, count, squared_norm,
                                                         max_norm);
  return launch_status();
}

TLH_API int tlh_adamw(const float *param, const float *grad, float *out, float *m1, float *m2,
                      const float *beta1, const float *beta2, const float *decay,
                      const float *lr, float eps, uint32_t step, size_t n, void *stream) {
  if (step == 0) return int(hipErrorInvalidValue);
  if (n == 0) return 0;
  adamw_kernel<<<stride_grid(n, 256), 256, 0, as_stream(stream)>>>(
      param, grad, out, m1, m2, beta1, beta2, decay, lr, eps, step, n);
  return launch_status();
}

TLH_API int tlh_adamw_multi(float *const *params, const float *const *grads, float *const *m1,
                            float *const *m2, const uint64_t *sizes, const uint32_t *steps,
                            uint32_t count, const float *beta1, const float *beta2,
                            const float *decay, const float *lr, float eps,
                            const float *squared_norm, float max_norm, void *stream) {
  if (count == 0) return 0;
  if (count > kMaxMultiTensors) return int(hipErrorInvalidValue);
  adamw_multi_kernel<<<1024, 256, 0, as_stream(stream)>>>(params, grads, m1, m2, sizes, steps,
                                                          count, beta1, beta2, decay, lr, eps,
                                                          squared_norm, max_norm);
  return launch_status();
}
