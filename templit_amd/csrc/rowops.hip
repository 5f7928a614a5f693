// Row operations: softmax (+ backward), cross-entropy (+ backward, fused
// forward/backward), RMS, RMSNorm (+ backward).
//
// Reference: softmax math.metal:857-882 and cross_entropy_rows(_backward)
// 884-953 run one thread per row with 3 passes over global memory; RMS and
// RMSNorm are 5-6 separate kernels (src/my_metal/runtime.cpp:1031-1072) and
// RMSNorm' is 7 runtime calls (include/passes/execute.h:330-356).
// Here one 64-lane wave owns a row: the row is read once into registers as
// float4s (up to 2048 columns), reduced with wave shuffles, and written once,
// so each kernel moves the minimum bytes (read x, write y).
#include "common.h"

#include "../../include/templit_hip.h"

using namespace tlh;

namespace {

constexpr int kBlock = 256; // 4 waves = 4 rows in flight per block

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline unsigned row_grid(size_t rows) {
  const size_t blocks = (rows + 3) / 4;
  return unsigned(blocks < 256 * 32 ? (blocks ? blocks : 1) : 256 * 32);
}

struct WaveRow {
  int lane;
  size_t row0, nrows; // first row of this wave, row stride across the grid
};

__device__ inline WaveRow wave_rows() {
  WaveRow w;
  w.lane = threadIdx.x & 63;
  w.row0 = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  w.nrows = (size_t(gridDim.x) * blockDim.x) >> 6;
  return w;
}

// Loads a row as V float4 per lane (element (k*64+lane)*4 .. +3); lanes past
// `cols` get `fill`.
template <int V>
__device__ inline void load_row(const float *row, uint32_t cols, int lane, f4 (&v)[V],
                                float fill) {
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const uint32_t idx = (uint32_t(k) * 64 + lane) * 4;
    if (idx < cols) v[k] = *reinterpret_cast<const f4 *>(row + idx);
    else v[k] = f4{fill, fill, fill, fill};
  }
}

template <int V>
__device__ inline void store_row(float *row, uint32_t cols, int lane, const f4 (&v)[V]) {
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const uint32_t idx = (uint32_t(k) * 64 + lane) * 4;
    if (idx < cols) *reinterpret_cast<f4 *>(row + idx) = v[k];
  }
}

template <int V> __device__ inline float row_max(const f4 (&v)[V]) {
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < V; ++k) m = fmaxf(fmaxf(m, fmaxf(v[k].x, v[k].y)), fmaxf(v[k].z, v[k].w));
  return wave_max(m);
}

// ---------------------------------------------------------------------------
// softmax
// ---------------------------------------------------------------------------
template <int V>
__global__ __launch_bounds__(kBlock) void softmax_v_kernel(const float *__restrict__ x,
                                                           float *__restrict__ out, size_t rows,
                                                           uint32_t cols) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    f4 v[V];
    load_row<V>(x + r * cols, cols, w.lane, v, -INFINITY);
    const float m = row_max<V>(v);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      v[k].x = expf(v[k].x - m); v[k].y = expf(v[k].y - m);
      v[k].z = expf(v[k].z - m); v[k].w = expf(v[k].w - m);
      s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    s = wave_sum(s);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      v[k].x = v[k].x / s; v[k].y = v[k].y / s; v[k].z = v[k].z / s; v[k].w = v[k].w / s;
    }
    store_row<V>(out + r * cols, cols, w.lane, v);
  }
}

__global__ __launch_bounds__(kBlock) void softmax_loop_kernel(const float *__restrict__ x,
                                                              float *__restrict__ out,
                                                              size_t rows, uint32_t cols) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    const float *row = x + r * cols;
    float m = -INFINITY;
    for (uint32_t j = w.lane; j < cols; j += 64) m = fmaxf(m, row[j]);
    m = wave_max(m);
    float s = 0.f;
    for (uint32_t j = w.lane; j < cols; j += 64) s += expf(row[j] - m);
    s = wave_sum(s);
    for (uint32_t j = w.lane; j < cols; j += 64) out[r * cols + j] = expf(row[j] - m) / s;
  }
}

// out = y * (g - sum(g*y))
template <int V>
__global__ __launch_bounds__(kBlock) void softmax_bwd_v_kernel(const float *__restrict__ g,
                                                               const float *__restrict__ y,
                                                               float *out, size_t rows,
                                                               uint32_t cols) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    f4 gv[V], yv[V];
    load_row<V>(g + r * cols, cols, w.lane, gv, 0.f);
    load_row<V>(y + r * cols, cols, w.lane, yv, 0.f);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k)
      s += (gv[k].x * yv[k].x + gv[k].y * yv[k].y) + (gv[k].z * yv[k].z + gv[k].w * yv[k].w);
    s = wave_sum(s);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      gv[k].x = yv[k].x * (gv[k].x - s); gv[k].y = yv[k].y * (gv[k].y - s);
      gv[k].z = yv[k].z * (gv[k].z - s); gv[k].w = yv[k].w * (gv[k].w - s);
    }
    store_row<V>(out + r * cols, cols, w.lane, gv);
  }
}

__global__ __launch_bounds__(kBlock) void softmax_bwd_loop_kernel(const float *__restrict__ g,
                                                                  const float *__restrict__ y,
                                                                  float *out, size_t rows,
                                                                  uint32_t cols) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    float s = 0.f;
    for (uint32_t j = w.lane; j < cols; j += 64) s += g[r * cols + j] * y[r * cols + j];
    s = wave_sum(s);
    for (uint32_t j = w.lane; j < cols; j += 64) {
      const float yy = y[r * cols + j];
      out[r * cols + j] = yy * (g[r * cols + j] - s);
    }
  }
}

// ---------------------------------------------------------------------------
// cross-entropy: loss = max + log(sum exp(x-max)) - x[t]; grad = p - onehot.
// mode bit 0: write losses; bit 1: write grad.
// ---------------------------------------------------------------------------
template <int V>
__global__ __launch_bounds__(kBlock) void ce_v_kernel(const float *__restrict__ logits,
                                                      const uint32_t *__restrict__ targets,
                                                      float *__restrict__ losses,
                                                      float *__restrict__ grad, size_t rows,
                                                      uint32_t vocab,
                                                      const float *__restrict__ row_scale,
                                                      float scale, int mode) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    const uint32_t t = targets[r];
    if (t >= vocab) { // invalid target -> +INF (math.metal:893-896, 921-926)
      if (mode & 1) {
        if (w.lane == 0) losses[r] = INFINITY;
      }
      if (mode & 2)
        for (uint32_t j = w.lane; j < vocab; j += 64) grad[r * vocab + j] = INFINITY;
      continue;
    }
    const float *row = logits + r * vocab;
    f4 v[V];
    load_row<V>(row, vocab, w.lane, v, -INFINITY);
    const float m = row_max<V>(v);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      v[k].x = expf(v[k].x - m); v[k].y = expf(v[k].y - m);
      v[k].z = expf(v[k].z - m); v[k].w = expf(v[k].w - m);
      s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    s = wave_sum(s);
    if ((mode & 1) && w.lane == 0) losses[r] = m + logf(s) - row[t];
    if (mode & 2) {
      const float sc = scale * (row_scale ? row_scale[r] : 1.0f);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const uint32_t base = (uint32_t(k) * 64 + w.lane) * 4;
        float p[4] = {v[k].x / s, v[k].y / s, v[k].z / s, v[k].w / s};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (base + q == t) p[q] -= 1.0f;
        v[k] = f4{p[0] * sc, p[1] * sc, p[2] * sc, p[3] * sc};
      }
      store_row<V>(grad + r * vocab, vocab, w.lane, v);
    }
  }
}

__global__ __launch_bounds__(kBlock) void ce_loop_kernel(const float *__restrict__ logits,
                                                         const uint32_t *__restrict__ targets,
                                                         float *__restrict__ losses,
                                                         float *__restrict__ grad, size_t rows,
                                                         uint32_t vocab,
                                                         const float *__restrict__ row_scale,
                                                         float scale, int mode) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    const uint32_t t = targets[r];
    if (t >= vocab) {
      if ((mode & 1) && w.lane == 0) losses[r] = INFINITY;
      if (mode & 2)
        for (uint32_t j = w.lane; j < vocab; j += 64) grad[r * vocab + j] = INFINITY;
      continue;
    }
    const float *row = logits + r * vocab;
    float m = -INFINITY;
    for (uint32_t j = w.lane; j < vocab; j += 64) m = fmaxf(m, row[j]);
    m = wave_max(m);
    float s = 0.f;
    for (uint32_t j = w.lane; j < vocab; j += 64) s += expf(row[j] - m);
    s = wave_sum(s);
    if ((mode & 1) && w.lane == 0) losses[r] = m + logf(s) - row[t];
    if (mode & 2) {
      const float sc = scale * (row_scale ? row_scale[r] : 1.0f);
      for (uint32_t j = w.lane; j < vocab; j += 64) {
        float p = expf(row[j] - m) / s;
        if (j == t) p -= 1.0f;
        grad[r * vocab + j] = p * sc;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// RMS / RMSNorm: rms = sqrt(sum(x^2)/D + eps); y = x / rms (* gain)
// ---------------------------------------------------------------------------
template <int V>
__global__ __launch_bounds__(kBlock) void rmsnorm_v_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ gain,
                                                           float *__restrict__ y,
                                                           float *__restrict__ rms_out,
                                                           size_t rows, uint32_t cols, float eps) {
  const WaveRow w = wave_rows();
  f4 gv[V];
  if (gain) load_row<V>(gain, cols, w.lane, gv, 0.f);
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    f4 v[V];
    load_row<V>(x + r * cols, cols, w.lane, v, 0.f);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k)
      s += (v[k].x * v[k].x + v[k].y * v[k].y) + (v[k].z * v[k].z + v[k].w * v[k].w);
    s = wave_sum(s);
    const float rms = sqrtf(s / float(cols) + eps);
    if (rms_out && w.lane == 0) rms_out[r] = rms;
    if (y) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        v[k].x = v[k].x / rms; v[k].y = v[k].y / rms; v[k].z = v[k].z / rms; v[k].w = v[k].w / rms;
        if (gain) {
          v[k].x *= gv[k].x; v[k].y *= gv[k].y; v[k].z *= gv[k].z; v[k].w *= gv[k].w;
        }
      }
      store_row<V>(y + r * cols, cols, w.lane, v);
    }
  }
}

__global__ __launch_bounds__(kBlock) void rmsnorm_loop_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ gain,
                                                              float *__restrict__ y,
                                                              float *__restrict__ rms_out,
                                                              size_t rows, uint32_t cols,
                                                              float eps) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    const float *row = x + r * cols;
    float s = 0.f;
    for (uint32_t j = w.lane; j < cols; j += 64) s += row[j] * row[j];
    s = wave_sum(s);
    const float rms = sqrtf(s / float(cols) + eps);
    if (rms_out && w.lane == 0) rms_out[r] = rms;
    if (y)
      for (uint32_t j = w.lane; j < cols; j += 64) {
        float v = row[j] / rms;
        if (gain) v *= gain[j];
        y[r * cols + j] = v;
      }
  }
}

// dx = beta*dx + (gy - n*mean(gy*n))/rms with n = x/rms, gy = g*gain;
// grad_gain[c] += sum_r g*n (atomics, pre-zeroed by the host wrapper).
template <int V>
__global__ __launch_bounds__(kBlock) void rmsnorm_bwd_v_kernel(
    const float *__restrict__ g, const float *__restrict__ x, const float *__restrict__ gain,
    float *dx, float *__restrict__ grad_gain, size_t rows, uint32_t cols, float eps,
    float beta) {
  const WaveRow w = wave_rows();
  f4 gnv[V], acc[V];
  if (gain) load_row<V>(gain, cols, w.lane, gnv, 0.f);
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
  const float inv_d = 1.0f / float(cols);
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    f4 xv[V], gv[V];
    load_row<V>(x + r * cols, cols, w.lane, xv, 0.f);
    load_row<V>(g + r * cols, cols, w.lane, gv, 0.f);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k)
      ss += (xv[k].x * xv[k].x + xv[k].y * xv[k].y) + (xv[k].z * xv[k].z + xv[k].w * xv[k].w);
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / float(cols) + eps);
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      xv[k].x /= rms; xv[k].y /= rms; xv[k].z /= rms; xv[k].w /= rms; // n
      if (grad_gain) {
        acc[k].x += gv[k].x * xv[k].x; acc[k].y += gv[k].y * xv[k].y;
        acc[k].z += gv[k].z * xv[k].z; acc[k].w += gv[k].w * xv[k].w;
      }
      if (gain) {
        gv[k].x *= gnv[k].x; gv[k].y *= gnv[k].y; gv[k].z *= gnv[k].z; gv[k].w *= gnv[k].w;
      }
      dot += (gv[k].x * xv[k].x + gv[k].y * xv[k].y) + (gv[k].z * xv[k].z + gv[k].w * xv[k].w);
    }
    const float m = wave_sum(dot) * inv_d;
    f4 o[V];
    if (beta != 0.f) load_row<V>(dx + r * cols, cols, w.lane, o, 0.f);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      f4 d;
      d.x = (gv[k].x - xv[k].x * m) / rms; d.y = (gv[k].y - xv[k].y * m) / rms;
      d.z = (gv[k].z - xv[k].z * m) / rms; d.w = (gv[k].w - xv[k].w * m) / rms;
      if (beta != 0.f) {
        d.x += beta * o[k].x; d.y += beta * o[k].y; d.z += beta * o[k].z; d.w += beta * o[k].w;
      }
      o[k] = d;
    }
    store_row<V>(dx + r * cols, cols, w.lane, o);
  }
  if (grad_gain) {
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const uint32_t idx = (uint32_t(k) * 64 + w.lane) * 4;
      if (idx < cols) {
        atomicAdd(grad_gain + idx, acc[k].x);
        atomicAdd(grad_gain + idx + 1, acc[k].y);
        atomicAdd(grad_gain + idx + 2, acc[k].z);
        atomicAdd(grad_gain + idx + 3, acc[k].w);
      }
    }
  }
}

__global__ __launch_bounds__(kBlock) void rmsnorm_bwd_loop_kernel(
    const float *__restrict__ g, const float *__restrict__ x, const float *__restrict__ gain,
    float *dx, float *__restrict__ grad_gain, size_t rows, uint32_t cols, float eps,
    float beta) {
  const WaveRow w = wave_rows();
  for (size_t r = w.row0; r < rows; r += w.nrows) {
    const float *xr = x + r * cols;
    const float *gr = g + r * cols;
    float ss = 0.f;
    for (uint32_t j = w.lane; j < cols; j += 64) ss += xr[j] * xr[j];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / float(cols) + eps);
    float dot = 0.f;
    for (uint32_t j = w.lane; j < cols; j += 64) {
      const float n = xr[j] / rms;
      const float gy = gain ? gr[j] * gain[j] : gr[j];
      dot += gy * n;
      if (grad_gain) atomicAdd(grad_gain + j, gr[j] * n);
    }
    const float m = wave_sum(dot) / float(cols);
    for (uint32_t j = w.lane; j < cols; j += 64) {
      const float n = xr[j] / rms;
      const float gy = gain ? gr[j] * gain[j] : gr[j];
      float d = (gy - n * m) / rms;
      if (beta != 0.f) d += beta * dx[r * cols + j];
      dx[r * cols + j] = d;
    }
  }
}

// Picks the register-cached kernel for cols % 4 == 0 and cols <= 2048.
inline int pick_v(uint32_t cols) {
  if (cols % 4 || cols > 2048) return 0;
  const uint32_t v4 = (cols + 255) / 256;
  if (v4 <= 1) return 1;
  if (v4 <= 2) return 2;
  if (v4 <= 4) return 4;
  return 8;
}

#define TLH_DISPATCH_V(V_, KERNEL, ...)                                                  \
  switch (V_) {                                                                          \
  case 1: KERNEL<1><<<grid, kBlock, 0, s>>>(__VA_ARGS__); break;                         \
  case 2: KERNEL<2><<<grid, kBlock, 0, s>>>(__VA_ARGS__); break;                         \
  case 4: KERNEL<4><<<grid, kBlock, 0, s>>>(__VA_ARGS__); break;                         \
  default: KERNEL<8><<<grid, kBlock, 0, s>>>(__VA_ARGS__); break;                        \
  }

int ce_launch(const float *logits, const uint32_t *targets, float *losses, float *grad,
              size_t rows, uint32_t vocab, const float *row_scale, float scale, int mode,
              void *stream) {
  if (rows == 0) return 0;
  if (vocab == 0) return int(hipErrorInvalidValue);
  hipStream_t s = as_stream(stream);
  const unsigned grid = row_grid(rows);
  const int v = (aligned16(logits) && (!grad || aligned16(grad))) ? pick_v(vocab) : 0;
  if (v) {
    TLH_DISPATCH_V(v, ce_v_kernel, logits, targets, losses, grad, rows, vocab, row_scale, scale,
                   mode)
  } else {
    ce_loop_kernel<<<grid, kBlock, 0, s>>>(logits, targets, losses, grad, rows, vocab, row_scale,
                                           scale, mode);
  }
  return launch_status();
}

} // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
TLH_API int tlh_softmax(const float *x, float *out, size_t rows, uint32_t cols, void *stream) {
  if (rows == 0) return 0;
  if (cols == 0) return int(hipErrorInvalidValue);
  hipStream_t s = as_stream(stream);
  const unsigned grid = row_grid(rows);
  const int v = (aligned16(x) && aligned16(out)) ? pick_v(cols) : 0;
  if (v) {
    TLH_DISPATCH_V(v, softmax_v_kernel, x, out, rows, cols)
  } else {
    softmax_loop_kernel<<<grid, kBlock, 0, s>>>(x, out, rows, cols);
  }
  return launch_status();
}

TLH_API int tlh_softmax_backward(const float *g, const float *y, float *out, size_t rows,
                                 uint32_t cols, void *stream) {
  if (rows == 0) return 0;
  if (cols == 0) return int(hipErrorInvalidValue);
  hipStream_t s = as_stream(stream);
  const unsigned grid = row_grid(rows);
  const int v = (aligned16(g) && aligned16(y) && aligned16(out)) ? pick_v(cols) : 0;
  if (v) {
    TLH_DISPATCH_V(v, softmax_bwd_v_kernel, g, y, out, rows, cols)
  } else {
    softmax_bwd_loop_kernel<<<grid, kBlock, 0, s>>>(g, y, out, rows, cols);
  }
  return launch_status();
}

TLH_API int tlh_cross_entropy_rows(const float *logits, const uint32_t *targets, float *losses,
                                   size_t rows, uint32_t vocab, void *stream) {
  return ce_launch(logits, targets, losses, nullptr, rows, vocab, nullptr, 1.0f, 1, stream);
}

TLH_API int tlh_cross_entropy_rows_backward(const float *logits, const uint32_t *targets,
                                            float *grad, size_t rows, uint32_t vocab,
                                            const float *row_scale, void *stream) {
  return ce_launch(logits, targets, nullptr, grad, rows, vocab, row_scale, 1.0f, 2, stream);
}

TLH_API int tlh_cross_entropy_rows_fused(const float *logits, const uint32_t *targets,
                                         float *losses, float *grad, size_t rows, uint32_t vocab,
                                         float scale, void *stream) {
  return ce_launch(logits, targets, losses, grad, rows, vocab, nullptr, scale, 3, stream);
}

TLH_API int tlh_rms(const float *x, float *rms, size_t rows, uint32_t cols, float eps,
                    void *stream) {
  return tlh_rms_norm(x, nullptr, nullptr, rms, rows, cols, eps, stream);
}

TLH_API int tlh_rms_norm(const float *x, const float *gain, float *y, float *rms_out,
                         size_t rows, uint32_t cols, float eps, void *stream) {
  if (rows == 0) return 0;
  if (cols == 0) return int(hipErrorInvalidValue);
  hipStream_t s = as_stream(stream);
  const unsigned grid = row_grid(rows);
  const int v = (aligned16(x) && (!y || aligned16(y)) && (!gain || aligned16(gain)))
                    ? pick_v(cols)
                    : 0;
  if (v) {
    TLH_DISPATCH_V(v, rmsnorm_v_kernel, x, gain, y, rms_out, rows, cols, eps)
  } else {
    rmsnorm_loop_kernel<<<grid, kBlock, 0, s>>>(x, gain, y, rms_out, rows, cols, eps);
  }
  return launch_status();
}

TLH_API int tlh_rms_norm_backward(const float *g, const float *x, const float *gain, float *dx,
                                  float *grad_gain, size_t rows, uint32_t cols, float eps,
                                  float beta, void *stream) {
  if (cols == 0) return int(hipErrorInvalidValue);
  hipStream_t s = as_stream(stream);
  if (grad_gain) {
    const int st = tlh_fill_f32(grad_gain, 0.0f, cols, stream);
    if (st) return st;
  }
  if (rows == 0) return 0;
  const unsigned grid = row_grid(rows);
  const int v = (aligned16(x) && aligned16(g) && aligned16(dx) && (!gain || aligned16(gain)))
                    ? pick_v(cols)
                    : 0;
  if (v) {
    TLH_DISPATCH_V(v, rmsnorm_bwd_v_kernel, g, x, gain, dx, grad_gain, rows, cols, eps, beta)
  } else {
    rmsnorm_bwd_loop_kernel<<<grid, kBlock, 0, s>>>(g, x, gain, dx, grad_gain, rows, cols, eps,
                                                    beta);
  }
  return launch_status();
}
