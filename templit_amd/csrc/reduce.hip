// Reductions: sum, sum_to_shape, max_to_shape, argmax, gradient norm,
// column sums.
//
// Reference kernels replaced (include/my_metal/math.metal): sum 549-564 (one
// thread over everything), sum_to_shape 618-679 and max_to_shape 681-714 (one
// thread per output, serial loop), argmax/argmax_reduce 715-777 (multi-pass,
// scratch buffers allocated per call, runtime.cpp:850-918), and
// accumulate_gradient_squared_norm 955-983.
// Here reductions are wavefront/block parallel: row reductions use one wave
// per row with shuffles, column reductions stripe rows over the threads of a
// block, and the leftover shapes fall back to a thread per output.
#include "common.h"

#include <algorithm>

#include "../../include/templit_hip.h"

using namespace tlh;

namespace {

constexpr int kMaxDims = 8;

template <bool MAX> __device__ inline float combine(float a, float b) {
  if constexpr (MAX) return b > a ? b : a;
  else return a + b;
}

template <bool MAX> __device__ inline float identity() {
  if constexpr (MAX) return -INFINITY;
  else return 0.0f;
}

template <bool MAX> __device__ inline float wave_reduce(float v) {
  if constexpr (MAX) return wave_max(v);
  else return wave_sum(v);
}

// ---- single-block total sum --------------------------------------------
__global__ __launch_bounds__(1024) void sum_all_kernel(const float *__restrict__ a, size_t n,
                                                       float *__restrict__ out, int accumulate) {
  __shared__ float scratch[16];
  float v = 0.0f;
  for (size_t i = threadIdx.x; i < n; i += blockDim.x) v += a[i];
  v = block_sum(v, scratch);
  if (threadIdx.x == 0) *out = accumulate ? *out + v : v;
}

// Partial sums of a large tensor (stage 1) -> `partials[blockIdx.x]`.
__global__ __launch_bounds__(256) void sum_partials_kernel(const float *__restrict__ a,
                                                           size_t n,
                                                           float *__restrict__ partials) {
  __shared__ float scratch[4];
  float v = 0.0f;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    v += a[i];
  v = block_sum(v, scratch);
  if (threadIdx.x == 0) partials[blockIdx.x] = v;
}

// ---- row reduce: out[r] = reduce(a[r, 0:cols]) -----------------------------
template <bool MAX>
__global__ __launch_bounds__(256) void row_reduce_kernel(const float *__restrict__ a,
                                                         float *__restrict__ out, size_t rows,
                                                         uint32_t cols) {
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const size_t nwaves = (size_t(gridDim.x) * blockDim.x) >> 6;
  for (size_t r = wave; r < rows; r += nwaves) {
    const float *row = a + r * cols;
    float v = identity<MAX>();
    for (uint32_t j = lane; j < cols; j += 64) v = combine<MAX>(v, row[j]);
    v = wave_reduce<MAX>(v);
    if (lane == 0) out[r] = v;
  }
}

// ---- column reduce: out[c] = beta*out[c] + reduce_r(a[r, c]) ---------------
// Block = 32 columns x 8 row groups.
template <bool MAX>
__global__ __launch_bounds__(256) void col_reduce_kernel(const float *__restrict__ a,
                                                         float *__restrict__ out, size_t rows,
                                                         uint32_t cols, float beta) {
  __shared__ float part[8][33];
  const int cx = threadIdx.x & 31, gy = threadIdx.x >> 5;
  const uint32_t c = blockIdx.x * 32 + cx;
  float v = identity<MAX>();
  if (c < cols)
    for (size_t r = gy; r < rows; r += 8) v = combine<MAX>(v, a[r * cols + c]);
  part[gy][cx] = v;
  __syncthreads();
  if (gy == 0 && c < cols) {
    float t = part[0][cx];
    for (int g = 1; g < 8; ++g) t = combine<MAX>(t, part[g][cx]);
    if (!MAX && beta != 0.0f) t += beta * out[c];
    out[c] = t;
  }
}

// ---- tall column sums, two passes (deterministic) -------------------------
// Pass 1: block (64-column group x, row chunk y) sums its chunk's rows for 64
// columns -- 16 threads x float4 across the columns, 16 row lanes, the lanes
// combined in a fixed order -- into partials[chunk][column]. Pass 2 adds each
// column's chunk partials in a fixed order (col_finish_kernel). Spreads [6144, 384]
// over 6 x 48 blocks where one block per 32 columns would use 12 CUs.
__global__ __launch_bounds__(256) void col_partials_kernel(const float *__restrict__ a,
                                                           float *__restrict__ partials,
                                                           size_t rows, uint32_t cols,
                                                           uint32_t chunk_rows) {
  __shared__ f4 part[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const uint32_t c = blockIdx.x * 64 + uint32_t(tx) * 4;
  const size_t r0 = size_t(blockIdx.y) * chunk_rows;
  const size_t r1 = r0 + chunk_rows < rows ? r0 + chunk_rows : rows;
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (c < cols)
    for (size_t r = r0 + ty; r < r1; r += 16) v += *reinterpret_cast<const f4 *>(a + r * cols + c);
  part[ty][tx] = v;
  __syncthreads();
  if (ty == 0 && c < cols) {
    f4 t = part[0][tx];
#pragma unroll
    for (int g = 1; g < 16; ++g) t += part[g][tx];
    *reinterpret_cast<f4 *>(partials + size_t(blockIdx.y) * cols + c) = t;
  }
}

// Pass 2: block per 64 columns; wave w adds chunks w, w + 4, ... (8 loads
// in flight, coalesced across the lanes' columns), and the 4 wave sums are
// added in wave order.
__global__ __launch_bounds__(256) void col_finish_kernel(const float *__restrict__ partials,
                                                         float *__restrict__ out, uint32_t chunks,
                                                         uint32_t cols, float beta) {
  __shared__ float wsum[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t c = blockIdx.x * 64 + uint32_t(lane);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < cols) {
    for (uint32_t k0 = uint32_t(w); k0 < chunks; k0 += 32) {
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j)
        if (k0 + 4 * j < chunks) acc[j] += partials[size_t(k0 + 4 * j) * cols + c];
    }
  }
  float t = acc[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) t += acc[j];
  wsum[w][lane] = t;
  __syncthreads();
  if (w == 0 && c < cols) {
    float r = ((wsum[0][lane] + wsum[1][lane]) + wsum[2][lane]) + wsum[3][lane];
    if (beta != 0.0f) r += beta * out[c];
    out[c] = r;
  }
}

// Row chunking of the two-pass column sum: about 512 blocks, chunks of at
// least 128 rows (a multiple of 16). chunks == 0: the single-pass kernel fits
// (few rows, or columns not float4-aligned).
struct ColSplit {
  uint32_t chunks = 0, chunk_rows = 0;
};
ColSplit col_split(size_t rows, uint32_t cols) {
  ColSplit cs;
  if (rows < 256 || cols % 4 != 0) return cs;
  // (rows >= 256 gives at least 2 chunks of 128 rows below)
  const size_t groups = (cols + 63) / 64;
  size_t chunks = std::max<size_t>(1, 512 / groups);
  chunks = std::min(chunks, rows / 128);
  if (chunks < 2) return cs;
  size_t chunk_rows = (rows + chunks - 1) / chunks;
  chunk_rows = (chunk_rows + 15) / 16 * 16;
  cs.chunks = uint32_t((rows + chunk_rows - 1) / chunk_rows);
  cs.chunk_rows = uint32_t(chunk_rows);
  return cs;
}

// ---- general: one thread per output element, serial over reduced dims -----
struct ReduceLayout {
  int ndim;                 // collapsed rank
  uint32_t shape[kMaxDims]; // input shape (collapsed)
  uint32_t reduced[kMaxDims];
  uint32_t in_stride[kMaxDims];
  uint32_t out_shape[kMaxDims]; // 1 on reduced dims
  size_t red_count;
};

template <bool MAX>
__global__ __launch_bounds__(256) void generic_reduce_kernel(const float *__restrict__ a,
                                                             float *__restrict__ out,
                                                             size_t n_out, ReduceLayout L) {
  for (size_t o = size_t(blockIdx.x) * blockDim.x + threadIdx.x; o < n_out;
       o += size_t(gridDim.x) * blockDim.x) {
    size_t rem = o, base = 0;
    for (int d = L.ndim - 1; d >= 0; --d) {
      const size_t c = rem % L.out_shape[d];
      rem /= L.out_shape[d];
      base += c * L.in_stride[d];
    }
    float acc = identity<MAX>();
    for (size_t i = 0; i < L.red_count; ++i) {
      size_t r = i, off = 0;
      for (int d = L.ndim - 1; d >= 0; --d) {
        if (!L.reduced[d]) continue;
        off += (r % L.shape[d]) * L.in_stride[d];
        r /= L.shape[d];
      }
      acc = combine<MAX>(acc, a[base + off]);
    }
    out[o] = acc;
  }
}

// A reduction's shape with size-1 dims dropped and runs of equally reduced
// (or kept) dims merged.
struct Collapsed {
  size_t n_in = 1, n_out = 1;
  uint32_t shp[kMaxDims], red[kMaxDims];
  int nd = 0;
};
int collapse(uint32_t ndim, const uint32_t *a_shape, const uint32_t *out_shape, Collapsed &c) {
  if (ndim == 0 || ndim > kMaxDims) return int(hipErrorInvalidValue);
  for (uint32_t d = 0; d < ndim; ++d) {
    if (out_shape[d] != a_shape[d] && out_shape[d] != 1) return int(hipErrorInvalidValue);
    c.n_in *= a_shape[d];
    c.n_out *= out_shape[d];
  }
  for (uint32_t d = 0; d < ndim; ++d) {
    if (a_shape[d] == 1) continue;
    const uint32_t r = out_shape[d] == 1 ? 1u : 0u;
    if (c.nd > 0 && c.red[c.nd - 1] == r) {
      c.shp[c.nd - 1] *= a_shape[d];
    } else {
      c.shp[c.nd] = a_shape[d];
      c.red[c.nd] = r;
      ++c.nd;
    }
  }
  return 0;
}

// Scratch floats the two-pass column sum needs for this reduction (0: none).
size_t sum_workspace_elems(const Collapsed &c) {
  if (c.n_out == 0 || c.n_in == 0 || c.n_in == c.n_out) return 0;
  if (c.nd != 2 || c.red[0] != 1) return 0;
  const ColSplit cs = col_split(c.shp[0], c.shp[1]);
  return size_t(cs.chunks) * c.shp[1];
}

template <bool MAX>
int reduce_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                    const uint32_t *out_shape, float *workspace, size_t workspace_elems,
                    void *stream) {
  Collapsed cl;
  if (const int st = collapse(ndim, a_shape, out_shape, cl)) return st;
  const size_t n_in = cl.n_in, n_out = cl.n_out;
  const uint32_t *shp = cl.shp, *red = cl.red;
  const int nd = cl.nd;
  hipStream_t s = as_stream(stream);
  if (n_out == 0) return 0;
  if (n_in == 0) return tlh_fill_f32(out, MAX ? -INFINITY : 0.0f, n_out, stream);
  if (n_in == n_out) return tlh_copy(a, out, n_in, stream);
  // nd >= 1 because n_in != n_out implies some dim > 1 is reduced.
  if (nd == 1) { // everything reduced
    if (MAX) {
      row_reduce_kernel<true><<<1, 64, 0, s>>>(a, out, 1, shp[0]);
    } else if (n_in <= (1u << 20)) {
      sum_all_kernel<<<1, 1024, 0, s>>>(a, n_in, out, 0);
    } else {
      row_reduce_kernel<false><<<1, 64, 0, s>>>(a, out, 1, shp[0]);
    }
    return launch_status();
  }
  if (nd == 2 && red[1] == 1) { // [K, R]: rows
    const size_t rows = shp[0];
    row_reduce_kernel<MAX><<<stride_grid(rows * 64, 256), 256, 0, s>>>(a, out, rows, shp[1]);
    return launch_status();
  }
  if (nd == 2 && red[0] == 1) { // [R, K]: columns
    const ColSplit cs = MAX ? ColSplit{} : col_split(shp[0], shp[1]);
    const bool aligned = (reinterpret_cast<uintptr_t>(a) & 15) == 0;
    if (cs.chunks && aligned && workspace && workspace_elems >= size_t(cs.chunks) * shp[1]) {
      col_partials_kernel<<<dim3(ceil_div(shp[1], 64), cs.chunks), 256, 0, s>>>(
          a, workspace, shp[0], shp[1], cs.chunk_rows);
      if (const int st = launch_status()) return st;
      col_finish_kernel<<<ceil_div(shp[1], 64), 256, 0, s>>>(workspace, out, cs.chunks, shp[1],
                                                              0.0f);
      return launch_status();
    }
    col_reduce_kernel<MAX><<<ceil_div(shp[1], 32), 256, 0, s>>>(a, out, shp[0], shp[1], 0.0f);
    return launch_status();
  }
  ReduceLayout L{};
  L.ndim = nd;
  size_t stride = 1;
  L.red_count = 1;
  for (int d = nd - 1; d >= 0; --d) {
    L.shape[d] = shp[d];
    L.reduced[d] = red[d];
    L.in_stride[d] = uint32_t(stride);
    L.out_shape[d] = red[d] ? 1 : shp[d];
    stride *= shp[d];
    if (red[d]) L.red_count *= shp[d];
  }
  generic_reduce_kernel<MAX><<<stride_grid(n_out, 256), 256, 0, s>>>(a, out, n_out, L);
  return launch_status();
}

// ---- argmax -----------------------------------------------------------------
// (value, index) pairs: larger value wins, ties go to the lower index; NaN
// never wins; an untouched pair carries index UINT32_MAX.
__device__ inline void argmax_combine(float &v, uint32_t &i, float v2, uint32_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__device__ inline void wave_argmax(float &v, uint32_t &i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float v2 = __shfl_xor(v, off, 64);
    const uint32_t i2 = __shfl_xor(i, off, 64);
    argmax_combine(v, i, v2, i2);
  }
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ a, size_t n,
                                                      uint32_t *__restrict__ out) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  float best = -INFINITY;
  uint32_t idx = 0xffffffffu;
  for (size_t j = threadIdx.x; j < n; j += blockDim.x) {
    const float x = a[j];
    if (x > best) { // first strictly larger value in this thread's stride
      best = x;
      idx = uint32_t(j);
    }
  }
  wave_argmax(best, idx);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    sv[w] = best;
    si[w] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    uint32_t i = si[0];
    for (int k = 1; k < int(blockDim.x >> 6); ++k) argmax_combine(v, i, sv[k], si[k]);
    *out = (i == 0xffffffffu) ? 0u : i;
  }
}

__global__ __launch_bounds__(256) void argmax_rows_kernel(const float *__restrict__ a,
                                                          size_t rows, uint32_t cols,
                                                          uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const size_t nwaves = (size_t(gridDim.x) * blockDim.x) >> 6;
  for (size_t r = wave; r < rows; r += nwaves) {
    const float *row = a + r * cols;
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    for (uint32_t j = lane; j < cols; j += 64) {
      const float x = row[j];
      if (x > best) {
        best = x;
        idx = j;
      }
    }
    wave_argmax(best, idx);
    if (lane == 0) out[r] = (idx == 0xffffffffu) ? 0u : idx;
  }
}

// ---- gradient squared norm -----------------------------------------------
// Metal's kernel: a 256-wide tree of squares per threadgroup plus one relaxed
// atomic add per group. Same structure here (wave shuffles instead of the
// LDS tree).
__global__ __launch_bounds__(256) void sqnorm_atomic_kernel(const float *__restrict__ g,
                                                            size_t n,
                                                            float *__restrict__ squared_norm) {
  __shared__ float scratch[4];
  float v = 0.0f;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const float x = g[i];
    v += x * x;
  }
  v = block_sum(v, scratch);
  if (threadIdx.x == 0) atomicAdd(squared_norm, v);
}

constexpr uint32_t kNormChunk = 4096;

// Multi-tensor: every block walks all tensors, taking chunk c of tensor t
// when c % gridDim.x == blockIdx.x; writes one partial per block.
__global__ __launch_bounds__(256) void sqnorm_multi_kernel(const float *__restrict__ const *grads,
                                                           const uint64_t *__restrict__ sizes,
                                                           uint32_t count,
                                                           float *__restrict__ partials) {
  __shared__ float scratch[4];
  __shared__ uint32_t first[kMaxMultiTensors + 1];
  // 16-byte aligned tensors: chunks of 1024 float4 (4096 floats), then the
  // last n % 4 elements as one more chunk; otherwise scalar chunks of 4096.
  auto split = [&](uint32_t t, uint64_t &n4, uint32_t &vchunks) {
    const uint64_t n = sizes[t];
    n4 = (reinterpret_cast<uintptr_t>(grads[t]) & 15) == 0 ? n / 4 : 0;
    vchunks = uint32_t((n4 + kNormChunk / 4 - 1) / (kNormChunk / 4));
    return n;
  };
  const uint32_t total = build_chunk_map(first, count, [&](uint32_t t) {
    uint64_t n4;
    uint32_t vchunks;
    const uint64_t n = split(t, n4, vchunks);
    return vchunks + uint32_t((n - 4 * n4 + kNormChunk - 1) / kNormChunk);
  });
  float v0 = 0.0f, v1 = 0.0f;
  for (uint32_t c = blockIdx.x; c < total; c += gridDim.x) {
    const uint32_t t = chunk_owner(first, count, c);
    const float *g = grads[t];
    uint64_t n4;
    uint32_t vchunks;
    const uint64_t n = split(t, n4, vchunks);
    const uint32_t k = c - first[t];
    if (k < vchunks) {
      const f4 *g4 = reinterpret_cast<const f4 *>(g);
      const uint64_t begin = uint64_t(k) * (kNormChunk / 4);
      const uint64_t end = begin + kNormChunk / 4 < n4 ? begin + kNormChunk / 4 : n4;
      uint64_t i = begin + threadIdx.x;
      for (; i + 256 < end; i += 512) { // two loads in flight per thread
        const f4 x = g4[i], y = g4[i + 256];
        v0 += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
        v1 += y.x * y.x + y.y * y.y + y.z * y.z + y.w * y.w;
      }
      if (i < end) {
        const f4 x = g4[i];
        v0 += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
      }
    } else {
      const uint64_t begin = 4 * n4 + uint64_t(k - vchunks) * kNormChunk;
      const uint64_t end = begin + kNormChunk < n ? begin + kNormChunk : n;
      for (uint64_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        const float x = g[i];
        v0 += x * x;
      }
    }
  }
  const float v = block_sum(v0 + v1, scratch);
  if (threadIdx.x == 0) partials[blockIdx.x] = v;
}

__global__ __launch_bounds__(1024) void sum_partials_final_kernel(const float *__restrict__ p,
                                                                 uint32_t n,
                                                                 float *__restrict__ out) {
  __shared__ float scratch[16];
  float v = 0.0f;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) v += p[i];
  v = block_sum(v, scratch);
  if (threadIdx.x == 0) *out = v;
}

} // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
TLH_API int tlh_sum(const float *a, size_t n, float *out, void *stream) {
  hipStream_t s = as_stream(stream);
  if (n == 0) return tlh_fill_f32(out, 0.0f, 1, stream);
  sum_all_kernel<<<1, 1024, 0, s>>>(a, n, out, 0);
  return launch_status();
}

TLH_API int tlh_sum_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                             const uint32_t *out_shape, void *stream) {
  return reduce_to_shape<false>(a, out, ndim, a_shape, out_shape, nullptr, 0, stream);
}

TLH_API int tlh_sum_to_shape_workspace(uint32_t ndim, const uint32_t *a_shape,
                                       const uint32_t *out_shape, size_t *elems) {
  if (!elems) return int(hipErrorInvalidValue);
  Collapsed cl;
  if (const int st = collapse(ndim, a_shape, out_shape, cl)) return st;
  *elems = sum_workspace_elems(cl);
  return 0;
}

TLH_API int tlh_sum_to_shape_ws(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                                const uint32_t *out_shape, float *workspace,
                                size_t workspace_elems, void *stream) {
  return reduce_to_shape<false>(a, out, ndim, a_shape, out_shape, workspace, workspace_elems,
                                stream);
}

TLH_API int tlh_max_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                             const uint32_t *out_shape, void *stream) {
  return reduce_to_shape<true>(a, out, ndim, a_shape, out_shape, nullptr, 0, stream);
}

TLH_API int tlh_argmax(const float *a, size_t n, uint32_t *out_index, void *stream) {
  if (n == 0 || n > 0xffffffffull) return int(hipErrorInvalidValue);
  argmax_kernel<<<1, 1024, 0, as_stream(stream)>>>(a, n, out_index);
  return launch_status();
}

TLH_API int tlh_argmax_rows(const float *a, size_t rows, uint32_t cols, uint32_t *out_index,
                            void *stream) {
  if (rows == 0) return 0;
  if (cols == 0) return int(hipErrorInvalidValue);
  argmax_rows_kernel<<<stride_grid(rows * 64, 256), 256, 0, as_stream(stream)>>>(a, rows, cols,
                                                                                 out_index);
  return launch_status();
}

TLH_API int tlh_accumulate_gradient_squared_norm(const float *g, size_t n, float *squared_norm,
                                                 void *stream) {
  if (n == 0) return 0;
  sqnorm_atomic_kernel<<<stride_grid(n, 256, 8), 256, 0, as_stream(stream)>>>(g, n,
                                                                              squared_norm);
  return launch_status();
}

TLH_API int tlh_gradient_squared_norm_multi(const float *const *grads, const uint64_t *sizes,
                                            uint32_t count, float *partials, float *squared_norm,
                                            void *stream) {
  hipStream_t s = as_stream(stream);
  if (count == 0) return tlh_fill_f32(squared_norm, 0.0f, 1, stream);
  if (count > kMaxMultiTensors) return int(hipErrorInvalidValue);
  sqnorm_multi_kernel<<<TLH_NORM_PARTIALS, 256, 0, s>>>(grads, sizes, count, partials);
  int st = launch_status();
  if (st) return st;
  sum_partials_final_kernel<<<1, 1024, 0, s>>>(partials, TLH_NORM_PARTIALS, squared_norm);
  return launch_status();
}

TLH_API int tlh_column_sum(const float *a, size_t rows, uint32_t cols, float *out, float beta,
                           void *stream) {
  if (cols == 0) return 0;
  col_reduce_kernel<false><<<ceil_div(cols, 32), 256, 0, as_stream(stream)>>>(a, out, rows, cols,
                                                                              beta);
  return launch_status();
}
