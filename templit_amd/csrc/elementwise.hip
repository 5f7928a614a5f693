// Elementwise kernels: broadcast binary ops, scalar ops, unary ops, GELU and
// its fused backward, transpose.
//
// Reference kernels replaced (include/my_metal/math.metal):
//   add/sub/hadamard/divide 401-510, add_scalar/divide_scalar/pow_scalar
//   427-434/511-518/527-534, sqrt/exp/sigmoid 519-548, GELU/GELU_derivative
//   821-855, transpose 566-584, copy 1045-1050.
// The Metal kernels decode every output index through `ndim` div/mod pairs
// and move one element per thread. Here the host first collapses adjacent
// dimensions that are contiguous in every operand and drops size-1 dims, and
// the common shapes (same-shape, scalar, row-bias, column-broadcast) run
// dedicated vectorised kernels; only the leftovers pay for the decode.
#include "common.h"

#include "../../include/templit_hip.h"

using namespace tlh;

namespace {

constexpr int kMaxDims = 8;

enum BinOp { kAdd = 0, kSub = 1, kMul = 2, kDiv = 3 };

template <int OP> __device__ inline float apply(float x, float y) {
  if constexpr (OP == kAdd) return x + y;
  else if constexpr (OP == kSub) return x - y;
  else if constexpr (OP == kMul) return x * y;
  else return x / y;
}

struct Layout {
  int ndim;
  uint32_t shape[kMaxDims];
  uint32_t sa[kMaxDims];
  uint32_t sb[kMaxDims];
};

// Same shape, both contiguous: 4 elements per thread.
template <int OP>
__global__ __launch_bounds__(256) void binary_same_kernel(const float *__restrict__ a,
                                                          const float *__restrict__ b,
                                                          float *__restrict__ out, size_t n4,
                                                          size_t n) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f4 x = reinterpret_cast<const f4 *>(a)[i];
    const f4 y = reinterpret_cast<const f4 *>(b)[i];
    f4 r;
    r.x = apply<OP>(x.x, y.x); r.y = apply<OP>(x.y, y.y);
    r.z = apply<OP>(x.z, y.z); r.w = apply<OP>(x.w, y.w);
    reinterpret_cast<f4 *>(out)[i] = r;
  }
  for (size_t i = n4 * 4 + size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = apply<OP>(a[i], b[i]);
}

// out[r, c] = a[r*sar + c*sac] op b[r*sbr + c*sbc] for a 2-D collapsed view;
// covers row-bias ([R,C] op [1,C]), column broadcast ([R,C] op [R,1]),
// scalar operands and the general two-dim case. Columns are the fast axis.
template <int OP>
__global__ __launch_bounds__(256) void binary_2d_kernel(const float *__restrict__ a,
                                                        const float *__restrict__ b,
                                                        float *__restrict__ out, uint32_t rows,
                                                        uint32_t cols, uint32_t sar,
                                                        uint32_t sac, uint32_t sbr,
                                                        uint32_t sbc) {
  const size_t n = size_t(rows) * cols;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t r = uint32_t(i / cols);
    const uint32_t c = uint32_t(i - size_t(r) * cols);
    out[i] = apply<OP>(a[size_t(r) * sar + size_t(c) * sac], b[size_t(r) * sbr + size_t(c) * sbc]);
  }
}

template <int OP>
__global__ __launch_bounds__(256) void binary_nd_kernel(const float *__restrict__ a,
                                                        const float *__restrict__ b,
                                                        float *__restrict__ out, size_t n,
                                                        Layout L) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    size_t rem = i, oa = 0, ob = 0;
    for (int d = L.ndim - 1; d >= 0; --d) {
      const size_t c = rem % L.shape[d];
      rem /= L.shape[d];
      oa += c * L.sa[d];
      ob += c * L.sb[d];
    }
    out[i] = apply<OP>(a[oa], b[ob]);
  }
}

// Drops size-1 dims and merges neighbours that are contiguous in both inputs.
void collapse(Layout &L) {
  int w = 0;
  for (int d = 0; d < L.ndim; ++d) {
    if (L.shape[d] == 1) continue;
    L.shape[w] = L.shape[d];
    L.sa[w] = L.sa[d];
    L.sb[w] = L.sb[d];
    ++w;
  }
  L.ndim = w;
  if (L.ndim == 0) {
    L.ndim = 1;
    L.shape[0] = 1;
    L.sa[0] = 0;
    L.sb[0] = 0;
    return;
  }
  int o = 0;
  for (int d = 1; d < L.ndim; ++d) {
    const bool ma = uint64_t(L.sa[o]) == uint64_t(L.sa[d]) * L.shape[d];
    const bool mb = uint64_t(L.sb[o]) == uint64_t(L.sb[d]) * L.shape[d];
    if (ma && mb) {
      L.shape[o] *= L.shape[d];
      L.sa[o] = L.sa[d];
      L.sb[o] = L.sb[d];
    } else {
      ++o;
      L.shape[o] = L.shape[d];
      L.sa[o] = L.sa[d];
      L.sb[o] = L.sb[d];
    }
  }
  L.ndim = o + 1;
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int OP>
int binary_launch(const float *a, const float *b, float *out, uint32_t ndim,
                  const uint32_t *out_shape, const uint32_t *stride_a,
                  const uint32_t *stride_b, void *stream) {
  if (ndim > kMaxDims) return int(hipErrorInvalidValue);
  Layout L{};
  L.ndim = int(ndim);
  size_t n = 1;
  for (uint32_t d = 0; d < ndim; ++d) {
    L.shape[d] = out_shape[d];
    L.sa[d] = stride_a[d];
    L.sb[d] = stride_b[d];
    n *= out_shape[d];
  }
  if (n == 0) return 0;
  collapse(L);
  hipStream_t s = as_stream(stream);
  if (L.ndim == 1 && L.sa[0] == 1 && L.sb[0] == 1 && aligned16(a) && aligned16(b) &&
      aligned16(out)) {
    binary_same_kernel<OP><<<stride_grid(n / 4 + 1, 256), 256, 0, s>>>(a, b, out, n / 4, n);
  } else if (L.ndim <= 2) {
    const uint32_t rows = L.ndim == 2 ? L.shape[0] : 1;
    const uint32_t cols = L.ndim == 2 ? L.shape[1] : L.shape[0];
    const uint32_t sar = L.ndim == 2 ? L.sa[0] : 0, sbr = L.ndim == 2 ? L.sb[0] : 0;
    const uint32_t sac = L.ndim == 2 ? L.sa[1] : L.sa[0];
    const uint32_t sbc = L.ndim == 2 ? L.sb[1] : L.sb[0];
    binary_2d_kernel<OP><<<stride_grid(n, 256), 256, 0, s>>>(a, b, out, rows, cols, sar, sac,
                                                            sbr, sbc);
  } else {
    binary_nd_kernel<OP><<<stride_grid(n, 256), 256, 0, s>>>(a, b, out, n, L);
  }
  return launch_status();
}

// ---- contiguous unary / scalar ops ----------------------------------------
enum UnOp { kSqrt, kExp, kSigmoid, kGelu, kGeluGrad, kCopy, kAddS, kDivS, kPowS };

template <int OP> __device__ inline float unary(float x, float s) {
  if constexpr (OP == kSqrt) return sqrtf(x);
  else if constexpr (OP == kExp) return expf(x);
  else if constexpr (OP == kSigmoid) return 1.0f / (1.0f + expf(-x));
  else if constexpr (OP == kGelu) return gelu_fwd(x);
  else if constexpr (OP == kGeluGrad) return gelu_grad(x);
  else if constexpr (OP == kCopy) return x;
  else if constexpr (OP == kAddS) return x + s;
  else if constexpr (OP == kDivS) return x / s;
  else return powf(x, s);
}

template <int OP>
__global__ __launch_bounds__(256) void unary_kernel(const float *__restrict__ a,
                                                    float *__restrict__ out, size_t n4, size_t n,
                                                    float s) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f4 x = reinterpret_cast<const f4 *>(a)[i];
    f4 r;
    r.x = unary<OP>(x.x, s); r.y = unary<OP>(x.y, s);
    r.z = unary<OP>(x.z, s); r.w = unary<OP>(x.w, s);
    reinterpret_cast<f4 *>(out)[i] = r;
  }
  for (size_t i = n4 * 4 + size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = unary<OP>(a[i], s);
}

template <int OP> int unary_launch(const float *a, float *out, size_t n, float s, void *stream) {
  if (n == 0) return 0;
  const size_t n4 = (aligned16(a) && aligned16(out)) ? n / 4 : 0;
  unary_kernel<OP><<<stride_grid(n4 ? n4 : n, 256), 256, 0, as_stream(stream)>>>(a, out, n4,
                                                                                   n, s);
  return launch_status();
}

__global__ __launch_bounds__(256) void gelu_backward_kernel(const float *__restrict__ g,
                                                            const float *__restrict__ x,
                                                            float *__restrict__ out, size_t n4,
                                                            size_t n) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const f4 gv = reinterpret_cast<const f4 *>(g)[i];
    const f4 xv = reinterpret_cast<const f4 *>(x)[i];
    f4 r;
    r.x = gv.x * gelu_grad(xv.x); r.y = gv.y * gelu_grad(xv.y);
    r.z = gv.z * gelu_grad(xv.z); r.w = gv.w * gelu_grad(xv.w);
    reinterpret_cast<f4 *>(out)[i] = r;
  }
  for (size_t i = n4 * 4 + size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = g[i] * gelu_grad(x[i]);
}

// ---- transpose -------------------------------------------------------------
struct Gather {
  int ndim;
  uint32_t shape[kMaxDims];
  uint32_t in_strides[kMaxDims];
};

__global__ __launch_bounds__(256) void gather_kernel(const float *__restrict__ a,
                                                     float *__restrict__ out, size_t n,
                                                     Gather G) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    size_t rem = i, off = 0;
    for (int d = G.ndim - 1; d >= 0; --d) {
      const size_t c = rem % G.shape[d];
      rem /= G.shape[d];
      off += c * G.in_strides[d];
    }
    out[i] = a[off];
  }
}

// Permutations that keep the last dimension contiguous (head split/merge,
// [B,T,H,D] <-> [B,H,T,D]): one float4 per thread, 32-bit index math. G is
// in float4 units (last extent and every stride divided by 4).
__global__ __launch_bounds__(256) void gather4_kernel(const f4 *__restrict__ a,
                                                      f4 *__restrict__ out, uint32_t n4,
                                                      Gather G) {
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    uint32_t rem = i;
    size_t off = 0;
    for (int d = G.ndim - 1; d >= 0; --d) {
      const uint32_t c = rem % uint32_t(G.shape[d]);
      rem /= uint32_t(G.shape[d]);
      off += size_t(c) * G.in_strides[d];
    }
    out[i] = a[off];
  }
}

// Batched 2-D transpose through a padded 64x64 LDS tile:
// out[z, i, j] = a[z*batch_stride + j*ld_in + i] with out [z, rows, cols]
// row-major (rows = input columns).
// One 64x64 tile of out[rows][cols] = in^T, in = src[cols][rows] with row
// pitch ld_in; i0 / j0 = the tile's first output row / column.
__device__ inline void transpose_tile(const float *__restrict__ src, float *__restrict__ dst,
                                      uint32_t rows, uint32_t cols, uint32_t ld_in,
                                      uint32_t i0, uint32_t j0, float (&tile)[64][65]) {
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  // all 16 loads of a thread in flight before the LDS writes
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t in_row = j0 + ty + 4 * i, in_col = i0 + tx;
    v[i] = (in_row < cols && in_col < rows) ? src[size_t(in_row) * ld_in + in_col] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) tile[ty + 4 * i][tx] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t o_row = i0 + ty + 4 * i, o_col = j0 + tx;
    if (o_row < rows && o_col < cols) dst[size_t(o_row) * cols + o_col] = tile[tx][ty + 4 * i];
  }
}

__global__ __launch_bounds__(256) void transpose_tiled_kernel(const float *__restrict__ a,
                                                              float *__restrict__ out,
                                                              uint32_t rows, uint32_t cols,
                                                              size_t in_batch_stride,
                                                              uint32_t ld_in) {
  __shared__ float tile[64][65];
  const uint32_t z = blockIdx.z;
  transpose_tile(a + size_t(z) * in_batch_stride, out + size_t(z) * rows * cols, rows, cols,
                 ld_in, blockIdx.y * 64, blockIdx.x * 64, tile);
}

// The same tiles for any permutation whose input is contiguous along the
// output's second-to-last dim: out[z, i, j] = a[off(z) + j*ld_in + i], the
// batch entry z's input offset from its coordinates in the leading output
// dims (composed views: the K^T of a head-split projection, [B,H,64,T] read
// from [B,T,H,64]).
struct BatchDims {
  int n;
  uint32_t shape[kMaxDims];
  uint32_t stride[kMaxDims];
};
__global__ __launch_bounds__(256) void transpose_batched_kernel(const float *__restrict__ a,
                                                                float *__restrict__ out,
                                                                uint32_t rows, uint32_t cols,
                                                                uint32_t ld_in, BatchDims B) {
  __shared__ float tile[64][65];
  uint32_t rem = blockIdx.z;
  size_t off = 0;
  for (int d = B.n - 1; d >= 0; --d) {
    const uint32_t c = rem % B.shape[d];
    rem /= B.shape[d];
    off += size_t(c) * B.stride[d];
  }
  transpose_tile(a + off, out + size_t(blockIdx.z) * rows * cols, rows, cols, ld_in,
                 blockIdx.y * 64, blockIdx.x * 64, tile);
}

// Block b handles output tile b - first_tile of the job whose tile range
// holds b; the threads test one job each to find it. A block that no job
// claims does nothing, and transpose_tile keeps every access inside the
// job's own rows x cols (so blocks past the last job's tiles write
// nothing). A table whose first_tile values descend anywhere would let two
// jobs claim one block: every block then exits and nothing is written.
__global__ __launch_bounds__(256) void transpose_multi_kernel(const float *__restrict__ src,
                                                              float *__restrict__ dst,
                                                              const tlh_transpose_job *jobs,
                                                              uint32_t count,
                                                              uint32_t total_tiles) {
  __shared__ float tile[64][65];
  __shared__ int which, descending;
  const uint32_t b = blockIdx.x;
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    which = -1;
    descending = 0;
  }
  __syncthreads();
  if (t < count) {
    const uint32_t end = t + 1 < count ? jobs[t + 1].first_tile : total_tiles;
    if (end < jobs[t].first_tile) descending = 1;
    else if (jobs[t].first_tile <= b && b < end) which = int(t);
  }
  __syncthreads();
  if (which < 0 || descending) return;
  const tlh_transpose_job j = jobs[which];
  // output [j.cols][j.rows] = source [j.rows][j.cols] transposed
  const uint32_t tiles_x = (j.rows + 63) / 64;
  const uint32_t local = b - j.first_tile;
  transpose_tile(src + j.src_offset, dst + j.dst_offset, j.cols, j.rows, j.cols,
                 (local / tiles_x) * 64, (local % tiles_x) * 64, tile);
}

} // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
TLH_API int tlh_add(const float *a, const float *b, float *out, uint32_t ndim,
                    const uint32_t *out_shape, const uint32_t *stride_a,
                    const uint32_t *stride_b, void *stream) {
  return binary_launch<kAdd>(a, b, out, ndim, out_shape, stride_a, stride_b, stream);
}
TLH_API int tlh_sub(const float *a, const float *b, float *out, uint32_t ndim,
                    const uint32_t *out_shape, const uint32_t *stride_a,
                    const uint32_t *stride_b, void *stream) {
  return binary_launch<kSub>(a, b, out, ndim, out_shape, stride_a, stride_b, stream);
}
TLH_API int tlh_hadamard(const float *a, const float *b, float *out, uint32_t ndim,
                         const uint32_t *out_shape, const uint32_t *stride_a,
                         const uint32_t *stride_b, void *stream) {
  return binary_launch<kMul>(a, b, out, ndim, out_shape, stride_a, stride_b, stream);
}
TLH_API int tlh_divide(const float *a, const float *b, float *out, uint32_t ndim,
                       const uint32_t *out_shape, const uint32_t *stride_a,
                       const uint32_t *stride_b, void *stream) {
  return binary_launch<kDiv>(a, b, out, ndim, out_shape, stride_a, stride_b, stream);
}

TLH_API int tlh_add_scalar(const float *a, float scalar, float *out, size_t n, void *stream) {
  return unary_launch<kAddS>(a, out, n, scalar, stream);
}
TLH_API int tlh_divide_scalar(const float *a, float scalar, float *out, size_t n,
                              void *stream) {
  return unary_launch<kDivS>(a, out, n, scalar, stream);
}
TLH_API int tlh_pow_scalar(const float *a, float exponent, float *out, size_t n,
                           void *stream) {
  return unary_launch<kPowS>(a, out, n, exponent, stream);
}
TLH_API int tlh_sqrt(const float *a, float *out, size_t n, void *stream) {
  return unary_launch<kSqrt>(a, out, n, 0.f, stream);
}
TLH_API int tlh_exp(const float *a, float *out, size_t n, void *stream) {
  return unary_launch<kExp>(a, out, n, 0.f, stream);
}
TLH_API int tlh_sigmoid(const float *a, float *out, size_t n, void *stream) {
  return unary_launch<kSigmoid>(a, out, n, 0.f, stream);
}
TLH_API int tlh_gelu(const float *a, float *out, size_t n, void *stream) {
  return unary_launch<kGelu>(a, out, n, 0.f, stream);
}
TLH_API int tlh_gelu_derivative(const float *a, float *out, size_t n, void *stream) {
  return unary_launch<kGeluGrad>(a, out, n, 0.f, stream);
}
TLH_API int tlh_copy(const float *a, float *out, size_t n, void *stream) {
  if (a == out) return 0;
  return unary_launch<kCopy>(a, out, n, 0.f, stream);
}

TLH_API int tlh_gelu_backward(const float *grad, const float *x, float *out, size_t n,
                              void *stream) {
  if (n == 0) return 0;
  const size_t n4 = (aligned16(grad) && aligned16(x) && aligned16(out)) ? n / 4 : 0;
  gelu_backward_kernel<<<stride_grid(n4 ? n4 : n, 256), 256, 0, as_stream(stream)>>>(
      grad, x, out, n4, n);
  return launch_status();
}

TLH_API int tlh_transpose_multi(const float *src, float *dst, const tlh_transpose_job *jobs,
                                uint32_t count, uint32_t total_tiles, void *stream) {
  if (count == 0 || total_tiles == 0) return 0;
  if (count > 256 || !src || !dst || !jobs) return int(hipErrorInvalidValue);
  transpose_multi_kernel<<<total_tiles, 256, 0, as_stream(stream)>>>(src, dst, jobs, count,
                                                                     total_tiles);
  return launch_status();
}

TLH_API int tlh_transpose(const float *a, float *out, uint32_t ndim_in,
                          const uint32_t *out_shape_in, const uint32_t *in_strides_in,
                          void *stream) {
  if (ndim_in > kMaxDims || ndim_in == 0) return int(hipErrorInvalidValue);
  if (a == out) return int(hipErrorInvalidValue);
  size_t n = 1;
  for (uint32_t d = 0; d < ndim_in; ++d) n *= out_shape_in[d];
  if (n == 0) return 0;
  hipStream_t s = as_stream(stream);
  // Size-1 dims dropped and adjacent output dims merged where the input
  // walks them as one run (stride[d] = shape[d+1] * stride[d+1]): the same
  // permutation with fewer dims, e.g. [B,T,H,D] <- [B,H,D,T] as [B,T,H*D].
  uint32_t out_shape[kMaxDims], in_strides[kMaxDims], ndim = 0;
  for (uint32_t d = 0; d < ndim_in; ++d) {
    if (out_shape_in[d] == 1) continue;
    if (ndim > 0 && in_strides[ndim - 1] == out_shape_in[d] * in_strides_in[d]) {
      out_shape[ndim - 1] *= out_shape_in[d];
      in_strides[ndim - 1] = in_strides_in[d];
      continue;
    }
    out_shape[ndim] = out_shape_in[d];
    in_strides[ndim] = in_strides_in[d];
    ++ndim;
  }
  if (ndim == 0) { // a single element
    out_shape[0] = 1;
    in_strides[0] = 1;
    ndim = 1;
  }
  // Batched swap of the last two dims of a contiguous input: tiled path.
  if (ndim >= 2) {
    const uint32_t R = out_shape[ndim - 2], C = out_shape[ndim - 1];
    bool last_two = in_strides[ndim - 2] == 1 && in_strides[ndim - 1] == R;
    size_t expect = size_t(R) * C;
    for (int d = int(ndim) - 3; d >= 0 && last_two; --d) {
      if (out_shape[d] != 1 && in_strides[d] != expect) last_two = false;
      expect *= out_shape[d];
    }
    const size_t batch = n / (size_t(R) * C);
    if (last_two && batch <= 65535 && R > 1 && C > 1) {
      dim3 grid(ceil_div(C, 64), ceil_div(R, 64), unsigned(batch));
      transpose_tiled_kernel<<<grid, 256, 0, s>>>(a, out, R, C, size_t(R) * C, R);
      return launch_status();
    }
    // any other layout whose input runs along the output's rows
    if (in_strides[ndim - 2] == 1 && in_strides[ndim - 1] > 1 && batch <= 65535 && R > 1 &&
        C > 1) {
      BatchDims B{};
      B.n = int(ndim) - 2;
      for (uint32_t d = 0; d + 2 < ndim; ++d) {
        B.shape[d] = out_shape[d];
        B.stride[d] = in_strides[d];
      }
      dim3 grid(ceil_div(C, 64), ceil_div(R, 64), unsigned(batch));
      transpose_batched_kernel<<<grid, 256, 0, s>>>(a, out, R, C, in_strides[ndim - 1], B);
      return launch_status();
    }
  }
  Gather G{};
  G.ndim = int(ndim);
  for (uint32_t d = 0; d < ndim; ++d) {
    G.shape[d] = out_shape[d];
    G.in_strides[d] = in_strides[d];
  }
  bool vec = in_strides[ndim - 1] == 1 && out_shape[ndim - 1] % 4 == 0 && aligned16(a) &&
             aligned16(out) && n / 4 <= 0xffffffffull;
  for (uint32_t d = 0; d + 1 < ndim && vec; ++d) vec = in_strides[d] % 4 == 0;
  if (vec) {
    G.shape[ndim - 1] /= 4;
    for (uint32_t d = 0; d + 1 < ndim; ++d) G.in_strides[d] /= 4;
    const uint32_t n4 = uint32_t(n / 4);
    gather4_kernel<<<stride_grid(n4, 256), 256, 0, s>>>(reinterpret_cast<const f4 *>(a),
                                                       reinterpret_cast<f4 *>(out), n4, G);
    return launch_status();
  }
  gather_kernel<<<stride_grid(n, 256), 256, 0, s>>>(a, out, n, G);
  return launch_status();
}
