// Embedding gather and scatter-add.
//
// Reference: embedding_lookup (math.metal:778-793, one thread per element
// with a div/mod each) and scatter_add_rows (794-820, relaxed float atomics),
// launched from src/my_metal/runtime.cpp:920-1030.
// Here rows move as float4 vectors when the row length allows it, and the
// GPT's token+position embedding is one fused kernel. The scatter adds in
// increasing index order without atomics: every element receives its sum in
// the order of the sequential loop, so the result is deterministic and
// bit-identical to that loop.
// The reference kernels index with unchecked ids. These check every id
// against the table's row count: a gather of an id >= rows writes NaN (a
// defined, visible result instead of a read outside the table) and a
// scatter of such an id is dropped.
#include "common.h"

#include <algorithm>

#include "../../include/templit_hip.h"

using namespace tlh;

namespace {

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// out[i, c4] = w[ids[i], c4] over float4 columns.
__global__ __launch_bounds__(256) void gather4_kernel(const f4 *__restrict__ w,
                                                      uint32_t rows,
                                                      const uint32_t *__restrict__ ids,
                                                      size_t n_ids, uint32_t dim4,
                                                      f4 *__restrict__ out) {
  const size_t n = n_ids * dim4;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const size_t r = i / dim4;
    const uint32_t c = uint32_t(i - r * dim4);
    const uint32_t id = ids[r];
    out[i] = id < rows ? w[size_t(id) * dim4 + c] : f4{NAN, NAN, NAN, NAN};
  }
}

__global__ __launch_bounds__(256) void gather1_kernel(const float *__restrict__ w,
                                                      uint32_t rows,
                                                      const uint32_t *__restrict__ ids,
                                                      size_t n_ids, uint32_t dim,
                                                      float *__restrict__ out) {
  const size_t n = n_ids * dim;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const size_t r = i / dim;
    const uint32_t c = uint32_t(i - r * dim);
    const uint32_t id = ids[r];
    out[i] = id < rows ? w[size_t(id) * dim + c] : NAN;
  }
}

// out[b,t,:] = tok[ids[b,t],:] + pos[t,:]
__global__ __launch_bounds__(256) void embed_pos4_kernel(const f4 *__restrict__ tok,
                                                         const f4 *__restrict__ pos,
                                                         uint32_t vocab,
                                                         const uint32_t *__restrict__ ids,
                                                         uint32_t batch, uint32_t seq,
                                                         uint32_t dim4, f4 *__restrict__ out) {
  const size_t n = size_t(batch) * seq * dim4;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const size_t r = i / dim4;
    const uint32_t c = uint32_t(i - r * dim4);
    const uint32_t t = uint32_t(r % seq);
    const uint32_t id = ids[r];
    const f4 a = id < vocab ? tok[size_t(id) * dim4 + c] : f4{NAN, NAN, NAN, NAN};
    const f4 p = pos[size_t(t) * dim4 + c];
    out[i] = f4{a.x + p.x, a.y + p.y, a.z + p.z, a.w + p.w};
  }
}

__global__ __launch_bounds__(256) void embed_pos1_kernel(const float *__restrict__ tok,
                                                         const float *__restrict__ pos,
                                                         uint32_t vocab,
                                                         const uint32_t *__restrict__ ids,
                                                         uint32_t batch, uint32_t seq,
                                                         uint32_t dim, float *__restrict__ out) {
  const size_t n = size_t(batch) * seq * dim;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const size_t r = i / dim;
    const uint32_t c = uint32_t(i - r * dim);
    const uint32_t t = uint32_t(r % seq);
    const uint32_t id = ids[r];
    out[i] = (id < vocab ? tok[size_t(id) * dim + c] : NAN) + pos[size_t(t) * dim + c];
  }
}

constexpr uint32_t kIdsPerThread = 4;
constexpr uint32_t kIdsPerPass = 256 * kIdsPerThread;
constexpr uint32_t kScatterLdsFloats = 12288; // 48 KiB of destination rows per block

// dst[ids[i], c] += values[i, c] for i = 0, 1, ... in order.
// Block (x, y) owns destination rows [x*rows_per_block, +rows_per_block) and
// columns [y*cols, +cols), held in LDS. It walks the ids 1024 at a time
// (the next 1024 already loading), compacts the positions that fall in its
// rows with a stable block prefix count, and adds those value rows in
// position order. Each element is updated by one thread only, in increasing
// i. Ids >= dst_rows match no block and are dropped.
__global__ __launch_bounds__(256) void scatter_rows_ordered_kernel(
    const float *__restrict__ values, const uint32_t *__restrict__ ids, uint32_t n_ids,
    uint32_t dim, uint32_t dst_rows, uint32_t rows_per_block, uint32_t cols,
    float *__restrict__ dst) {
  extern __shared__ float acc[]; // rows_per_block x cols
  __shared__ uint32_t match_pos[kIdsPerPass];
  __shared__ uint32_t match_row[kIdsPerPass];
  __shared__ uint32_t wave_total[4];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t r0 = blockIdx.x * rows_per_block;
  const uint32_t nrows = min(rows_per_block, dst_rows - r0);
  const uint32_t c0 = blockIdx.y * cols;
  const uint32_t ncols = min(cols, dim - c0);
  for (uint32_t e = tid; e < nrows * ncols; e += 256) {
    const uint32_t q = e / ncols, c = e - q * ncols;
    acc[q * cols + c] = dst[size_t(r0 + q) * dim + c0 + c];
  }
  uint32_t cur[kIdsPerThread], nxt[kIdsPerThread];
  auto load = [&](uint32_t base, uint32_t (&v)[kIdsPerThread]) {
#pragma unroll
    for (uint32_t j = 0; j < kIdsPerThread; ++j) {
      const uint32_t i = base + tid * kIdsPerThread + j;
      v[j] = i < n_ids ? ids[i] : 0xffffffffu;
    }
  };
  load(0, cur);
  for (uint32_t base = 0; base < n_ids; base += kIdsPerPass) {
    if (base + kIdsPerPass < n_ids) load(base + kIdsPerPass, nxt);
    // ids below r0 wrap to large values in the unsigned difference
    uint32_t count = 0;
#pragma unroll
    for (uint32_t j = 0; j < kIdsPerThread; ++j) count += (cur[j] - r0 < nrows) ? 1u : 0u;
    uint32_t incl = count;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t t = __shfl_up(incl, o, 64);
      if (int(lane) >= o) incl += t;
    }
    if (lane == 63) wave_total[wave] = incl;
    __syncthreads();
    uint32_t slot = incl - count, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
      const uint32_t t = wave_total[w];
      if (w < wave) slot += t;
      total += t;
    }
#pragma unroll
    for (uint32_t j = 0; j < kIdsPerThread; ++j) {
      if (cur[j] - r0 < nrows) {
        match_pos[slot] = base + tid * kIdsPerThread + j;
        match_row[slot] = cur[j] - r0;
        ++slot;
      }
    }
    __syncthreads();
    uint32_t m = 0;
    for (; m + 4 <= total; m += 4) { // four value rows in flight
      const size_t p0 = size_t(match_pos[m]) * dim + c0, p1 = size_t(match_pos[m + 1]) * dim + c0,
                   p2 = size_t(match_pos[m + 2]) * dim + c0,
                   p3 = size_t(match_pos[m + 3]) * dim + c0;
      float *a0 = acc + match_row[m] * cols, *a1 = acc + match_row[m + 1] * cols,
            *a2 = acc + match_row[m + 2] * cols, *a3 = acc + match_row[m + 3] * cols;
      for (uint32_t c = tid; c < ncols; c += 256) {
        const float v0 = values[p0 + c], v1 = values[p1 + c], v2 = values[p2 + c],
                    v3 = values[p3 + c];
        a0[c] += v0; // same thread, program order: rows that repeat stay in order
        a1[c] += v1;
        a2[c] += v2;
        a3[c] += v3;
      }
    }
    for (; m < total; ++m) {
      const size_t p0 = size_t(match_pos[m]) * dim + c0;
      float *a0 = acc + match_row[m] * cols;
      for (uint32_t c = tid; c < ncols; c += 256) a0[c] += values[p0 + c];
    }
    __syncthreads(); // match_* and wave_total are rewritten by the next pass
#pragma unroll
    for (uint32_t j = 0; j < kIdsPerThread; ++j) cur[j] = nxt[j];
  }
  for (uint32_t e = tid; e < nrows * ncols; e += 256) {
    const uint32_t q = e / ncols, c = e - q * ncols;
    dst[size_t(r0 + q) * dim + c0 + c] = acc[q * cols + c];
  }
}

} // namespace

TLH_API int tlh_embedding_lookup(const float *weights, uint32_t rows, uint32_t dim,
                                 const uint32_t *ids, size_t n_ids, float *out, void *stream) {
  if (n_ids == 0 || dim == 0) return 0;
  hipStream_t s = as_stream(stream);
  if (dim % 4 == 0 && aligned16(weights) && aligned16(out)) {
    const uint32_t dim4 = dim / 4;
    gather4_kernel<<<stride_grid(n_ids * dim4, 256), 256, 0, s>>>(
        reinterpret_cast<const f4 *>(weights), rows, ids, n_ids, dim4, reinterpret_cast<f4 *>(out));
  } else {
    gather1_kernel<<<stride_grid(n_ids * dim, 256), 256, 0, s>>>(weights, rows, ids, n_ids, dim,
                                                                 out);
  }
  return launch_status();
}

TLH_API int tlh_embedding_add_positions(const float *tok, uint32_t vocab, const float *pos,
                                        const uint32_t *ids, uint32_t batch, uint32_t seq,
                                        uint32_t dim, float *out, void *stream) {
  const size_t n = size_t(batch) * seq * dim;
  if (n == 0) return 0;
  hipStream_t s = as_stream(stream);
  if (dim % 4 == 0 && aligned16(tok) && aligned16(pos) && aligned16(out)) {
    const uint32_t dim4 = dim / 4;
    embed_pos4_kernel<<<stride_grid(n / 4, 256), 256, 0, s>>>(
        reinterpret_cast<const f4 *>(tok), reinterpret_cast<const f4 *>(pos), vocab, ids, batch,
        seq, dim4, reinterpret_cast<f4 *>(out));
  } else {
    embed_pos1_kernel<<<stride_grid(n, 256), 256, 0, s>>>(tok, pos, vocab, ids, batch, seq, dim,
                                                          out);
  }
  return launch_status();
}

TLH_API int tlh_scatter_add_rows(const float *values, const uint32_t *ids, size_t n_ids,
                                 uint32_t dim, float *dst, uint32_t dst_rows, void *stream) {
  if (n_ids == 0 || dim == 0 || dst_rows == 0) return 0;
  if (n_ids > 0xffffffffu - kIdsPerPass) return int(hipErrorInvalidValue);
  // Column chunks only when one row does not fit the LDS budget; rows per
  // block sized for ~512 blocks (each block reads every id once).
  const uint32_t cols = std::min<uint32_t>(dim, kScatterLdsFloats);
  const uint32_t fit = kScatterLdsFloats / cols;
  const uint32_t want = (dst_rows + 511) / 512;
  const uint32_t rows_per_block = std::max<uint32_t>(1, std::min(fit, want));
  const dim3 grid((dst_rows + rows_per_block - 1) / rows_per_block, (dim + cols - 1) / cols);
  const size_t lds = size_t(rows_per_block) * cols * sizeof(float);
  scatter_rows_ordered_kernel<<<grid, 256, lds, as_stream(stream)>>>(
      values, ids, uint32_t(n_ids), dim, dst_rows, rows_per_block, cols, dst);
  return launch_status();
}
