// Embedding gather and scatter-add.
//
// Reference: embedding_lookup (math.metal:778-793, one thread per element
// with a div/mod each) and scatter_add_rows (794-820, relaxed float atomics),
// launched from src/my_metal/runtime.cpp:920-1030.
// Here rows move as float4 vectors when the row length allows it, and the
// GPT's token+position embedding is one fused kernel.
// The reference kernels index with unchecked ids. These check every id
// against the table's row count: a gather of an id >= rows writes NaN (a
// defined, visible result instead of a read outside the table) and a
// scatter of such an id is dropped.
#include "common.h"

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

__global__ __launch_bounds__(256) void scatter_add_kernel(const float *__restrict__ values,
                                                          const uint32_t *__restrict__ ids,
                                                          size_t n_ids, uint32_t dim,
                                                          uint32_t dst_rows,
                                                          float *__restrict__ dst) {
  const size_t n = n_ids * dim;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x) {
    const size_t r = i / dim;
    const uint32_t c = uint32_t(i - r * dim);
    const uint32_t id = ids[r];
    if (id < dst_rows) atomicAdd(dst + size_t(id) * dim + c, values[i]);
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
  if (n_ids == 0 || dim == 0) return 0;
  scatter_add_kernel<<<stride_grid(n_ids * dim, 256), 256, 0, as_stream(stream)>>>(
      values, ids, n_ids, dim, dst_rows, dst);
  return launch_status();
}
