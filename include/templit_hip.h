/*
 * templit_hip.h -- C-ABI of libtemplit_hip.so, the gfx950 (MI355X) kernel
 * library behind hip::Runtime.
 *
 * This is the drop-in boundary for the TempLit runtime backend. The Metal
 * backend reaches its GPU through metal-cpp and 31 kernels that
 * src/my_metal/runtime.cpp loads by name (runtime.cpp:251-282) from
 * include/my_metal/math.metal. Here every kernel name becomes one extern "C"
 * entry point taking plain device pointers, sizes and a stream:
 *
 *   - every function returns an int: a hipError_t code, 0 on success;
 *   - data pointers are device pointers unless named host_*; they are
 *     borrowed only for the work enqueued by the call. Shape and stride
 *     arrays (`*_shape`, `*_strides`, `stride_*`, `batch_*`) are host arrays
 *     read before the call returns. Pointer/size tables of the multi-tensor
 *     entry points are device arrays (so a captured graph can replay them);
 *   - `stream` is a hipStream_t (NULL = the legacy default stream);
 *   - work is enqueued asynchronously in call order on `stream` (the Metal
 *     runtime's single serial compute encoder, runtime.cpp:290-317);
 *   - shapes are uint32 (the reference's rtensor::index_type,
 *     include/RTensor/RTensor.h:18-21); element counts are size_t;
 *   - no C++ types or exceptions cross this boundary. Shape validation that
 *     the reference performs in C++ (std::invalid_argument etc.) is done by
 *     the host runtime above this layer; these functions only reject
 *     arguments they cannot execute (hipErrorInvalidValue).
 *
 * Each declaration cites the reference interface it replaces (path:line in
 * the TempLit tree).
 */
#ifndef TEMPLIT_HIP_H
#define TEMPLIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Device, memory, streams, events, graphs
 * ------------------------------------------------------------------------- */

/* metal::init (src/my_metal/metal.cpp:18-27): select the device once;
 * idempotent for the same device. */
int tlh_init(int device);
int tlh_device_count(int *count);
/* Compute units of the current device (256 on MI355X). */
int tlh_device_cu_count(int *count);
const char *tlh_error_string(int code);
int tlh_device_synchronize(void);

/* Command queue / command buffer (runtime.cpp:238, 290-317). */
int tlh_stream_create(void **stream);
int tlh_stream_destroy(void *stream);
/* cmdBuff_->waitUntilCompleted (runtime.cpp:310-317). */
int tlh_stream_synchronize(void *stream);

/* device->newBuffer (include/my_metal/storage.h:13-16) and its release. */
int tlh_malloc(void **ptr, size_t bytes);
int tlh_free(void *ptr);
/* Pinned host staging memory for stream-ordered host<->device copies. */
int tlh_host_alloc(void **host_ptr, size_t bytes);
int tlh_host_free(void *host_ptr);

/* Storage::write / read (include/my_metal/storage.h:26-40); asynchronous on
 * `stream`: synchronise before reusing or reading the host buffer. */
int tlh_memcpy_h2d(void *dst, const void *host_src, size_t bytes, void *stream);
int tlh_memcpy_d2h(void *host_dst, const void *src, size_t bytes, void *stream);
/* Storage::clone (storage.h:45-50) and the blit copy of scatter_add_rows
 * (runtime.cpp:989-1009). */
int tlh_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
/* Storage::fill (storage.h:41-43) and the blit zero-fill of scatter_index
 * (runtime.cpp:1018-1027). Kernel fills, safe inside captured graphs. */
int tlh_fill_f32(float *dst, float value, size_t n, void *stream);
int tlh_fill_u32(uint32_t *dst, uint32_t value, size_t n, void *stream);
/* counters[i] += delta on the stream: AdamW's per-parameter ++step_
 * (include/optimiser/AdamW.h:78) as a kernel, so a captured training step
 * advances the step count on every replay. */
int tlh_increment_u32(uint32_t *counters, size_t n, uint32_t delta, void *stream);
/* Synthetic data on the device: element i of dst is the i-th value of a
 * SplitMix64 stream seeded with `seed` (normal: Box-Muller over pairs;
 * uniform: next() % bound). Used for random-init weights and benchmark
 * batches; the reference draws these on the host (include/nn/layer.h:15-30). */
int tlh_fill_normal(float *dst, size_t n, uint64_t seed, float mean, float std,
                    void *stream);
int tlh_fill_uniform_u32(uint32_t *dst, size_t n, uint64_t seed, uint32_t bound,
                         void *stream);
/* Storage::compare (storage.h:52-59): byte equality. `scratch` is one device
 * int. Synchronous. */
int tlh_compare(const void *a, const void *b, size_t bytes, int *host_equal,
                int *scratch, void *stream);

int tlh_event_create(void **event);
int tlh_event_record(void *event, void *stream);
int tlh_event_synchronize(void *event);
int tlh_event_elapsed_ms(void *start, void *end, float *host_ms);
int tlh_event_destroy(void *event);
/* `stream` waits, on the device, for the work recorded in `event`: a fork or
 * join between two streams (captured as a graph dependency while recording).
 * No reference counterpart: the Metal runtime has one serial encoder. */
int tlh_stream_wait_event(void *stream, void *event);

/* Command-buffer record/commit as a hipGraph (runtime.cpp:290-309).
 * begin/end_capture: thread-local capture, instantiated on end. */
int tlh_graph_begin_capture(void *stream);
int tlh_graph_end_capture(void *stream, void **exec);
int tlh_graph_launch(void *exec, void *stream);
int tlh_graph_destroy(void *exec);
/* Relaxed-mode capture that returns the un-instantiated graph, for callers
 * (hip::Runtime's graph mode) that cache executable graphs and refresh them
 * with tlh_graph_exec_update: *updated = 1 when `exec` took `graph`'s
 * parameters (same topology), 0 when it must be re-instantiated. */
int tlh_graph_begin_capture_relaxed(void *stream);
int tlh_graph_end_capture_graph(void *stream, void **graph);
int tlh_graph_instantiate(void *graph, void **exec);
int tlh_graph_exec_update(void *exec, void *graph, int *updated);
int tlh_graph_free(void *graph);
int tlh_stream_is_capturing(void *stream, int *capturing);

/* Profiling ranges (roctx; seen by rocprofv3 --marker-trace): stand in for
 * Runtime::start_profile / end_profile (runtime.cpp:42-63). */
int tlh_range_push(const char *name);
int tlh_range_pop(void);

/* ---------------------------------------------------------------------------
 * Elementwise (math.metal:401-548, 821-855, 1045-1050)
 * ------------------------------------------------------------------------- */

/* Broadcast binary ops, kernels add/sub/hadamard/divide
 * (math.metal:401-510) launched by call_binary_op (runtime.cpp:65-95).
 * `out` is contiguous with `ndim` dims `out_shape`; stride_a / stride_b are
 * the element strides of a and b aligned to out, 0 on broadcast dims -- what
 * broadcast_strides (runtime.cpp:18-39) computes. ndim <= 8. `out` may alias
 * a or b when it has their shape (in-place, execute.h:249). */
int tlh_add(const float *a, const float *b, float *out, uint32_t ndim,
            const uint32_t *out_shape, const uint32_t *stride_a,
            const uint32_t *stride_b, void *stream);
int tlh_sub(const float *a, const float *b, float *out, uint32_t ndim,
            const uint32_t *out_shape, const uint32_t *stride_a,
            const uint32_t *stride_b, void *stream);
int tlh_hadamard(const float *a, const float *b, float *out, uint32_t ndim,
                 const uint32_t *out_shape, const uint32_t *stride_a,
                 const uint32_t *stride_b, void *stream);
int tlh_divide(const float *a, const float *b, float *out, uint32_t ndim,
               const uint32_t *out_shape, const uint32_t *stride_a,
               const uint32_t *stride_b, void *stream);

/* Scalar ops add_scalar / divide_scalar / pow_scalar (math.metal:427-434,
 * 511-518, 527-534; call_scalar_op runtime.cpp:116-136). */
int tlh_add_scalar(const float *a, float scalar, float *out, size_t n, void *stream);
int tlh_divide_scalar(const float *a, float scalar, float *out, size_t n, void *stream);
int tlh_pow_scalar(const float *a, float exponent, float *out, size_t n, void *stream);

/* Unary ops sqrt / exp / sigmoid (math.metal:519-548; call_unary_op
 * runtime.cpp:97-114), GELU / GELU_derivative (math.metal:821-855,
 * runtime.cpp:1073-1081), copy (math.metal:1045-1050, runtime.cpp:1170-1186). */
int tlh_sqrt(const float *a, float *out, size_t n, void *stream);
int tlh_exp(const float *a, float *out, size_t n, void *stream);
int tlh_sigmoid(const float *a, float *out, size_t n, void *stream);
int tlh_gelu(const float *a, float *out, size_t n, void *stream);
int tlh_gelu_derivative(const float *a, float *out, size_t n, void *stream);
int tlh_copy(const float *a, float *out, size_t n, void *stream);

/* Fused GELU backward: out = grad * GELU'(x). Replaces the executor's
 * GELU_derivative + hadamard pair (autograd of expr/gelu.h). */
int tlh_gelu_backward(const float *grad, const float *x, float *out, size_t n,
                      void *stream);

/* Many row-major matrices transposed in one launch (no counterpart in the
 * reference: the GPT step program keeps K-contiguous copies of its weights
 * for the forward products with it). Job i transposes the rows x cols
 * matrix at src + src_offset into the cols x rows matrix at dst +
 * dst_offset; first_tile is the number of 64x64 output tiles of the jobs
 * before it and total_tiles the sum over all jobs. `jobs` is a device array
 * of `count` <= 256 entries; sources and destinations must not overlap.
 * Tiles past the last job's own (total_tiles larger than the sum) write
 * nothing; a table whose first_tile values descend (or exceed total_tiles)
 * is inconsistent, and then the launch writes nothing at all. */
typedef struct tlh_transpose_job {
  uint64_t src_offset, dst_offset;
  uint32_t rows, cols;
  uint32_t first_tile, reserved;
} tlh_transpose_job;
int tlh_transpose_multi(const float *src, float *dst, const tlh_transpose_job *jobs,
                        uint32_t count, uint32_t total_tiles, void *stream);

/* transpose (math.metal:566-584, runtime.cpp:529-569): `out` is contiguous
 * with `ndim` dims `out_shape`; in_strides are the input's strides with the
 * two swapped axes exchanged (runtime.cpp:549-553). Any permutation of
 * strides works. ndim <= 8. */
int tlh_transpose(const float *a, float *out, uint32_t ndim,
                  const uint32_t *out_shape, const uint32_t *in_strides,
                  void *stream);

/* ---------------------------------------------------------------------------
 * Matrix products (math.metal:13-400, runtime.cpp:375-505)
 * ------------------------------------------------------------------------- */

/* Runtime::mult: C[b..,M,N] = A[b..,M,K] . B[b..,K,N] in fp32 on the MFMA
 * units. Row/column element strides of each operand (a_rs, a_cs, ...) follow
 * runtime.cpp:458-463; one of each pair must be 1 (column-major operands run
 * the transposed-operand kernels). C must be row-major (c_cs == 1). Batch
 * dims (<= 4) decode like matmul_contiguous (math.metal:48-61): batch element
 * strides per operand, 0 = broadcast (runtime.cpp:437-446). */
int tlh_matmul(const float *a, const float *b, float *c, uint32_t M, uint32_t K,
               uint32_t N, uint32_t a_rs, uint32_t a_cs, uint32_t b_rs,
               uint32_t b_cs, uint32_t c_rs, uint32_t c_cs, uint32_t batch_ndim,
               const uint32_t *batch_shape, const uint32_t *batch_stride_a,
               const uint32_t *batch_stride_b, const uint32_t *batch_stride_c,
               void *stream);
/* Scratch (floats) that tlh_matmul_ws can use for this product: the K-chunk
 * partials of the tail split or of split-K (see tlh_gemm_workspace_size);
 * 0 when the plan needs none. Takes tlh_matmul's shape and stride
 * arguments. */
int tlh_matmul_workspace_size(uint32_t M, uint32_t K, uint32_t N, uint32_t a_rs,
                              uint32_t a_cs, uint32_t b_rs, uint32_t b_cs, uint32_t c_rs,
                              uint32_t c_cs, uint32_t batch_ndim, const uint32_t *batch_shape,
                              const uint32_t *batch_stride_a, const uint32_t *batch_stride_b,
                              const uint32_t *batch_stride_c, size_t *elems);
/* tlh_matmul with that scratch (partials summed in a fixed order: the
 * result does not depend on the split). A null or too small workspace runs
 * the unsplit plan of tlh_matmul. */
int tlh_matmul_ws(const float *a, const float *b, float *c, uint32_t M, uint32_t K,
                  uint32_t N, uint32_t a_rs, uint32_t a_cs, uint32_t b_rs, uint32_t b_cs,
                  uint32_t c_rs, uint32_t c_cs, uint32_t batch_ndim,
                  const uint32_t *batch_shape, const uint32_t *batch_stride_a,
                  const uint32_t *batch_stride_b, const uint32_t *batch_stride_c,
                  float *workspace, size_t workspace_elems, void *stream);

/* tlh_matmul_ws with a bias row added in the product's epilogue: c =
 * a.b + bias, bias [N] shared by every row and batch entry; the same bits as
 * the product followed by the broadcast add. With gelu_pre non-NULL (no
 * batch entries) gelu_pre = a.b + bias and c = GELU(gelu_pre), as
 * tlh_gelu computes it. The reference runtime has no fused form: it serves
 * the executor's LINEAR, mult then add of the bias (include/passes/
 * execute.h:242-253), and the GELU that may follow (execute.h:477-482). */
int tlh_matmul_bias_ws(const float *a, const float *b, float *c, const float *bias,
                       float *gelu_pre, uint32_t M,
                       uint32_t K, uint32_t N, uint32_t a_rs, uint32_t a_cs, uint32_t b_rs,
                       uint32_t b_cs, uint32_t c_rs, uint32_t c_cs, uint32_t batch_ndim,
                       const uint32_t *batch_shape, const uint32_t *batch_stride_a,
                       const uint32_t *batch_stride_b, const uint32_t *batch_stride_c,
                       float *workspace, size_t workspace_elems, void *stream);
/* Allocation-free form of tlh_matmul_ws. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Takes tlh_matmul's arguments; the K-chunk partials live in a
 * library-owned device array of TLH_NOALLOC_SCRATCH_FLOATS floats (32 MiB)
 * that each GPU holds from tlh_init (or the first call on that device)
 * until the process ends. Runs the plan and gives the results of
 * tlh_matmul_ws with tlh_matmul_workspace_size's workspace, bit for bit.
 * Returns hipErrorInvalidValue, launching nothing, when that size exceeds
 * TLH_NOALLOC_SCRATCH_FLOATS (use tlh_matmul_ws then). Every call on one GPU
 * shares the array: calls on one stream are ordered, calls that overlap on
 * one GPU (other streams, other threads) race. Calls no allocator. */
#define TLH_NOALLOC_SCRATCH_FLOATS (8u * 1024u * 1024u)
int tlh_matmul_noalloc(const float *a, const float *b, float *c, uint32_t M, uint32_t K,
                       uint32_t N, uint32_t a_rs, uint32_t a_cs, uint32_t b_rs,
                       uint32_t b_cs, uint32_t c_rs, uint32_t c_cs, uint32_t batch_ndim,
                       const uint32_t *batch_shape, const uint32_t *batch_stride_a,
                       const uint32_t *batch_stride_b, const uint32_t *batch_stride_c,
                       void *stream);

/* Fused GEMM used by the program layer (no reference counterpart; it fuses
 * EXPR_LINEAR = mult + in-place bias add (execute.h:241-252), the GELU that
 * follows, the residual add, and MULT_LHS/RHS_DERIVATIVE's transposes
 * (execute.h:187-232) into one launch). */
enum {
  TLH_EPI_STORE = 0,    /* C = acc (+bias) (+beta*C) (+residual) */
  TLH_EPI_GELU = 1,     /* aux = acc + bias; C = GELU(aux) */
  TLH_EPI_GELU_BWD = 2  /* C = acc * GELU'(aux) */
};

typedef struct tlh_gemm_desc {
  const float *a;        /* op(A) [M,K]: stored [M,K] (lda), or [K,M] if trans_a */
  const float *b;        /* op(B) [K,N]: stored [K,N] (ldb), or [N,K] if trans_b */
  float *c;              /* [M,N] row stride ldc, or head layout (remap_*) */
  const float *bias;     /* [N] or NULL */
  const float *residual; /* indexed like c, or NULL */
  float *aux;            /* GELU pre-activation, indexed like c, or NULL */
  float *workspace;      /* partials, tlh_gemm_workspace_size elems (or NULL) */
  int32_t m, n, k;
  int32_t lda, ldb, ldc;
  int32_t trans_a, trans_b;
  float beta;
  int32_t epilogue;
  /* if remap_h > 0: element (m = b*remap_t + t, n = h*remap_d + d) is stored
   * at ((b*remap_h + h)*remap_t + t)*remap_d + d. M is a multiple of
   * remap_t (whole sequences) or at most remap_t (rows of one sequence; c
   * may point t0 rows into the planes to store rows t0.. of a sequence). */
  int32_t remap_t, remap_h, remap_d;
  /* if non-NULL: bias_grad[n] = beta*bias_grad[n] + sum_k op(B)[k][n]. For a
   * weight gradient C = X^T.dY this is the bias gradient (the reference's
   * sum_to_shape of dY to [1,N], runtime.cpp:661-739), computed from the dY
   * tiles the GEMM already stages in LDS. Not with remap_* or batching. */
  float *bias_grad;
  /* Batched form (batch > 1): entry z reads a + z*batch_stride_a,
   * b + z*batch_stride_b, bias + z*bias_batch_stride and writes
   * c + z*batch_stride_c and bias_grad + z*bias_batch_stride (element
   * strides; 0 shares an operand). No residual, aux or GELU epilogue.
   * With sum_batches != 0 the entries are instead summed into one c:
   * c = sum_z op(A_z).op(B_z) (+bias, +beta*c, +residual once), i.e. one
   * product over K*batch whose K range z uses operands z (k must be a
   * multiple of 32; no bias_grad). batch <= 1 is the single product. */
  int32_t batch;
  uint32_t batch_stride_a, batch_stride_b, batch_stride_c, bias_batch_stride;
  int32_t sum_batches;
  /* fp32 elements available at `workspace`; 0 = sized with
   * tlh_gemm_workspace_size for this descriptor. Besides split-K partials
   * the workspace holds the K-chunk partials of a tail split: when the
   * output tiles do not spread evenly over the CUs, the tiles beyond a
   * multiple of the CU count are cut into K chunks and summed in a fixed
   * order afterwards (used only when the workspace is large enough). */
  size_t workspace_elems;
} tlh_gemm_desc;

int tlh_gemm(const tlh_gemm_desc *desc, void *stream);
/* fp32 elements of workspace tlh_gemm wants for `desc` (0: none needed).
 * One-row products (m = 1, neither operand transposed, b float4-aligned, no
 * bias gradient) run as a GEMV over K chunks when a workspace is given:
 * their chunk sums are added in a fixed order (deterministic). */
int tlh_gemm_workspace_size(const tlh_gemm_desc *desc, size_t *elems);
/* Tuning hook: force every following tlh_gemm / tlh_matmul to use a
 * bm x bn tile (64 or 128 each; or 96 x 96 with bk 32 (4 waves) or 64 (8
 * waves); or 96 x 64 with bk 32 (4 waves) or 64 (8 waves); or, with bm = 16, the 16x16x4
 * MFMA kernel at bn x bn, bn 64 or
 * 128, bk 32), a K tile of bk (16 or 32) and, where a
 * workspace allows it, `splits` K splits; bm = bn = 0 restores the
 * automatic plan. Process-wide, for measurement sweeps. A forced split
 * count needs a workspace sized for it (tlh_gemm_workspace_size).
 * bk = -1 / -2 instead switches the XCD-aware block order off / on
 * (default on), bk = -3 / -4 the tail split off / on (default on),
 * bk = -5 / -6 the rectangular XCD tile blocks off / on (default on),
 * bk = -7 / -8 the one-row (GEMV) path off / on (default on), bk = -9 /
 * -10 the float4 split-K reduce over a (plane, entry) grid off / on
 * (default on; off runs the grid-stride reduce, same bits), bk = -11 /
 * -12 the planner's 96x96 and 96x64 tiles off / on (default on), bk = -13 / -14 the
 * split-major XCD order of split-K and batched grids off / on (default on;
 * same bits), bk = -15 / -16 split weight gradients (A transposed, B not)
 * on the 16x16x4 kernel off / on (default on), bk = -17 / -18 products with
 * neither operand transposed on the 16x16x4 kernel where the planner takes
 * 128x128 / 64x128 tiles, or 64x64 tiles at K >= 384, off / on (default
 * on); these leave the plan alone. */
int tlh_gemm_set_plan(int bm, int bn, int splits, int bk);

/* ---------------------------------------------------------------------------
 * Reductions (math.metal:549-564, 618-777, 955-983)
 * ------------------------------------------------------------------------- */

/* sum of all elements (math.metal:549-564, runtime.cpp:506-518). */
int tlh_sum(const float *a, size_t n, float *out, void *stream);
/* sum_to_shape (math.metal:618-679, runtime.cpp:661-739): `a` is contiguous
 * with `ndim` dims a_shape; `out` is contiguous with the rank-aligned shape
 * out_shape (1 on reduced dims, equal otherwise). ndim <= 8. */
int tlh_sum_to_shape(const float *a, float *out, uint32_t ndim,
                     const uint32_t *a_shape, const uint32_t *out_shape,
                     void *stream);
/* Scratch (floats) that tlh_sum_to_shape_ws uses for this reduction; 0 when
 * it needs none. The tall column sums -- [R, K] -> [1, K] with R >= 256 and
 * K % 4 == 0, the bias gradients -- split the rows into chunks over about
 * 512 blocks and add the chunk partials in a fixed order (deterministic). */
int tlh_sum_to_shape_workspace(uint32_t ndim, const uint32_t *a_shape,
                               const uint32_t *out_shape, size_t *elems);
/* tlh_sum_to_shape with that scratch; with less scratch than asked for it
 * runs the single-pass kernels of tlh_sum_to_shape. */
int tlh_sum_to_shape_ws(const float *a, float *out, uint32_t ndim,
                        const uint32_t *a_shape, const uint32_t *out_shape,
                        float *workspace, size_t workspace_elems, void *stream);
/* max_to_shape (math.metal:681-714, runtime.cpp:595-659,741-745); same
 * shape rules as tlh_sum_to_shape. */
int tlh_max_to_shape(const float *a, float *out, uint32_t ndim,
                     const uint32_t *a_shape, const uint32_t *out_shape,
                     void *stream);
/* argmax (math.metal:715-777, runtime.cpp:850-918): index of the first
 * maximum (lowest index on ties; NaNs never win). n >= 1. */
int tlh_argmax(const float *a, size_t n, uint32_t *out_index, void *stream);
/* Top-k sampling with temperature, one row at a time on the device:
 * inference::sample_top_k (include/inference.h:14-43) -- candidates are the
 * top_k (clamped to [1, vocab]) largest logits, descending (equal logits:
 * lower token first, where the reference's partial_sort leaves the order
 * unspecified; NaN ranks as -INF), weights exp((l_i - l_0) / temperature)
 * in fp32 and std::discrete_distribution's draw (cumulative sums of w_i / S
 * in double, the last set to 1, the first >= u) -- plus the EOS re-draw of
 * inference::autoregression (inference.h:80-84): with resample_eos a draw
 * that yields eos_token is repeated with the next uniform, at most
 * max_draws draws (then the last result stands; the reference would loop
 * on). Uniform d of row r is uniforms[r * max_draws + d] when `uniforms`
 * (device, rows * max_draws doubles in [0, 1)) is given -- e.g. the
 * generate_canonical<double, 53> draws of the reference's std::mt19937 --
 * else output number counter + r * max_draws + d + 1 of the SplitMix64
 * stream seeded with `seed`, as (x >> 11) * 2^-53. tokens[r] = the token;
 * draws[r] (optional) = the draws used. 1 <= vocab <= 4096; temperature
 * finite and > 0; row_stride >= vocab when rows > 1 (0 with one row is
 * ignored). */
int tlh_sample_top_k(const float *logits, uint32_t rows, uint32_t vocab, uint32_t row_stride,
                     uint32_t top_k, float temperature, uint64_t seed, uint64_t counter,
                     const double *uniforms, uint32_t eos_token, int resample_eos,
                     uint32_t max_draws, uint32_t *tokens, uint32_t *draws, void *stream);
/* Row argmax: out[r] = argmax over a[r, 0:cols] (greedy decoding). */
int tlh_argmax_rows(const float *a, size_t rows, uint32_t cols,
                    uint32_t *out_index, void *stream);
/* accumulate_gradient_squared_norm (math.metal:955-983,
 * runtime.cpp:1083-1101): *squared_norm += sum(g^2). */
int tlh_accumulate_gradient_squared_norm(const float *g, size_t n,
                                         float *squared_norm, void *stream);
/* Multi-tensor version (Compiled::step(max_norm)'s loop over every gradient,
 * include/passes/compile.h:241-245, in one launch): *squared_norm = sum over
 * `count` tensors of g^2. grads / sizes are device arrays; `partials` is
 * device scratch of TLH_NORM_PARTIALS floats. Deterministic (fixed
 * reduction order, no atomics). count <= 2048. */
#define TLH_NORM_PARTIALS 1024
int tlh_gradient_squared_norm_multi(const float *const *grads,
                                    const uint64_t *sizes, uint32_t count,
                                    float *partials, float *squared_norm,
                                    void *stream);
/* Column sums: out[c] (+)= sum_r a[r, c]  (bias gradients, the
 * sum_to_shape [.., N] -> [1, N] case). beta scales the old out. */
int tlh_column_sum(const float *a, size_t rows, uint32_t cols, float *out,
                   float beta, void *stream);

/* ---------------------------------------------------------------------------
 * Row ops (math.metal:857-953, runtime.cpp:747-841, 1031-1072)
 * ------------------------------------------------------------------------- */

/* softmax over the last dim (math.metal:857-882, runtime.cpp:747-766). */
int tlh_softmax(const float *x, float *out, size_t rows, uint32_t cols,
                void *stream);
/* Softmax backward: out = y * (g - sum(g*y)) per row (EXPR_SFTMX_DERIVATIVE,
 * execute.h:291-308). out may alias g. */
int tlh_softmax_backward(const float *g, const float *y, float *out,
                         size_t rows, uint32_t cols, void *stream);
/* cross_entropy_rows (math.metal:884-910, runtime.cpp:768-804): loss[r] =
 * max + log(sum exp(x - max)) - x[t]; target >= vocab -> +INF. */
int tlh_cross_entropy_rows(const float *logits, const uint32_t *targets,
                           float *losses, size_t rows, uint32_t vocab,
                           void *stream);
/* cross_entropy_rows_backward (math.metal:912-953, runtime.cpp:806-841):
 * grad = softmax(x) - onehot(t); target >= vocab -> row of +INF. If
 * row_scale != NULL each row is multiplied by row_scale[r] (fuses the
 * upstream hadamard of autograd). */
int tlh_cross_entropy_rows_backward(const float *logits, const uint32_t *targets,
                                    float *grad, size_t rows, uint32_t vocab,
                                    const float *row_scale, void *stream);
/* Fused forward + backward in one pass over the logits: losses as
 * tlh_cross_entropy_rows, grad as tlh_cross_entropy_rows_backward times
 * `scale` (the uniform root gradient 1/(B*T) of src/train.cpp:109-113). */
int tlh_cross_entropy_rows_fused(const float *logits, const uint32_t *targets,
                                 float *losses, float *grad, size_t rows,
                                 uint32_t vocab, float scale, void *stream);
/* RMS (runtime.cpp:1031-1052): rms[r] = sqrt(sum(x^2)/cols + eps). */
int tlh_rms(const float *x, float *rms, size_t rows, uint32_t cols, float eps,
            void *stream);
/* RMSNorm (runtime.cpp:1060-1072): y = x / rms (* gain[c] if gain != NULL);
 * rms_out (nullable) receives rms per row. Single pass. */
int tlh_rms_norm(const float *x, const float *gain, float *y, float *rms_out,
                 size_t rows, uint32_t cols, float eps, void *stream);
/* RMSNorm backward (EXPR_RMSN_DERIVATIVE, execute.h:330-356, extended with
 * the optional gain): with n = x/rms, gy = g*gain,
 * dx = (gy - n*mean(gy*n)) / rms; dx_out = beta*dx_out + dx. grad_gain
 * (nullable) receives sum over rows of g*n (overwritten). */
int tlh_rms_norm_backward(const float *g, const float *x, const float *gain,
                          float *dx, float *grad_gain, size_t rows,
                          uint32_t cols, float eps, float beta, void *stream);

/* ---------------------------------------------------------------------------
 * Embedding (math.metal:778-820, runtime.cpp:920-1030)
 * ------------------------------------------------------------------------- */

/* embedding_lookup / gather_rows (math.metal:778-793, runtime.cpp:920-950):
 * out[i, :] = weights[ids[i], :], a bit-exact copy. weights is [rows, dim].
 * The reference reads unchecked; here a row whose id is >= rows is written
 * as NaN, so a bad id never reads outside the table. */
int tlh_embedding_lookup(const float *weights, uint32_t rows, uint32_t dim,
                         const uint32_t *ids, size_t n_ids, float *out,
                         void *stream);
/* Fused token+position embedding: out[b,t,:] = tok[ids[b,t],:] + pos[t,:]
 * (GPT.h:62-64: add(embedding(input), embedding(positions))). tok is
 * [vocab, dim]; an id >= vocab gives a NaN row. */
int tlh_embedding_add_positions(const float *tok, uint32_t vocab, const float *pos,
                                const uint32_t *ids, uint32_t batch,
                                uint32_t seq, uint32_t dim, float *out,
                                void *stream);
/* scatter_add_rows (math.metal:794-820, runtime.cpp:952-981): dst[ids[i],:]
 * += values[i,:]. The reference adds with relaxed float atomics (summation
 * order varies run to run); here every element receives its contributions
 * in increasing i, without atomics, so the result is deterministic and
 * equals the sequential loop bit for bit. dst is [dst_rows, dim]; ids >=
 * dst_rows are dropped. The caller pre-fills dst (base copy or zero,
 * runtime.cpp:983-1030). */
int tlh_scatter_add_rows(const float *values, const uint32_t *ids, size_t n_ids,
                         uint32_t dim, float *dst, uint32_t dst_rows, void *stream);
/* ---------------------------------------------------------------------------
 * Attention (no reference op: replaces the decomposed chain of
 * include/nn/multi_head.h:33-55)
 * ------------------------------------------------------------------------- */

/* Fused causal multi-head attention forward:
 *   O = softmax(Q K^T * scale + mask) V,  mask = 0 / -inf above the diagonal
 * q, k, v: [B, H, T, D] contiguous; o: [B, T, H*D] (heads merged, the
 * layout merge_last_dims produces) when o_merged != 0, else [B, H, T, D];
 * lse: [B, H, T] log-sum-exp of the scaled masked scores (for backward).
 * D must be 64. */
int tlh_attention_forward(const float *q, const float *k, const float *v,
                          float *o, float *lse, uint32_t batch, uint32_t heads,
                          uint32_t seq, uint32_t head_dim, float scale,
                          int causal, int o_merged, void *stream);
/* Single-query causal attention for incremental decoding: the query of
 * position t attends to keys 0..t (no reference op: the reference recomputes
 * the whole window per token, include/inference.h:70-98). q, k, v are
 * [heads, t_stride, 64] planes -- the forward's head layout at batch 1 --
 * and o is [heads * 64] (heads merged). t < t_stride <= 8192; head_dim 64. */
int tlh_attention_decode(const float *q, const float *k, const float *v, float *o,
                         uint32_t heads, uint32_t t_stride, uint32_t t,
                         uint32_t head_dim, float scale, void *stream);
/* Backward. do_ and o in the same layout as the forward's o (o_merged);
 * dq, dk, dv: [B, H, T, D] unless dqkv_merged != 0, then [B, T, H*D].
 * `delta` is scratch [B, H, T]. */
int tlh_attention_backward(const float *q, const float *k, const float *v,
                           const float *o, const float *do_, const float *lse,
                           float *delta, float *dq, float *dk, float *dv,
                           uint32_t batch, uint32_t heads, uint32_t seq,
                           uint32_t head_dim, float scale, int causal,
                           int o_merged, int dqkv_merged, void *stream);

/* ---------------------------------------------------------------------------
 * Optimiser (math.metal:985-1043, runtime.cpp:1103-1168)
 * ------------------------------------------------------------------------- */

/* clip_gradient (math.metal:985-1006): out = g * min(1, max_norm /
 * sqrt(max(*squared_norm, 1e-12))). out may alias g. */
int tlh_clip_gradient(const float *g, const float *squared_norm, float max_norm,
                      float *out, size_t n, void *stream);
/* clip_gradient over `count` tensors in one launch: dsts[i][j] = srcs[i][j]
 * * min(1, max_norm / sqrt(max(*squared_norm, 1e-12))) for j < sizes[i],
 * the arithmetic of tlh_clip_gradient; dsts[i] may be srcs[i], other
 * tensors must not overlap. No counterpart in the reference: it serves
 * Compiled::step(max_norm)'s per-gradient clip calls (compile.h:246-249),
 * which hip::Runtime collects. Device arrays; count <= 2048. */
int tlh_clip_multi(const float *const *srcs, float *const *dsts, const uint64_t *sizes,
                   uint32_t count, const float *squared_norm, float max_norm, void *stream);
/* adamW (math.metal:1008-1043, runtime.cpp:1129-1168): beta1, beta2, decay,
 * lr are 1-element device tensors (include/optimiser/AdamW.h:15-39). out may
 * alias param. step >= 1. */
int tlh_adamw(const float *param, const float *grad, float *out, float *m1,
              float *m2, const float *beta1, const float *beta2,
              const float *decay, const float *lr, float eps, uint32_t step,
              size_t n, void *stream);

/* Multi-tensor fused clip + AdamW: one launch updates `count` tensors in
 * place. Device arrays: params/grads/m1/m2 pointers, sizes, steps (uint32
 * per tensor: the per-parameter step_ of AdamW.h:42,78). If squared_norm
 * != NULL the gradient is scaled by min(1, max_norm/sqrt(max(s,1e-12)))
 * first (Compiled::step(max_norm), compile.h:236-258). count <= 2048. */
int tlh_adamw_multi(float *const *params, const float *const *grads,
                    float *const *m1, float *const *m2, const uint64_t *sizes,
                    const uint32_t *steps, uint32_t count, const float *beta1,
                    const float *beta2, const float *decay, const float *lr,
                    float eps, const float *squared_norm, float max_norm,
                    void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TEMPLIT_HIP_H */
