// hip::Runtime -- the MI355X runtime backend of TempLit.
//
// Same operation surface as metal::Runtime (include/my_metal/runtime.h:
// 74-181), which is what passes::Compiled prepare()/forward()/backward()/
// step() dispatches through (the passes::Runnable concept,
// include/passes/concepts.h:13-92):
//   - every op takes its inputs by const reference and writes into a
//     destination the caller has already shaped; the shape is validated
//     first and a mismatch throws (std::invalid_argument, or the exception
//     type the reference uses for that op) before any work is enqueued;
//   - a, b and the destination may be the same tensor (in-place use);
//   - start()/submit()/wait()/abort() keep the Metal command-buffer state
//     machine: double start, submit before start and wait before submit
//     throw std::logic_error; ops outside start..submit throw it too.
//
// MI355X execution model. Every op calls the extern "C" kernel library
// (include/templit_hip.h) on the context's single in-order stream:
//   - eager mode (default): kernels are launched as the executor calls the
//     ops, so the GPU starts while the host is still encoding; submit() only
//     closes the recording and wait() synchronises the stream (and reports
//     any asynchronous kernel error as std::runtime_error);
//   - graph mode (set_graph_mode(true)): start() begins a stream capture,
//     submit() ends it and launches the recorded hipGraph. Executable graphs
//     are cached by the sequence of ops and shapes recorded; a repeat of a
//     known sequence refreshes the cached graph's kernel arguments
//     (hipGraphExecUpdate: new pointers, scalars, AdamW step) instead of
//     instantiating it again. Host writes made while recording (a constant
//     the executor sets, AdamW's first zero-fill of its moments) happen at
//     record time, as on Metal.
#pragma once

#include "RTensor/RTensor.h"
#include "my_hip/hip.h"
#include "my_hip/storage.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <span>
#include <string_view>

namespace hip {

class Runtime {
public:
  using Tensor = RTensor<HIP, kernel_type>;
  using IndexTensor = RTensor<HIP, index_type>;

  // Requires hip::init() (std::logic_error otherwise, as on Metal).
  Runtime();
  Runtime(const Runtime &) = delete;
  Runtime &operator=(const Runtime &) = delete;
  ~Runtime();

  // ---- lifecycle (runtime.cpp:170-317) ----
  void start();
  void submit();
  void wait();
  void abort() noexcept;
  void cleanup() noexcept;

  // Profiling span markers (Metal: GPU-trace capture). Here they bracket a
  // region for rocprofv3 (a kernel-trace run attributes the enclosed
  // dispatches to it); `output_path` names the region.
  void start_profile(std::string_view output_path);
  void end_profile();

  // ---- execution mode ----
  void set_graph_mode(bool enabled);
  bool graph_mode() const;
  struct GraphStats {
    size_t captures = 0;       // recordings submitted as graphs
    size_t instantiations = 0; // executable graphs built
    size_t updates = 0;        // cached graphs refreshed in place
  };
  GraphStats graph_stats() const;

  // ---- elementwise (runtime.cpp:321-373) ----
  void add(const Tensor &a, const Tensor &b, Tensor &out);
  void add(const Tensor &a, kernel_type scalar, Tensor &out);
  void sub(const Tensor &a, const Tensor &b, Tensor &out);
  void hadamard(const Tensor &a, const Tensor &b, Tensor &out);
  void divide(const Tensor &a, const Tensor &b, Tensor &out);
  void divide(const Tensor &a, kernel_type scalar, Tensor &out);
  void pow(const Tensor &a, kernel_type exponent, Tensor &out);
  void sigmoid(const Tensor &a, Tensor &out);
  void sqrt(const Tensor &a, Tensor &out);
  void exp(const Tensor &a, Tensor &out);
  void GELU(const Tensor &a, Tensor &out);
  void GELU_derivative(const Tensor &a, Tensor &out);
  void copy(const Tensor &a, Tensor &out);
  void sqe(const Tensor &prediction, const Tensor &target, Tensor &out);

  // ---- products and layout (runtime.cpp:375-505, 529-593) ----
  void mult(const Tensor &a, const Tensor &b, Tensor &out);
  void transpose(const Tensor &a, Tensor &out, int32_t dim_a = -2, int32_t dim_b = -1);
  void split_last_dim(const Tensor &a, Tensor &out, uint32_t outer, uint32_t inner);
  void merge_last_dims(const Tensor &a, Tensor &out, uint32_t outer, uint32_t inner);

  // ---- reductions (runtime.cpp:506-527, 595-745, 850-918) ----
  void sum(const Tensor &a, Tensor &out);
  void sum(const Tensor &a, size_t axis, Tensor &out);
  void sum_to_shape(const Tensor &a, std::span<const uint32_t> shape, Tensor &out);
  void max_to_shape(const Tensor &a, std::span<const uint32_t> shape, Tensor &out);
  void argmax(const Tensor &a, IndexTensor &out);

  // ---- row ops (runtime.cpp:747-841, 1031-1072) ----
  void softmax(const Tensor &x, Tensor &out);
  void cross_entropy(const Tensor &logits, const IndexTensor &targets, Tensor &out);
  void cross_entropy_derivative(const Tensor &logits, const IndexTensor &targets, Tensor &out);
  void RMS(const Tensor &a, Tensor &out);
  void RMSNorm(const Tensor &a, Tensor &out);

  // ---- embedding (runtime.cpp:920-1030) ----
  void embedding_lookup(const Tensor &weights, const IndexTensor &ids, Tensor &out);
  void gather_rows(const Tensor &values, const IndexTensor &ids, Tensor &out);
  void scatter_add_rows(const Tensor &base, const IndexTensor &ids, const Tensor &values,
                        Tensor &out);
  void scatter_index(const Tensor &values, const IndexTensor &ids, Tensor &out);

  // ---- optimiser (runtime.cpp:1083-1168) ----
  void accumulate_gradient_squared_norm(const Tensor &gradient, Tensor &squared_norm);
  void clip_gradient(const Tensor &gradient, const Tensor &squared_norm, kernel_type max_norm,
                     Tensor &out);
  void adamW(const Tensor &parameter, const Tensor &gradient, Tensor &out, Tensor &momentum1,
             Tensor &momentum2, const Tensor &beta1, const Tensor &beta2, const Tensor &decay,
             const Tensor &learning_rate, kernel_type epsilon, uint32_t step);

  // ---- fused extensions (no Metal counterpart; used by fused programs) ----
  // RMSNorm with an explicit epsilon and an optional per-column gain
  // ([last dim] or empty handle): y = x / sqrt(mean(x^2) + eps) * gain.
  void RMSNorm(const Tensor &a, const Tensor &gain, kernel_type epsilon, Tensor &out);
  // Softmax backward y * (g - sum(g*y)) per row: the executor's
  // SFTMX_DERIVATIVE chain (execute.h:291-308) in one kernel.
  void softmax_derivative(const Tensor &grad, const Tensor &y, Tensor &out);
  // grad * GELU'(x): GELU_derivative followed by hadamard, fused.
  void GELU_backward(const Tensor &grad, const Tensor &x, Tensor &out);
  // RMSNorm backward (execute.h:330-356): (g - y*mean(g*y)) / rms.
  void RMSNorm_derivative(const Tensor &grad, const Tensor &x, Tensor &out);
  // Causal multi-head attention over [B, H, T, 64] operands:
  // out = softmax(q k^T * scale + causal mask) v; lse [B, H, T] keeps the
  // row log-sum-exp for the backward. Replaces the decomposed chain of
  // include/nn/multi_head.h:37-52.
  void causal_attention(const Tensor &q, const Tensor &k, const Tensor &v, kernel_type scale,
                        Tensor &out, Tensor &lse);
  void causal_attention_backward(const Tensor &q, const Tensor &k, const Tensor &v,
                                 const Tensor &out, const Tensor &grad_out, const Tensor &lse,
                                 kernel_type scale, Tensor &grad_q, Tensor &grad_k,
                                 Tensor &grad_v);

private:
  struct State;
  std::unique_ptr<State> state_;

  // Throws unless recording; then runs the in-place clips batched so far
  // (unless `run_clips` is false: another clip joins the batch).
  void require_recording(const char *op, bool run_clips = true) const;
  void note(uint32_t op, std::span<const uint32_t> shape);
  void RMS_impl(const Tensor &a, Tensor &out);
  // sum_to_shape's reduction, `aligned` being the target right-aligned to
  // a's rank
  void reduce_to(const Tensor &a, const std::vector<uint32_t> &aligned, Tensor &out);
};

} // namespace hip
