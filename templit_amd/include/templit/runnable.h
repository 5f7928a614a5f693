// The runtime contract the TempLit executor dispatches through, restated so
// this backend can check itself against it without the reference tree.
// Requirement for requirement it is passes::Runnable and its parts
// (include/passes/concepts.h:13-92): every op returns void and writes into
// a caller-shaped destination; indices are T::rebind<uint32_t>; AdamW's
// hyper-parameters are 1-element tensors; abort() is noexcept.
#pragma once

#include <concepts>
#include <cstddef>
#include <cstdint>

namespace templit {

template <typename T, typename Run>
concept GradientRuntime = requires(Run &run, T out, const T &a, const T &b) {
  { run.copy(a, out) } -> std::same_as<void>;
  { run.add(a, b, out) } -> std::same_as<void>;
};

template <typename T, typename Run>
concept ExecutionRuntime = GradientRuntime<T, Run> && requires(Run &run, T out, const T &a,
                                                               const T &b) {
  { run.sub(a, b, out) } -> std::same_as<void>;
  { run.mult(a, b, out) } -> std::same_as<void>;
  { run.transpose(a, out) } -> std::same_as<void>;
  { run.transpose(a, out, int32_t{}, int32_t{}) } -> std::same_as<void>;
  { run.split_last_dim(a, out, uint32_t{}, uint32_t{}) } -> std::same_as<void>;
  { run.merge_last_dims(a, out, uint32_t{}, uint32_t{}) } -> std::same_as<void>;
  { run.sigmoid(a, out) } -> std::same_as<void>;
  { run.hadamard(a, b, out) } -> std::same_as<void>;
  { run.divide(a, b, out) } -> std::same_as<void>;
  { run.sqrt(a, out) } -> std::same_as<void>;
  { run.sum(a, out) } -> std::same_as<void>;
  { run.sum(a, std::size_t{}, out) } -> std::same_as<void>;
  { run.sum_to_shape(a, a.shape(), out) } -> std::same_as<void>;
  { run.softmax(a, out) } -> std::same_as<void>;
  { run.sqe(a, b, out) } -> std::same_as<void>;
  { run.start() } -> std::same_as<void>;
  { run.submit() } -> std::same_as<void>;
  { run.wait() } -> std::same_as<void>;
  { run.abort() } noexcept -> std::same_as<void>;
};

template <typename T, typename Run>
concept NeuralRuntime = requires(Run &run, T out, const T &a, typename T::value_type s) {
  { run.divide(a, s, out) } -> std::same_as<void>;
  { run.pow(a, s, out) } -> std::same_as<void>;
  { run.RMS(a, out) } -> std::same_as<void>;
  { run.RMSNorm(a, out) } -> std::same_as<void>;
  { run.GELU(a, out) } -> std::same_as<void>;
  { run.GELU_derivative(a, out) } -> std::same_as<void>;
};

template <typename T, typename Run>
concept IndexedRuntime = requires(Run &run, T out, const T &a, const T &b,
                                  const typename T::template rebind<uint32_t> &ids) {
  { run.embedding_lookup(a, ids, out) } -> std::same_as<void>;
  { run.gather_rows(a, ids, out) } -> std::same_as<void>;
  { run.scatter_add_rows(a, ids, b, out) } -> std::same_as<void>;
  { run.scatter_index(a, ids, out) } -> std::same_as<void>;
  { run.cross_entropy(a, ids, out) } -> std::same_as<void>;
  { run.cross_entropy_derivative(a, ids, out) } -> std::same_as<void>;
};

template <typename T, typename Run>
concept GradientClippingRuntime = requires(Run &run, T out, const T &g, const T &s,
                                           typename T::value_type max_norm) {
  { run.accumulate_gradient_squared_norm(g, out) } -> std::same_as<void>;
  { run.clip_gradient(g, s, max_norm, out) } -> std::same_as<void>;
};

template <typename T, typename Run>
concept AdamWRuntime = requires(Run &run, T out, T m1, T m2, const T &p, const T &g,
                                const T &beta1, const T &beta2, const T &decay, const T &lr,
                                typename T::value_type eps) {
  { run.adamW(p, g, out, m1, m2, beta1, beta2, decay, lr, eps, uint32_t{}) } -> std::same_as<void>;
};

template <typename T, typename Run>
concept Runnable = ExecutionRuntime<T, Run> && NeuralRuntime<T, Run> && IndexedRuntime<T, Run> &&
                   GradientClippingRuntime<T, Run> && AdamWRuntime<T, Run>;

} // namespace templit
