// oracle_runtime.h -- a CPU runtime over the oracle's restated kernels.
//
// TEST INFRASTRUCTURE ONLY: the checker the drop-in test (dropin_gpt.cpp)
// runs the reference executor on, next to hip::Runtime. It is never linked
// into the product libraries.
//
// orc::Runtime offers the operation surface of passes::Runnable
// (include/passes/concepts.h:13-92) on RTensor<orc::Host, float>, with host
// memory behind Storage<orc::Host, T>. Every op maps shapes to the oracle's
// C functions (oracle.h), which restate the reference CPU runtime
// (src/CPU/cpu.cpp) and the Metal kernels (include/my_metal/math.metal);
// the shape plumbing follows src/my_metal/runtime.cpp (broadcast strides
// 18-39, mult 375-505, reductions 595-739, RMS 1031-1072, scatter
// 952-1030, clip/AdamW validation 1103-1168).
#pragma once

#include "oracle.h"

#include "RTensor/RTensor.h"
#include "RTensor/dimension.h"
#include "RTensor/infer_shape.h"
#include "RTensor/storage.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <span>
#include <stdexcept>
#include <vector>

namespace orc {
struct Host {};
} // namespace orc

template <typename T> class Storage<orc::Host, T> {
public:
  explicit Storage(size_t n) : ref_count(1), data_(n) {}
  Storage(const Storage &) = delete;
  Storage &operator=(const Storage &) = delete;
  int ref_count;
  T *data() { return data_.data(); }
  const T *data() const { return data_.data(); }
  void write(std::span<const T> v, size_t off) {
    if (off + v.size() > data_.size()) throw std::out_of_range("write out of bounds");
    std::copy(v.begin(), v.end(), data_.begin() + off);
  }
  void read(std::span<T> v, size_t off) const {
    if (off + v.size() > data_.size()) throw std::out_of_range("read out of bounds");
    std::copy(data_.begin() + off, data_.begin() + off + v.size(), v.begin());
  }
  void fill(T value) { std::fill(data_.begin(), data_.end(), value); }
  Storage *clone() const {
    auto *s = new Storage(data_.size());
    s->data_ = data_;
    return s;
  }
  bool compare(const Storage &o) const {
    return o.data_.size() == data_.size() &&
           std::memcmp(o.data_.data(), data_.data(), data_.size() * sizeof(T)) == 0;
  }

private:
  std::vector<T> data_;
};

namespace orc {

class Runtime {
public:
  using Tensor = RTensor<Host, float>;
  using IndexTensor = RTensor<Host, uint32_t>;

  void start() {
    if (active_ || submitted_) throw std::logic_error("oracle runtime already started");
    active_ = true;
  }
  void submit() {
    if (!active_) throw std::logic_error("oracle runtime has not started");
    active_ = false;
    submitted_ = true;
  }
  void wait() {
    if (!submitted_ || active_) throw std::logic_error("oracle runtime has not been submitted");
    submitted_ = false;
  }
  void abort() noexcept { active_ = submitted_ = false; }

  void add(const Tensor &a, const Tensor &b, Tensor &o) { binary(ORC_ADD, a, b, o); }
  void sub(const Tensor &a, const Tensor &b, Tensor &o) { binary(ORC_SUB, a, b, o); }
  void hadamard(const Tensor &a, const Tensor &b, Tensor &o) { binary(ORC_MUL, a, b, o); }
  void divide(const Tensor &a, const Tensor &b, Tensor &o) { binary(ORC_DIV, a, b, o); }
  void add(const Tensor &a, float s, Tensor &o) { scalar(ORC_ADD_SCALAR, a, s, o); }
  void divide(const Tensor &a, float s, Tensor &o) { scalar(ORC_DIVIDE_SCALAR, a, s, o); }
  void pow(const Tensor &a, float s, Tensor &o) { scalar(ORC_POW_SCALAR, a, s, o); }
  void sigmoid(const Tensor &a, Tensor &o) { unary(ORC_SIGMOID, a, o); }
  void sqrt(const Tensor &a, Tensor &o) { unary(ORC_SQRT, a, o); }
  void exp(const Tensor &a, Tensor &o) { unary(ORC_EXP, a, o); }
  void GELU(const Tensor &a, Tensor &o) { unary(ORC_GELU, a, o); }
  void GELU_derivative(const Tensor &a, Tensor &o) { unary(ORC_GELU_DERIVATIVE, a, o); }
  void copy(const Tensor &a, Tensor &o) {
    if (a.shape() != o.shape()) throw std::invalid_argument("copy destination has incorrect shape");
    unary(ORC_COPY, a, o);
  }
  void sqe(const Tensor &p, const Tensor &t, Tensor &o) {
    sub(p, t, o);
    hadamard(o, o, o);
  }

  void mult(const Tensor &a, const Tensor &b, Tensor &o) {
    if (o.shape() != rtensor::infer_mult(a.shape(), b.shape()))
      throw std::invalid_argument("matmul destination has incorrect shape");
    const size_t ra = a.shape().size(), rb = b.shape().size(), ro = o.shape().size();
    const uint32_t M = a.shape()[ra - 2], K = a.shape()[ra - 1], N = b.shape()[rb - 1];
    std::vector<uint32_t> batch(o.shape().begin(), o.shape().end() - 2);
    const auto sa = strides(std::span(a.shape()).first(ra - 2), batch, size_t(M) * K);
    const auto sb = strides(std::span(b.shape()).first(rb - 2), batch, size_t(K) * N);
    orc_matmul(d(a), d(b), d(o), M, K, N, uint32_t(batch.size()), batch.data(), sa.data(),
               sb.data());
  }

  void transpose(const Tensor &a, Tensor &o, int32_t x = -2, int32_t y = -1) {
    if (o.shape() != rtensor::infer_transpose(a.shape(), x, y))
      throw std::invalid_argument("transpose destination has incorrect shape");
    auto s = a.strides();
    std::swap(s[rtensor::normalise_dimension(s.size(), x)],
              s[rtensor::normalise_dimension(s.size(), y)]);
    orc_transpose(d(a), d(o), uint32_t(o.shape().size()), o.shape().data(), s.data());
  }
  void split_last_dim(const Tensor &a, Tensor &o, uint32_t outer, uint32_t inner) {
    if (o.shape() != rtensor::infer_split_last_dim(a.shape(), outer, inner))
      throw std::invalid_argument("split_last_dim destination has incorrect shape");
    orc_unary(ORC_COPY, d(a), d(o), o.numel());
  }
  void merge_last_dims(const Tensor &a, Tensor &o, uint32_t outer, uint32_t inner) {
    if (o.shape() != rtensor::infer_merge_last_dims(a.shape(), outer, inner))
      throw std::invalid_argument("merge_last_dims destination has incorrect shape");
    orc_unary(ORC_COPY, d(a), d(o), o.numel());
  }

  void sum(const Tensor &a, Tensor &o) { *d(o) = orc_sum(d(a), a.numel()); }
  void sum(const Tensor &a, size_t axis, Tensor &o) {
    if (axis >= a.shape().size()) throw std::out_of_range("sum axis out of range");
    sum_to_shape(a, o.shape(), o);
  }
  void sum_to_shape(const Tensor &a, std::span<const uint32_t> shape, Tensor &o) {
    (void)rtensor::infer_sum_to_shape(a.shape(), shape);
    std::vector<uint32_t> aligned(a.shape().size(), 1);
    std::copy(shape.begin(), shape.end(), aligned.end() - shape.size());
    if (aligned == a.shape()) {
      orc_unary(ORC_COPY, d(a), d(o), o.numel());
      return;
    }
    orc_sum_to_shape(d(a), d(o), uint32_t(aligned.size()), a.shape().data(), aligned.data());
  }
  void max_to_shape(const Tensor &a, std::span<const uint32_t> shape, Tensor &o) {
    if (std::equal(shape.begin(), shape.end(), a.shape().begin(), a.shape().end())) {
      o = a;
      return;
    }
    orc_max_to_shape(d(a), d(o), uint32_t(shape.size()), a.shape().data(), shape.data());
  }
  void argmax(const Tensor &a, IndexTensor &o) { *d(o) = orc_argmax(d(a), a.numel()); }

  void softmax(const Tensor &x, Tensor &o) {
    orc_softmax(d(x), d(o), x.numel() / x.shape().back(), x.shape().back());
  }
  void cross_entropy(const Tensor &l, const IndexTensor &t, Tensor &o) {
    if (o.shape() != rtensor::infer_cross_entropy(l.shape(), t.shape()))
      throw std::invalid_argument("cross_entropy destination has incorrect shape");
    orc_cross_entropy_rows(d(l), d(t), d(o), t.numel(), l.shape().back());
  }
  void cross_entropy_derivative(const Tensor &l, const IndexTensor &t, Tensor &o) {
    if (o.shape() != rtensor::infer_cross_entropy_derivative(l.shape(), t.shape()))
      throw std::invalid_argument("cross_entropy_derivative destination has incorrect shape");
    orc_cross_entropy_rows_backward(d(l), d(t), d(o), t.numel(), l.shape().back());
  }
  // RMS with the reference's epsilon 1e-6 inside the root (runtime.cpp:1044-1052).
  void RMS(const Tensor &a, Tensor &o) {
    orc_rms(d(a), d(o), a.numel() / a.shape().back(), a.shape().back(), 1e-6f);
  }
  void RMSNorm(const Tensor &a, Tensor &o) {
    orc_rms_norm(d(a), nullptr, d(o), nullptr, a.numel() / a.shape().back(), a.shape().back(),
                 1e-6f);
  }

  void embedding_lookup(const Tensor &w, const IndexTensor &ids, Tensor &o) {
    orc_embedding_lookup(d(w), w.shape()[1], d(ids), ids.numel(), d(o));
  }
  void gather_rows(const Tensor &w, const IndexTensor &ids, Tensor &o) { embedding_lookup(w, ids, o); }
  void scatter_add_rows(const Tensor &base, const IndexTensor &ids, const Tensor &v, Tensor &o) {
    if (base.get_storage() != o.get_storage()) orc_unary(ORC_COPY, d(base), d(o), o.numel());
    orc_scatter_add_rows(d(v), d(ids), ids.numel(), o.shape()[1], d(o));
  }
  void scatter_index(const Tensor &v, const IndexTensor &ids, Tensor &o) {
    std::fill(d(o), d(o) + o.numel(), 0.0f);
    orc_scatter_add_rows(d(v), d(ids), ids.numel(), o.shape()[1], d(o));
  }

  void accumulate_gradient_squared_norm(const Tensor &g, Tensor &s) {
    orc_accumulate_gradient_squared_norm(d(g), g.numel(), d(s));
  }
  void clip_gradient(const Tensor &g, const Tensor &s, float max_norm, Tensor &o) {
    if (!(max_norm > 0.0f) || !std::isfinite(max_norm))
      throw std::invalid_argument("maximum gradient norm must be finite and positive");
    orc_clip_gradient(d(g), d(s), max_norm, d(o), g.numel());
  }
  void adamW(const Tensor &p, const Tensor &g, Tensor &o, Tensor &m1, Tensor &m2,
             const Tensor &b1, const Tensor &b2, const Tensor &decay, const Tensor &lr, float eps,
             uint32_t step) {
    if (step == 0) throw std::invalid_argument("AdamW step must be greater than zero");
    orc_adamw(d(p), d(g), d(o), d(m1), d(m2), *d(b1), *d(b2), *d(decay), *d(lr), eps, step,
              p.numel());
  }

private:
  bool active_ = false, submitted_ = false;

  template <typename T> static T *d(const RTensor<Host, T> &t) {
    return const_cast<T *>(t.get_storage()->data());
  }

  // Element strides of a batch shape right-aligned to `batch`, 0 where it
  // broadcasts; `matrix` elements per batch entry.
  static std::vector<uint32_t> strides(std::span<const uint32_t> shape,
                                       const std::vector<uint32_t> &batch, size_t matrix) {
    std::vector<uint32_t> out(batch.size(), 0);
    size_t stride = matrix;
    for (size_t i = shape.size(); i-- > 0;) {
      const size_t o = batch.size() - shape.size() + i;
      if (shape[i] != 1) out[o] = uint32_t(stride);
      stride *= shape[i];
    }
    return out;
  }

  void binary(int op, const Tensor &a, const Tensor &b, Tensor &o) {
    const auto sa = aligned_strides(a, o), sb = aligned_strides(b, o);
    orc_binary(op, d(a), d(b), d(o), uint32_t(o.shape().size()), o.shape().data(), sa.data(),
               sb.data());
  }
  static std::vector<uint32_t> aligned_strides(const Tensor &t, const Tensor &o) {
    std::vector<uint32_t> out(o.shape().size(), 0);
    if (t.shape().size() > o.shape().size()) throw std::runtime_error("invalid broadcast");
    const size_t off = o.shape().size() - t.shape().size();
    for (size_t i = 0; i < t.shape().size(); ++i) {
      if (t.shape()[i] == o.shape()[off + i]) out[off + i] = t.strides()[i];
      else if (t.shape()[i] != 1) throw std::runtime_error("invalid broadcast");
    }
    return out;
  }
  void unary(int op, const Tensor &a, Tensor &o) { orc_unary(op, d(a), d(o), o.numel()); }
  void scalar(int op, const Tensor &a, float s, Tensor &o) {
    if (a.shape() != o.shape())
      throw std::invalid_argument("scalar operation input and output shapes must match");
    orc_scalar(op, d(a), s, d(o), o.numel());
  }
};

} // namespace orc
