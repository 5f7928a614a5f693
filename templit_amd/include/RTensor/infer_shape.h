// Output-shape rules of the runtime operations. Same function names and
// results as the reference's shape inference (include/RTensor/
// infer_shape.h:15-340) because executor code calls them to size the
// destinations it hands to the runtime:
//   - elementwise ops broadcast right-aligned (a dim of 1 stretches);
//   - mult broadcasts the batch dims and appends [M, N];
//   - reductions keep the rank (reduced dims become 1) or drop leading dims;
//   - errors: std::invalid_argument (incompatible shapes), std::runtime_error
//     (matmul rank / batch broadcast), std::out_of_range (axis).
#pragma once

#include "RTensor/RTensor.h"
#include "RTensor/dimension.h"

#include <algorithm>
#include <cstdint>
#include <limits>
#include <numeric>
#include <span>
#include <stdexcept>

namespace rtensor {

// Right-aligned broadcast of two shapes. `error` selects the exception type
// (mult reports batch mismatches as runtime_error, elementwise ops as
// invalid_argument).
template <typename Error = std::invalid_argument>
inline shape_type broadcast_shapes(std::span<const index_type> a, std::span<const index_type> b) {
  const size_t rank = std::max(a.size(), b.size());
  shape_type out(rank);
  for (size_t k = 0; k < rank; ++k) {
    const index_type da = k < a.size() ? a[a.size() - 1 - k] : 1;
    const index_type db = k < b.size() ? b[b.size() - 1 - k] : 1;
    if (da != db && da != 1 && db != 1) throw Error("shapes cannot be broadcast");
    out[rank - 1 - k] = std::max(da, db);
  }
  return out;
}

inline shape_type create_out(std::span<const index_type> a, std::span<const index_type> b) {
  return broadcast_shapes(a, b);
}
inline shape_type infer_add(std::span<const index_type> a, std::span<const index_type> b) {
  return broadcast_shapes(a, b);
}
inline shape_type infer_sub(std::span<const index_type> a, std::span<const index_type> b) {
  return broadcast_shapes(a, b);
}
inline shape_type infer_hadamard(std::span<const index_type> a, std::span<const index_type> b) {
  return broadcast_shapes(a, b);
}
inline shape_type infer_divide(std::span<const index_type> a, std::span<const index_type> b) {
  return broadcast_shapes(a, b);
}

inline shape_type infer_mult(std::span<const index_type> a, std::span<const index_type> b) {
  if (a.size() < 2 || b.size() < 2) throw std::runtime_error("matmul requires rank >= 2");
  if (a[a.size() - 1] != b[b.size() - 2])
    throw std::invalid_argument("matmul inner dimensions do not match");
  shape_type out = broadcast_shapes<std::runtime_error>(a.first(a.size() - 2), b.first(b.size() - 2));
  out.push_back(a[a.size() - 2]);
  out.push_back(b[b.size() - 1]);
  return out;
}

inline shape_type infer_unary(std::span<const index_type> s) { return shape_type(s.begin(), s.end()); }
inline shape_type infer_sigmoid(std::span<const index_type> s) { return infer_unary(s); }
inline shape_type infer_sqrt(std::span<const index_type> s) { return infer_unary(s); }
inline shape_type infer_exp(std::span<const index_type> s) { return infer_unary(s); }

inline shape_type infer_rms(std::span<const index_type> s) {
  if (s.empty()) throw std::invalid_argument("RMS requires rank >= 1");
  shape_type out(s.begin(), s.end());
  out.back() = 1;
  return out;
}

inline shape_type infer_rms_norm(std::span<const index_type> s) {
  if (s.empty()) throw std::invalid_argument("RMSNorm requires rank >= 1");
  return infer_unary(s);
}

inline shape_type infer_sum(std::span<const index_type>) { return {1}; }

inline shape_type infer_transpose(std::span<const index_type> s, int32_t dim_a = -2,
                                  int32_t dim_b = -1) {
  if (s.size() < 2) throw std::invalid_argument("transpose requires rank >= 2");
  const size_t x = normalise_dimension(s.size(), dim_a);
  const size_t y = normalise_dimension(s.size(), dim_b);
  if (x == y) throw std::invalid_argument("transpose dimensions must be different");
  shape_type out(s.begin(), s.end());
  std::swap(out[x], out[y]);
  return out;
}

inline shape_type infer_split_last_dim(std::span<const index_type> s, index_type outer,
                                       index_type inner) {
  if (s.empty()) throw std::invalid_argument("split_last_dim requires rank >= 1");
  if (outer == 0 || inner == 0 || uint64_t(outer) * inner != s.back())
    throw std::invalid_argument("split_last_dim factors must match the final dimension");
  shape_type out(s.begin(), s.end() - 1);
  out.push_back(outer);
  out.push_back(inner);
  return out;
}

inline shape_type infer_merge_last_dims(std::span<const index_type> s, index_type outer,
                                        index_type inner) {
  if (s.size() < 2) throw std::invalid_argument("merge_last_dims requires rank >= 2");
  if (s[s.size() - 2] != outer || s.back() != inner)
    throw std::invalid_argument("merge_last_dims factors do not match the final dimensions");
  const uint64_t merged = uint64_t(outer) * inner;
  if (merged > std::numeric_limits<index_type>::max())
    throw std::length_error("merged tensor dimension exceeds index capacity");
  shape_type out(s.begin(), s.end() - 2);
  out.push_back(index_type(merged));
  return out;
}

inline shape_type infer_embedding_lookup(std::span<const index_type> weights,
                                         std::span<const index_type> ids) {
  if (weights.size() != 2) throw std::invalid_argument("embedding weights must have rank 2");
  shape_type out(ids.begin(), ids.end());
  out.push_back(weights.back());
  return out;
}

inline shape_type infer_cross_entropy(std::span<const index_type> logits,
                                      std::span<const index_type> targets) {
  if (logits.size() < 2 || logits.back() == 0)
    throw std::invalid_argument("cross_entropy requires logits with a non-empty final dimension");
  if (targets.size() + 1 != logits.size())
    throw std::invalid_argument("cross_entropy target rank must be one less than logits rank");
  if (!std::equal(targets.begin(), targets.end(), logits.begin()))
    throw std::invalid_argument("cross_entropy target shape must match logits leading dimensions");
  shape_type out(targets.begin(), targets.end());
  out.push_back(1);
  return out;
}

inline shape_type infer_cross_entropy_derivative(std::span<const index_type> logits,
                                                 std::span<const index_type> targets) {
  (void)infer_cross_entropy(logits, targets);
  return shape_type(logits.begin(), logits.end());
}

inline shape_type infer_scatter_index(std::span<const index_type> values,
                                      std::span<const index_type> ids,
                                      std::span<const index_type> output) {
  if (output.size() != 2) throw std::invalid_argument("scatter output must have rank 2");
  shape_type expected(ids.begin(), ids.end());
  expected.push_back(output.back());
  if (!std::equal(values.begin(), values.end(), expected.begin(), expected.end()))
    throw std::invalid_argument("scatter values shape does not match IDs and output");
  return shape_type(output.begin(), output.end());
}

inline shape_type infer_scatter_add_rows(std::span<const index_type> base,
                                         std::span<const index_type> ids,
                                         std::span<const index_type> values) {
  return infer_scatter_index(values, ids, base);
}

// `out` may drop leading dims of `a`; every kept dim equals a's or is 1.
inline shape_type infer_reduce_to_shape(std::span<const index_type> a,
                                        std::span<const index_type> out) {
  if (out.size() > a.size()) throw std::invalid_argument("cannot reduce to a shape with a higher rank");
  const size_t lead = a.size() - out.size();
  for (size_t i = 0; i < a.size(); ++i) {
    const index_type o = i < lead ? 1 : out[i - lead];
    if (a[i] != o && o != 1) throw std::invalid_argument("invalid reduce_to_shape");
  }
  return shape_type(out.begin(), out.end());
}

inline shape_type infer_sum_to_shape(std::span<const index_type> a, std::span<const index_type> out) {
  return infer_reduce_to_shape(a, out);
}
inline shape_type infer_max_to_shape(std::span<const index_type> a, std::span<const index_type> out) {
  return infer_reduce_to_shape(a, out);
}

inline shape_type infer_sum(std::span<const index_type> s, size_t axis) {
  if (axis >= s.size()) throw std::out_of_range("sum axis out of range");
  shape_type out(s.begin(), s.end());
  out[axis] = 1;
  return infer_sum_to_shape(s, out);
}

inline shape_type infer_softmax(std::span<const index_type> s) {
  if (s.empty()) throw std::invalid_argument("softmax requires rank >= 1");
  return infer_unary(s);
}

inline shape_type infer_argmax(std::span<const index_type> s) {
  if (std::accumulate(s.begin(), s.end(), size_t{1}, std::multiplies<>{}) == 0)
    throw std::invalid_argument("argmax requires a non-empty tensor");
  return {1, 1};
}

} // namespace rtensor
