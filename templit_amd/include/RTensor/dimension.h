// Negative-axis normalisation (reference: include/RTensor/dimension.h:9-16):
// axis d of a rank-r tensor is d if d >= 0, r + d otherwise; anything
// outside [0, r) is std::out_of_range.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>

namespace rtensor {

inline size_t normalise_dimension(size_t rank, int32_t dimension) {
  const int64_t axis = dimension < 0 ? int64_t(rank) + dimension : int64_t(dimension);
  if (axis < 0 || axis >= int64_t(rank)) throw std::out_of_range("tensor dimension out of range");
  return size_t(axis);
}

} // namespace rtensor
