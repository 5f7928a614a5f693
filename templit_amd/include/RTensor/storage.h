// Storage concepts of the tensor type: what RTensor<Device, T> asks of the
// device-specific Storage<Device, T>. Same names and requirements as the
// reference (include/RTensor/storage.h:7-29), so a storage written for one
// satisfies the other.
#pragma once

#include <concepts>
#include <cstddef>
#include <span>

template <typename Device, typename T> class Storage;

template <typename S, typename T>
concept WritableStorage = requires(S &s, std::span<const T> values, size_t offset) {
  s.write(values, offset);
};

template <typename S, typename T>
concept ReadableStorage = requires(const S &s, std::span<T> out, size_t offset) {
  s.read(out, offset);
};

template <typename S, typename T>
concept FillableStorage = requires(S &s, const T &value) { s.fill(value); };

template <typename S>
concept ComparableStorage = requires(const S &s) {
  { s.compare(s) } -> std::same_as<bool>;
};

template <typename S>
concept CloneableStorage = requires(const S &s) {
  { s.clone() } -> std::same_as<S *>;
};
