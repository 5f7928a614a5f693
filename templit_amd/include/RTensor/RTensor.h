// RTensor<Device, T>: the tensor handle the runtime surface is written
// against. Its public interface is the reference's
// (include/RTensor/RTensor.h:23-368) so that executor code written for that
// type compiles unchanged against this one:
//   - uint32 shape and row-major strides computed at construction, at most
//     2^32-1 elements (std::length_error beyond);
//   - a reference-counted Storage<Device, T> shared by copies and views
//     (public `int ref_count` on the storage);
//   - host element access get/set, bulk set/read, contiguous-only view,
//     from_values / from_zeros, clone, byte-equality ==, archive save/load.
// Device memory management belongs to Storage<Device, T>; this class only
// holds shape, strides and the storage pointer.
#pragma once

#include "RTensor/storage.h"
#include "model_utils/archive_concepts.h"

#include <cassert>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <initializer_list>
#include <limits>
#include <numeric>
#include <ostream>
#include <span>
#include <stdexcept>
#include <utility>
#include <vector>

namespace rtensor {
using index_type = uint32_t;
using shape_type = std::vector<index_type>;

// Row-major strides of `shape`; throws if the element count does not fit
// the 32-bit index type. Returns the element count (1 for rank 0).
inline size_t contiguous_strides(std::span<const index_type> shape, shape_type &strides) {
  strides.assign(shape.size(), 0);
  size_t count = 1;
  for (size_t i = shape.size(); i-- > 0;) {
    strides[i] = static_cast<index_type>(count);
    count *= shape[i];
    if (count > std::numeric_limits<index_type>::max())
      throw std::length_error("RTensor exceeds 32-bit indexing capacity");
  }
  return count;
}
} // namespace rtensor

template <typename device, typename T> class RTensor {
public:
  using device_type = device;
  using index_type = rtensor::index_type;
  using shape_type = rtensor::shape_type;
  using value_type = T;
  template <typename U> using rebind = RTensor<device, U>;
  using storage_type = Storage<device, T>;

  // An empty handle with no storage (what a default-constructed slot holds
  // until it is assigned).
  RTensor() = default;

  RTensor(std::initializer_list<index_type> dims)
      : RTensor(std::span<const index_type>(dims.begin(), dims.size())) {}

  RTensor(std::span<const index_type> dims) : shape_(dims.begin(), dims.end()) {
    const size_t count = rtensor::contiguous_strides(shape_, strides_);
    storage_ = new storage_type(count);
    storage_->ref_count = 1;
  }

  // A [1,1] tensor holding `value` (the reference's scalar constructor).
  RTensor(T value)
    requires WritableStorage<Storage<device, T>, T>
      : shape_{1, 1}, strides_{1, 1} {
    storage_ = new storage_type(1);
    storage_->ref_count = 1;
    storage_->write(std::span<const T>(&value, 1), 0);
  }

  RTensor(const RTensor &other)
      : shape_(other.shape_), strides_(other.strides_), storage_(other.storage_) {
    if (storage_) storage_->ref_count += 1;
  }

  RTensor(RTensor &&other) noexcept
      : shape_(std::move(other.shape_)), strides_(std::move(other.strides_)),
        storage_(std::exchange(other.storage_, nullptr)) {}

  RTensor &operator=(const RTensor &other) {
    if (this == &other) return *this;
    storage_type *incoming = other.storage_;
    if (incoming) incoming->ref_count += 1;
    release();
    shape_ = other.shape_;
    strides_ = other.strides_;
    storage_ = incoming;
    return *this;
  }

  RTensor &operator=(RTensor &&other) noexcept {
    if (this == &other) return *this;
    release();
    shape_ = std::move(other.shape_);
    strides_ = std::move(other.strides_);
    storage_ = std::exchange(other.storage_, nullptr);
    other.shape_.clear();
    other.strides_.clear();
    return *this;
  }

  ~RTensor() { release(); }

  const storage_type *get_storage() const { return storage_; }
  storage_type *get_storage() { return storage_; }
  const shape_type &shape() const { return shape_; }
  const shape_type &strides() const { return strides_; }

  // Number of elements; 0 for a handle without a shape.
  size_t numel() const {
    if (shape_.empty()) return 0;
    return std::accumulate(shape_.begin(), shape_.end(), size_t{1}, std::multiplies<>{});
  }

  RTensor clone() const
    requires CloneableStorage<Storage<device, T>>
  {
    RTensor out;
    out.shape_ = shape_;
    out.strides_ = strides_;
    out.storage_ = storage_->clone();
    return out;
  }

  static RTensor from_values(std::initializer_list<std::initializer_list<T>> rows)
    requires WritableStorage<Storage<device, T>, T>
  {
    if (rows.size() == 0) return RTensor({0, 0});
    const size_t cols = rows.begin()->size();
    std::vector<T> flat;
    flat.reserve(rows.size() * cols);
    for (const auto &row : rows) {
      if (row.size() != cols) throw std::invalid_argument("Tensor initializer must be rectangular");
      flat.insert(flat.end(), row.begin(), row.end());
    }
    RTensor out({static_cast<index_type>(rows.size()), static_cast<index_type>(cols)});
    out.set(std::span<const T>(flat));
    return out;
  }

  static RTensor from_zeros(std::initializer_list<index_type> dims)
    requires FillableStorage<Storage<device, T>, T>
  {
    return from_zeros(std::span<const index_type>(dims.begin(), dims.size()));
  }

  static RTensor from_zeros(std::span<const index_type> dims)
    requires FillableStorage<Storage<device, T>, T>
  {
    RTensor out(dims);
    out.storage_->fill(T{});
    return out;
  }

  bool operator==(const RTensor &other) const
    requires ComparableStorage<Storage<device, T>>
  {
    return shape_ == other.shape_ && strides_ == other.strides_ &&
           storage_->compare(*other.storage_);
  }

  template <typename... Indices>
  T get(Indices... indices) const
    requires((std::convertible_to<Indices, size_t> && ...) &&
             ReadableStorage<Storage<device, T>, T>)
  {
    assert(sizeof...(Indices) == shape_.size());
    T out;
    storage_->read(std::span<T>(&out, 1), offset_of(indices...));
    return out;
  }

  template <typename... Indices>
  void set(T value, Indices... indices)
    requires((std::convertible_to<Indices, size_t> && ...) &&
             WritableStorage<Storage<device, T>, T>)
  {
    assert(sizeof...(Indices) == shape_.size());
    storage_->write(std::span<const T>(&value, 1), offset_of(indices...));
  }

  void set(std::span<const T> values)
    requires WritableStorage<Storage<device, T>, T>
  {
    const size_t expected =
        std::accumulate(shape_.begin(), shape_.end(), size_t{1}, std::multiplies<>{});
    if (values.size() != expected)
      throw std::invalid_argument("RTensor: values size does not match tensor shape");
    storage_->write(values, 0);
  }

  void read(std::span<T> values) const
    requires ReadableStorage<Storage<device, T>, T>
  {
    if (!storage_) throw std::logic_error("cannot read an uninitialised tensor");
    if (values.size() != numel())
      throw std::invalid_argument("RTensor: output size does not match tensor shape");
    storage_->read(values, 0);
  }

  // A reshaped handle on the same storage; only contiguous tensors can be
  // viewed and the element count must be preserved.
  RTensor view(std::span<const index_type> new_shape) const {
    if (!storage_) throw std::logic_error("cannot create a view of an uninitialised tensor");
    size_t expected_stride = 1;
    for (size_t i = shape_.size(); i-- > 0;) {
      if (strides_[i] != expected_stride)
        throw std::invalid_argument("cannot reshape a non-contiguous tensor");
      expected_stride *= shape_[i];
    }
    shape_type new_strides;
    const size_t new_count = rtensor::contiguous_strides(new_shape, new_strides);
    if (new_count != expected_stride)
      throw std::invalid_argument("view shape must preserve element count");
    RTensor out(*this);
    out.shape_.assign(new_shape.begin(), new_shape.end());
    out.strides_ = std::move(new_strides);
    return out;
  }

  friend std::ostream &operator<<(std::ostream &os, const RTensor &t)
    requires ReadableStorage<Storage<device, T>, T>
  {
    if (t.shape_.empty()) return os << "[]";
    std::vector<T> data(t.numel());
    t.storage_->read(std::span<T>(data), 0);
    size_t next = 0;
    std::function<void(size_t)> print = [&](size_t dim) {
      os << '[';
      for (size_t i = 0; i < t.shape_[dim]; ++i) {
        if (i) os << ", ";
        if (dim + 1 == t.shape_.size()) os << data[next++];
        else print(dim + 1);
      }
      os << ']';
    };
    print(0);
    return os;
  }

  // Archive layout of one tensor: "size" = the uint32 shape, "data" = the
  // elements in row-major order (reference RTensor.h:328-355).
  template <WritableArchive Arch> void save(Arch &archive) const {
    if (!storage_) throw std::logic_error("cannot save an uninitialised tensor");
    std::vector<T> data(numel());
    storage_->read(std::span<T>(data), 0);
    archive.write("size", std::as_bytes(std::span<const index_type>(shape_)));
    archive.write("data", std::as_bytes(std::span<const T>(data)));
  }

  template <ReadableArchive Arch> void load(const Arch &archive) {
    if (!storage_) throw std::logic_error("cannot load into an uninitialised tensor");
    shape_type stored(shape_.size());
    archive.read("size", std::as_writable_bytes(std::span(stored)));
    if (stored != shape_)
      throw std::runtime_error("current tensor shape and loaded tensor shape do not match");
    std::vector<T> data(numel());
    archive.read("data", std::as_writable_bytes(std::span(data)));
    storage_->write(std::span<const T>(data), 0);
  }

private:
  template <typename... Indices> size_t offset_of(Indices... indices) const {
    size_t offset = 0, dim = 0;
    ((offset += static_cast<size_t>(indices) * strides_[dim++]), ...);
    return offset;
  }

  void release() noexcept {
    if (!storage_) return;
    if (--storage_->ref_count == 0) delete storage_;
    storage_ = nullptr;
  }

  shape_type shape_;
  shape_type strides_;
  storage_type *storage_ = nullptr;
};
