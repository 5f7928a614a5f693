// Storage<hip::HIP, T>: device memory behind RTensor<hip::HIP, T>.
//
// Interface of the Metal storage (include/my_metal/storage.h:11-63): public
// `int ref_count`, write/read(span, offset) with std::out_of_range on
// overflow, fill, clone, byte compare, non-copyable. The memory is HBM from
// the context's caching pool rather than a shared-mode buffer, so host
// access is an explicit, stream-ordered transfer (hip.h). data() is the
// device pointer the runtime hands to kernels (Metal: get_buffer()).
#pragma once

#include "RTensor/storage.h"
#include "my_hip/hip.h"

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <span>
#include <stdexcept>
#include <type_traits>
#include <utility>
#include <vector>

template <typename T> class Storage<hip::HIP, T> {
  static_assert(std::is_trivially_copyable_v<T>, "device storage holds trivially copyable values");

public:
  explicit Storage(size_t size)
      : ref_count(1), size_(size), data_(static_cast<T *>(hip::detail::allocate(size * sizeof(T)))) {}
  Storage(const Storage &) = delete;
  Storage &operator=(const Storage &) = delete;
  Storage(Storage &&) = delete;
  Storage &operator=(Storage &&) = delete;
  ~Storage() {
    hip::detail::before_access(data_, hip::detail::kAccessRelease);
    hip::detail::release(data_, size_ * sizeof(T));
  }

  int ref_count;

  T *data() { return data_; }
  const T *data() const { return data_; }
  void *get_buffer() const { return const_cast<T *>(data_); }
  size_t size() const { return size_; }

  void write(std::span<const T> values, size_t offset) {
    if (offset + values.size() > size_) throw std::out_of_range("write out of bounds");
    if (values.empty()) return;
    hip::detail::before_access(data_, hip::detail::kAccessWrite);
    hip::detail::write(data_ + offset, values.data(), values.size_bytes());
  }

  void read(std::span<T> out, size_t offset) const {
    if (offset + out.size() > size_) throw std::out_of_range("read out of bounds");
    if (out.empty()) return;
    hip::detail::before_access(data_, hip::detail::kAccessRead);
    hip::detail::read(out.data(), data_ + offset, out.size_bytes());
  }

  void fill(T value) {
    if (size_ == 0) return;
    hip::detail::before_access(data_, hip::detail::kAccessWrite);
    if constexpr (sizeof(T) == 4) {
      uint32_t pattern;
      std::memcpy(&pattern, &value, 4);
      hip::detail::fill32(data_, pattern, size_);
    } else {
      std::vector<T> host(size_, value);
      hip::detail::write(data_, host.data(), size_ * sizeof(T));
    }
  }

  Storage *clone() const {
    auto *other = new Storage(size_);
    if (size_) {
      hip::detail::before_access(data_, hip::detail::kAccessRead);
      hip::detail::copy(other->data_, data_, size_ * sizeof(T));
    }
    return other;
  }

  // Exchanges the device blocks of two storages of one size: the runtime
  // hands a block that pending work still reads to a storage of its own
  // instead of copying it out before the block is overwritten.
  void exchange_block(Storage &other) {
    if (other.size_ != size_) throw std::invalid_argument("exchange_block: sizes differ");
    std::swap(data_, other.data_);
  }

  bool compare(const Storage &other) const {
    if (other.size_ != size_) return false;
    hip::detail::before_access(data_, hip::detail::kAccessRead);
    hip::detail::before_access(other.data_, hip::detail::kAccessRead);
    return hip::detail::equal(data_, other.data_, size_ * sizeof(T));
  }

private:
  size_t size_;
  T *data_;
};
