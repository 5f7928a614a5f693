// Checkpoint archive concepts used by RTensor::save/load: an archive maps a
// name to a byte blob (reference: include/model_utils/archive_concepts.h:7-23).
#pragma once

#include <concepts>
#include <cstddef>
#include <span>
#include <string>

template <typename A>
concept WritableArchive = requires(A &a, const std::string &name,
                                   std::span<const std::byte> bytes) {
  { a.write(name, bytes) } -> std::same_as<void>;
};

template <typename A>
concept ReadableArchive = requires(const A &a, const std::string &name,
                                   std::span<std::byte> bytes) {
  { a.read(name, bytes) } -> std::same_as<void>;
};

template <typename A>
concept ArchiveType = WritableArchive<A> && ReadableArchive<A>;
