// Batch loader over a token span (see model_utils/Dataset.h for the
// dataset). Same interface and behaviour as the reference's
// (include/model_utils/loader.h, src/model_utils/loader.cpp:5-43): each
// sample start is drawn uniformly from [0, size - len] with
// std::uniform_int_distribution<size_t> over std::mt19937(seed) -- the
// same standard-library engine and distribution, so one seed gives the
// reference's batches on the same C++ standard library.
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <span>
#include <vector>

class Loader {
public:
  struct Batch {
    std::vector<uint32_t> inputs;  // [batch, sequence], row-major
    std::vector<uint32_t> targets; // inputs shifted by one position
  };

private:
  std::span<const uint32_t> dataset_;
  std::mt19937 generator_;
  Batch batch_;

public:
  // Throws std::invalid_argument for an empty dataset.
  explicit Loader(std::span<const uint32_t> dataset, uint32_t seed = 1);

  // `len` consecutive tokens from a uniformly drawn start; throws
  // std::invalid_argument if len is 0 or longer than the dataset.
  std::span<const uint32_t> get_sample(size_t len);
  // batch_size samples of sequence_size + 1 tokens; valid until the next call.
  const Batch &get_batch(size_t batch_size, size_t sequence_size);
};
