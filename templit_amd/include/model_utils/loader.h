// Batch loader over a token span (the dataset is model_utils/Dataset.h).
//
// A drop-in for the reference's Loader (include/model_utils/loader.h,
// behaviour of src/model_utils/loader.cpp:5-43). Sample starts are the
// reference's draws: std::uniform_int_distribution<size_t> over [0, size -
// len] from std::mt19937(seed), one draw per sample in batch order, so one
// seed gives the reference's batches on the same C++ standard library.
// get_batch fills one [batch, sequence] buffer of inputs and its one-token
// shift of targets, reused across calls (the form the GPT program uploads
// to the device in one copy each).
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

  // Throws std::invalid_argument for an empty dataset. `dataset` must
  // outlive the loader.
  explicit Loader(std::span<const uint32_t> dataset, uint32_t seed = 1);

  // `len` consecutive tokens from a uniformly drawn start; throws
  // std::invalid_argument if len is 0 or longer than the dataset.
  std::span<const uint32_t> get_sample(size_t len);
  // batch_size windows of sequence_size + 1 tokens, split into inputs and
  // targets; the reference stays valid until the next call.
  const Batch &get_batch(size_t batch_size, size_t sequence_size);

private:
  size_t draw_start(size_t len);

  std::span<const uint32_t> tokens_;
  std::mt19937 engine_;
  Batch out_;
};
