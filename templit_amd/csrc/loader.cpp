// Batch loader (see model_utils/loader.h).
// Reference behaviour: src/model_utils/loader.cpp:5-43.
#include "model_utils/loader.h"

#include <algorithm>
#include <stdexcept>

Loader::Loader(std::span<const uint32_t> dataset, uint32_t seed)
    : dataset_(dataset), generator_(seed) {
  if (dataset_.empty()) throw std::invalid_argument("a loader needs a non-empty dataset");
}

std::span<const uint32_t> Loader::get_sample(size_t len) {
  if (len == 0 || len > dataset_.size())
    throw std::invalid_argument("sample length must lie in [1, dataset size]");
  std::uniform_int_distribution<size_t> start(0, dataset_.size() - len);
  return dataset_.subspan(start(generator_), len);
}

const Loader::Batch &Loader::get_batch(size_t batch_size, size_t sequence_size) {
  if (batch_size == 0 || sequence_size == 0)
    throw std::invalid_argument("batch and sequence sizes must be non-zero");
  batch_.inputs.resize(batch_size * sequence_size);
  batch_.targets.resize(batch_size * sequence_size);
  for (size_t b = 0; b < batch_size; ++b) {
    const auto sample = get_sample(sequence_size + 1);
    std::copy(sample.begin(), sample.end() - 1, batch_.inputs.begin() + b * sequence_size);
    std::copy(sample.begin() + 1, sample.end(), batch_.targets.begin() + b * sequence_size);
  }
  return batch_;
}
