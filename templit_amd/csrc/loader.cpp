// Batch loader (model_utils/loader.h); the reference's draws
// (src/model_utils/loader.cpp:5-43).
#include "model_utils/loader.h"

#include <stdexcept>

Loader::Loader(std::span<const uint32_t> dataset, uint32_t seed)
    : tokens_(dataset), engine_(seed) {
  if (tokens_.empty()) throw std::invalid_argument("a loader needs a non-empty dataset");
}

// Start of a `len`-token window, uniform over every window that fits.
size_t Loader::draw_start(size_t len) {
  if (len == 0 || len > tokens_.size())
    throw std::invalid_argument("sample length must lie in [1, dataset size]");
  return std::uniform_int_distribution<size_t>(0, tokens_.size() - len)(engine_);
}

std::span<const uint32_t> Loader::get_sample(size_t len) {
  return tokens_.subspan(draw_start(len), len);
}

const Loader::Batch &Loader::get_batch(size_t batch_size, size_t sequence_size) {
  if (batch_size == 0 || sequence_size == 0)
    throw std::invalid_argument("batch and sequence sizes must be non-zero");
  out_.inputs.resize(batch_size * sequence_size);
  out_.targets.resize(batch_size * sequence_size);
  uint32_t *x = out_.inputs.data(), *y = out_.targets.data();
  for (size_t b = 0; b < batch_size; ++b, x += sequence_size, y += sequence_size) {
    const uint32_t *window = tokens_.data() + draw_start(sequence_size + 1);
    for (size_t t = 0; t < sequence_size; ++t) {
      x[t] = window[t];
      y[t] = window[t + 1];
    }
  }
  return out_;
}
