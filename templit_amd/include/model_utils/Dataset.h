// Token dataset for training (the batch loader is model_utils/loader.h).
// Same interface and behaviour as the reference's
// (include/model_utils/Dataset.h, src/model_utils/dataset.cpp:16-102), so
// a training driver switches by include path:
//  * a .tokens file is raw native-order uint32 token ids;
//  * a text file maps bytes to ids 0..255 and each blank line ("\n\n") to
//    the end-of-sequence id 256;
//  * the training split ends after the first end-of-sequence id at or past
//    training_fraction of the tokens (else exactly there).
#pragma once

#include <cstddef>
#include <cstdint>
#include <iosfwd>
#include <span>
#include <vector>

class Dataset {
  std::vector<uint32_t> data_;
  size_t split_index_ = 0;

public:
  static constexpr uint32_t kEndOfSequence = 256;

  // Throws std::invalid_argument for a fraction outside (0, 1), fewer than
  // two tokens, or a split that leaves one side empty.
  explicit Dataset(std::span<const uint32_t> tokens, double training_fraction = 0.95);

  // Throws std::runtime_error on a failed stream (or, for tokens, a byte
  // count that is not a multiple of 4).
  static Dataset load_text(std::istream &input, double training_fraction = 0.95);
  static Dataset load_tokens(std::istream &input, double training_fraction = 0.95);

  void save(std::ostream &output) const;

  std::span<const uint32_t> training_split() const;
  std::span<const uint32_t> validation_split() const;
  std::span<const uint32_t> get() const;
};
