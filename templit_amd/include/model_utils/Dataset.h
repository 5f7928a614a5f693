// Token dataset for training runs (the batch loader is model_utils/loader.h).
//
// A drop-in for the reference's Dataset (include/model_utils/Dataset.h,
// behaviour of src/model_utils/dataset.cpp:16-102): the same public
// interface, file formats and split rule, so a training driver switches by
// include path.
//  * A .tokens file is raw native-order uint32 token ids.
//  * A text file maps each byte to the id of its value (0..255) and each
//    pair of consecutive newlines to the end-of-sequence id 256.
//  * The validation split starts one past the first end-of-sequence id at or
//    after floor(n * training_fraction), or at that index when none follows.
//
// Both loaders decode the stream in fixed-size chunks straight into the
// token buffer that the dataset then owns (no whole-file byte copy), so a
// multi-GB token file costs its own size in host memory once.
#pragma once

#include <cstddef>
#include <cstdint>
#include <iosfwd>
#include <span>
#include <vector>

class Dataset {
public:
  static constexpr uint32_t kEndOfSequence = 256;

  // Copies `tokens`. Throws std::invalid_argument for a fraction outside
  // (0, 1), fewer than two tokens, or a split that leaves one side empty.
  explicit Dataset(std::span<const uint32_t> tokens, double training_fraction = 0.95);

  // Throw std::runtime_error for a stream that cannot be read (or, for
  // tokens, a byte count that is not a multiple of 4), then validate as the
  // constructor does.
  static Dataset load_text(std::istream &input, double training_fraction = 0.95);
  static Dataset load_tokens(std::istream &input, double training_fraction = 0.95);

  // Writes the token ids in the .tokens format; std::runtime_error on failure.
  void save(std::ostream &output) const;

  std::span<const uint32_t> training_split() const { return all().first(validation_start_); }
  std::span<const uint32_t> validation_split() const { return all().subspan(validation_start_); }
  std::span<const uint32_t> get() const { return all(); }

private:
  // Takes the decoded buffer over without copying it (the tag keeps a
  // caller's braced or temporary vector on the public span constructor).
  struct Adopt {};
  Dataset(Adopt, std::vector<uint32_t> &&ids, double training_fraction);

  std::span<const uint32_t> all() const { return {ids_.data(), ids_.size()}; }

  std::vector<uint32_t> ids_;
  size_t validation_start_ = 0;
};
