// Token dataset (model_utils/Dataset.h). The formats and the split rule are
// the reference's (src/model_utils/dataset.cpp:16-102); the decoding here is
// a chunked stream decoder that writes ids straight into the dataset's own
// buffer.
#include "model_utils/Dataset.h"

#include <array>
#include <cstring>
#include <istream>
#include <ostream>
#include <stdexcept>
#include <string>
#include <utility>

namespace {

// Feeds `input` to `sink(bytes, count)` in 64 KiB chunks until end of file.
// A stream that is already failed, or that reports a read error, throws.
template <typename Sink> void for_each_chunk(std::istream &input, const char *what, Sink &&sink) {
  if (!input) throw std::runtime_error(std::string("cannot read the ") + what);
  std::array<char, 64 * 1024> chunk;
  while (input) {
    input.read(chunk.data(), std::streamsize(chunk.size()));
    const std::streamsize got = input.gcount();
    if (got > 0) sink(reinterpret_cast<const unsigned char *>(chunk.data()), size_t(got));
  }
  if (input.bad()) throw std::runtime_error(std::string("read error in the ") + what);
}

// Text format: byte b is id b, except that two consecutive newlines are one
// end-of-sequence id. A newline is held back until the next byte shows
// whether it starts such a pair (also across chunk boundaries), so "\n\n\n"
// decodes to end-of-sequence then 10.
class TextDecoder {
public:
  explicit TextDecoder(std::vector<uint32_t> &ids) : ids_(ids) {}

  void feed(const unsigned char *bytes, size_t count) {
    for (size_t i = 0; i < count; ++i) {
      const unsigned char c = bytes[i];
      if (newline_held_) {
        newline_held_ = false;
        if (c == '\n') {
          ids_.push_back(Dataset::kEndOfSequence);
          continue;
        }
        ids_.push_back('\n');
      }
      if (c == '\n')
        newline_held_ = true;
      else
        ids_.push_back(c);
    }
  }

  void finish() {
    if (newline_held_) ids_.push_back('\n');
    newline_held_ = false;
  }

private:
  std::vector<uint32_t> &ids_;
  bool newline_held_ = false;
};

// .tokens format: native-order uint32 words. Whole words of a chunk are
// copied in one block; a word split across chunks is assembled in `partial_`.
class WordDecoder {
public:
  explicit WordDecoder(std::vector<uint32_t> &ids) : ids_(ids) {}

  void feed(const unsigned char *bytes, size_t count) {
    while (count > 0 && held_ > 0) { // complete the word begun in the last chunk
      partial_[held_++] = *bytes++;
      --count;
      if (held_ == sizeof(uint32_t)) push_partial();
    }
    const size_t words = count / sizeof(uint32_t);
    if (words > 0) {
      const size_t at = ids_.size();
      ids_.resize(at + words);
      std::memcpy(ids_.data() + at, bytes, words * sizeof(uint32_t));
    }
    for (size_t i = words * sizeof(uint32_t); i < count; ++i) partial_[held_++] = bytes[i];
  }

  void finish() const {
    if (held_ != 0) throw std::runtime_error("a token file holds whole uint32 ids");
  }

private:
  void push_partial() {
    uint32_t word;
    std::memcpy(&word, partial_.data(), sizeof(word));
    ids_.push_back(word);
    held_ = 0;
  }

  std::vector<uint32_t> &ids_;
  std::array<unsigned char, sizeof(uint32_t)> partial_{};
  size_t held_ = 0;
};

// One past the first end-of-sequence id at or after floor(n * fraction); the
// floor itself when no end-of-sequence id follows it.
size_t validation_start(const std::vector<uint32_t> &ids, double fraction) {
  const size_t floor_index = size_t(double(ids.size()) * fraction);
  for (size_t i = floor_index; i < ids.size(); ++i)
    if (ids[i] == Dataset::kEndOfSequence) return i + 1;
  return floor_index;
}

} // namespace

Dataset::Dataset(Adopt, std::vector<uint32_t> &&ids, double training_fraction)
    : ids_(std::move(ids)) {
  if (!(training_fraction > 0.0 && training_fraction < 1.0))
    throw std::invalid_argument("training fraction must lie strictly between 0 and 1");
  if (ids_.size() < 2) throw std::invalid_argument("a dataset needs two tokens or more");
  validation_start_ = validation_start(ids_, training_fraction);
  if (validation_start_ == 0 || validation_start_ >= ids_.size())
    throw std::invalid_argument("the training split would leave a partition empty");
}

Dataset::Dataset(std::span<const uint32_t> tokens, double training_fraction)
    : Dataset(Adopt{}, std::vector<uint32_t>(tokens.begin(), tokens.end()), training_fraction) {}

Dataset Dataset::load_text(std::istream &input, double training_fraction) {
  std::vector<uint32_t> ids;
  TextDecoder decoder(ids);
  for_each_chunk(input, "text dataset",
                 [&](const unsigned char *b, size_t n) { decoder.feed(b, n); });
  decoder.finish();
  return Dataset(Adopt{}, std::move(ids), training_fraction);
}

Dataset Dataset::load_tokens(std::istream &input, double training_fraction) {
  std::vector<uint32_t> ids;
  WordDecoder decoder(ids);
  for_each_chunk(input, "token dataset",
                 [&](const unsigned char *b, size_t n) { decoder.feed(b, n); });
  decoder.finish();
  return Dataset(Adopt{}, std::move(ids), training_fraction);
}

void Dataset::save(std::ostream &output) const {
  output.write(reinterpret_cast<const char *>(ids_.data()),
               std::streamsize(ids_.size() * sizeof(uint32_t)));
  if (!output) throw std::runtime_error("cannot write the token dataset");
}
