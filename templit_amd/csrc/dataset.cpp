// Token dataset (see model_utils/Dataset.h).
// Reference behaviour: src/model_utils/dataset.cpp:16-102.
#include "model_utils/Dataset.h"

#include <algorithm>
#include <cstring>
#include <istream>
#include <iterator>
#include <ostream>
#include <stdexcept>
#include <string>

Dataset::Dataset(std::span<const uint32_t> tokens, double training_fraction)
    : data_(tokens.begin(), tokens.end()) {
  if (!(training_fraction > 0.0 && training_fraction < 1.0))
    throw std::invalid_argument("training fraction must lie strictly between 0 and 1");
  if (data_.size() < 2) throw std::invalid_argument("a dataset needs two tokens or more");
  const size_t target = static_cast<size_t>(static_cast<double>(data_.size()) * training_fraction);
  const auto eos = std::find(data_.begin() + std::ptrdiff_t(target), data_.end(), kEndOfSequence);
  split_index_ = eos == data_.end() ? target : size_t(eos - data_.begin()) + 1;
  if (split_index_ == 0 || split_index_ >= data_.size())
    throw std::invalid_argument("the training split would leave a partition empty");
}

Dataset Dataset::load_text(std::istream &input, double training_fraction) {
  if (!input) throw std::runtime_error("cannot read the text dataset");
  const std::string bytes{std::istreambuf_iterator<char>(input), std::istreambuf_iterator<char>()};
  std::vector<uint32_t> tokens;
  tokens.reserve(bytes.size());
  for (size_t i = 0; i < bytes.size(); ++i) {
    if (bytes[i] == '\n' && i + 1 < bytes.size() && bytes[i + 1] == '\n') {
      tokens.push_back(kEndOfSequence); // a blank line ends a sequence
      ++i;
    } else {
      tokens.push_back(static_cast<unsigned char>(bytes[i]));
    }
  }
  return Dataset(tokens, training_fraction);
}

Dataset Dataset::load_tokens(std::istream &input, double training_fraction) {
  if (!input) throw std::runtime_error("cannot read the token dataset");
  const std::vector<char> bytes{std::istreambuf_iterator<char>(input),
                                std::istreambuf_iterator<char>()};
  if (bytes.size() % sizeof(uint32_t) != 0)
    throw std::runtime_error("a token file holds whole uint32 ids");
  std::vector<uint32_t> tokens(bytes.size() / sizeof(uint32_t));
  if (!bytes.empty()) std::memcpy(tokens.data(), bytes.data(), bytes.size());
  return Dataset(tokens, training_fraction);
}

void Dataset::save(std::ostream &output) const {
  output.write(reinterpret_cast<const char *>(data_.data()),
               std::streamsize(data_.size() * sizeof(uint32_t)));
  if (!output) throw std::runtime_error("cannot write the token dataset");
}

std::span<const uint32_t> Dataset::training_split() const {
  return std::span<const uint32_t>(data_).first(split_index_);
}

std::span<const uint32_t> Dataset::validation_split() const {
  return std::span<const uint32_t>(data_).subspan(split_index_);
}

std::span<const uint32_t> Dataset::get() const { return std::span<const uint32_t>(data_); }
