// The fixed checks of the dataset / loader tests, run against any
// Dataset / Loader pair with the reference's interface; prints one line
// per result. Shared by oracle/loader_tool.cpp (the reference's classes)
// and tests/cpp/test_loader.cpp (templit_amd's). TEST INFRASTRUCTURE ONLY.
#pragma once

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <span>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace loader_test_content {

inline unsigned long long fnv(std::span<const uint32_t> v) {
  uint64_t h = 1469598103934665603ull;
  for (uint32_t x : v) h = (h ^ x) * 1099511628211ull;
  return static_cast<unsigned long long>(h);
}

template <typename F> void expect_throw(const char *what, F &&f) {
  try {
    f();
    std::printf("%s: no exception\n", what);
  } catch (const std::invalid_argument &) {
    std::printf("%s: invalid_argument\n", what);
  } catch (const std::runtime_error &) {
    std::printf("%s: runtime_error\n", what);
  }
}

template <typename DatasetT, typename LoaderT>
void describe(const DatasetT &d, const char *name) {
  std::printf("%s: %zu tokens, fnv %016llx, train %zu, validation %zu\n", name, d.get().size(),
              fnv(d.get()), d.training_split().size(), d.validation_split().size());
  for (uint32_t seed : {1u, 2u, 12345u}) {
    LoaderT loader(d.training_split(), seed);
    for (int i = 0; i < 3; ++i) {
      const auto &b = loader.get_batch(4, 16);
      std::printf("%s seed %u batch %d: inputs %016llx targets %016llx first %u %u %u\n", name,
                  seed, i, fnv(b.inputs), fnv(b.targets), b.inputs[0], b.inputs[1],
                  b.targets[0]);
    }
    const auto s = loader.get_sample(d.training_split().size()); // the whole split
    std::printf("%s seed %u whole-split sample %016llx\n", name, seed, fnv(s));
  }
}

template <typename DatasetT, typename LoaderT>
int run(const char *tokens_path, const char *text_path) {
  {
    std::ifstream in(tokens_path, std::ios::binary);
    describe<DatasetT, LoaderT>(DatasetT::load_tokens(in), "tokens 0.95");
  }
  {
    std::ifstream in(tokens_path, std::ios::binary);
    describe<DatasetT, LoaderT>(DatasetT::load_tokens(in, 0.5), "tokens 0.5");
  }
  {
    std::ifstream in(text_path, std::ios::binary);
    describe<DatasetT, LoaderT>(DatasetT::load_text(in, 0.8), "text 0.8");
  }
  {
    std::ifstream in(tokens_path, std::ios::binary);
    const DatasetT d = DatasetT::load_tokens(in);
    std::ostringstream out;
    d.save(out);
    std::istringstream back(out.str());
    std::printf("save/load: %s\n",
                fnv(DatasetT::load_tokens(back).get()) == fnv(d.get()) ? "same" : "differs");
  }
  const std::vector<uint32_t> two = {1, 256};
  expect_throw("fraction 1.0", [&] { DatasetT d(two, 1.0); });
  expect_throw("fraction 0.0", [&] { DatasetT d(two, 0.0); });
  expect_throw("one token", [&] { DatasetT d(std::span<const uint32_t>(two).first(1)); });
  expect_throw("split leaves validation empty",
               [&] { DatasetT d(std::vector<uint32_t>{1, 2, 256}, 0.9); });
  expect_throw("odd byte count", [&] {
    std::istringstream in(std::string("abcde"));
    DatasetT::load_tokens(in);
  });
  expect_throw("empty loader", [&] { LoaderT l{std::span<const uint32_t>()}; });
  expect_throw("sample longer than the data", [&] {
    LoaderT l{std::span<const uint32_t>(two)};
    l.get_sample(3);
  });
  expect_throw("zero batch", [&] {
    LoaderT l{std::span<const uint32_t>(two)};
    l.get_batch(0, 1);
  });
  return 0;
}

} // namespace loader_test_content
