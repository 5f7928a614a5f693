// Drives the reference's own inference::sample_top_k (include/inference.h:
// 14-43, compiled from the reference tree where it lies) for
// tests/test_oracle_sampler.py. TEST INFRASTRUCTURE ONLY (built into
// oracle/_ref/, never shipped).
//
//   ref_sampler_tool V TOP_K TEMPERATURE SEED DRAWS < logits.txt
//
// reads V logits (one per line, C99 hex floats), then calls sample_top_k
// DRAWS times on one std::mt19937(SEED), printing per call the token and the
// uniform that call's std::discrete_distribution drew: generate_canonical<
// double, 53> over a copy of the engine taken before the call (one draw
// consumes two 32-bit outputs, as the discrete_distribution call does).
#include <inference.h>

#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

namespace {
// The one-row [1, 1, V] logits view sample_top_k reads (shape().back(),
// get(0, position, token)).
struct Row {
  std::vector<uint32_t> dims;
  const std::vector<float> *values;
  const std::vector<uint32_t> &shape() const { return dims; }
  float get(uint32_t, uint32_t, uint32_t token) const { return (*values)[token]; }
};
} // namespace

int main(int argc, char **argv) {
  if (argc != 6) {
    std::fprintf(stderr, "usage: %s V TOP_K TEMPERATURE SEED DRAWS < logits\n", argv[0]);
    return 2;
  }
  const uint32_t vocab = uint32_t(std::strtoul(argv[1], nullptr, 10));
  const uint32_t top_k = uint32_t(std::strtoul(argv[2], nullptr, 10));
  const float temperature = std::strtof(argv[3], nullptr);
  const uint32_t seed = uint32_t(std::strtoul(argv[4], nullptr, 10));
  const uint32_t draws = uint32_t(std::strtoul(argv[5], nullptr, 10));
  std::vector<float> logits(vocab);
  for (uint32_t i = 0; i < vocab; ++i) {
    char buf[64];
    if (std::scanf("%63s", buf) != 1) return 3;
    logits[i] = std::strtof(buf, nullptr);
  }
  const Row row{{1, 1, vocab}, &logits};
  std::mt19937 rng(seed);
  for (uint32_t d = 0; d < draws; ++d) {
    std::mt19937 probe = rng;
    const double u = std::generate_canonical<double, 53>(probe);
    const uint32_t token = inference::sample_top_k(row, 0, top_k, temperature, rng);
    std::printf("%u %a\n", token, u);
  }
  return 0;
}
