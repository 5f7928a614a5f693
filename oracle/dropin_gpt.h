// dropin_gpt.h -- shared declarations of the drop-in test program (see
// dropin_gpt.cpp). TEST INFRASTRUCTURE ONLY.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace hip {
class Runtime;
}
namespace orc {
class Runtime;
}

namespace dropin {

// Small instance of the reference GPT: the executor's op sequence does not
// depend on the sizes, only the shapes do.
constexpr uint32_t kVocab = 96, kSeq = 24, kDim = 64, kHeads = 2, kBatch = 3;
constexpr uint32_t kFfn = 4 * kDim, kLayers = 4;
constexpr float kLr = 3e-4f, kBeta1 = 0.9f, kBeta2 = 0.95f, kEps = 1e-8f, kWd = 0.1f;
constexpr int kSteps = 2;

using Tensors = std::vector<std::vector<float>>;

using Blobs = std::map<std::string, std::vector<std::byte>>; // archive name -> bytes

struct Outcome {
  Tensors params0;                        // parameters after prepare()
  std::vector<std::vector<float>> losses; // per step: per-row losses
  std::vector<Tensors> grads, params;     // per step: gradients, updated params
  Blobs archive; // Compiled::save + save_optimisers after the last step
};

// src/train.cpp's loop body for kSteps steps of the reference nn::GPT on
// the given runtime, from std::mt19937(seed).
Outcome train_hip(hip::Runtime &rt, const std::vector<uint32_t> &tokens,
                  const std::vector<uint32_t> &targets, uint32_t seed, float max_norm);
Outcome train_oracle(orc::Runtime &rt, const std::vector<uint32_t> &tokens,
                     const std::vector<uint32_t> &targets, uint32_t seed, float max_norm);

} // namespace dropin
