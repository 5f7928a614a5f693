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

// Model sizes of the reference GPT (4 decoder blocks) the program trains.
// The executor's op sequence does not depend on the sizes, only the shapes
// do: SmallDims keeps the oracle anchor fast; BenchDims is the GPT example's
// benchmark model (V 2048, T 192, d 384, 6 heads) at batch 2, where the
// products take the tile plans, split-K and tail splits of batch 32.
struct SmallDims {
  static constexpr uint32_t vocab = 96, seq = 24, dim = 64, heads = 2, batch = 3;
};
struct BenchDims {
  static constexpr uint32_t vocab = 2048, seq = 192, dim = 384, heads = 6, batch = 2;
};
constexpr uint32_t kVocab = SmallDims::vocab, kSeq = SmallDims::seq, kDim = SmallDims::dim,
                   kHeads = SmallDims::heads, kBatch = SmallDims::batch;
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
// the given runtime, from std::mt19937(seed): SmallDims, and (the _bench
// forms, each in its own translation unit) BenchDims.
Outcome train_hip(hip::Runtime &rt, const std::vector<uint32_t> &tokens,
                  const std::vector<uint32_t> &targets, uint32_t seed, float max_norm);
Outcome train_oracle(orc::Runtime &rt, const std::vector<uint32_t> &tokens,
                     const std::vector<uint32_t> &targets, uint32_t seed, float max_norm);
Outcome train_hip_bench(hip::Runtime &rt, const std::vector<uint32_t> &tokens,
                        const std::vector<uint32_t> &targets, uint32_t seed, float max_norm);
Outcome train_oracle_bench(orc::Runtime &rt, const std::vector<uint32_t> &tokens,
                           const std::vector<uint32_t> &targets, uint32_t seed, float max_norm);

} // namespace dropin
