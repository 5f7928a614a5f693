// train_oracle_bench: the reference executor on the CPU oracle runtime at the
// benchmark model's sizes (BenchDims). TEST INFRASTRUCTURE.
#include "dropin_train.h"

#include "oracle_runtime.h"

namespace dropin {
Outcome train_oracle_bench(orc::Runtime &rt, const std::vector<uint32_t> &tokens,
                           const std::vector<uint32_t> &targets, uint32_t seed, float max_norm) {
  return train<RTensor<orc::Host, float>, BenchDims>(rt, tokens, targets, seed, max_norm);
}
} // namespace dropin
