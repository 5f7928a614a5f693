// train_oracle: the reference executor on the CPU oracle runtime. TEST
// INFRASTRUCTURE.
#include "dropin_train.h"

#include "oracle_runtime.h"

namespace dropin {
Outcome train_oracle(orc::Runtime &rt, const std::vector<uint32_t> &tokens,
                     const std::vector<uint32_t> &targets, uint32_t seed, float max_norm) {
  return train<RTensor<orc::Host, float>, SmallDims>(rt, tokens, targets, seed, max_norm);
}
} // namespace dropin
