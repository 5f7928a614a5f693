// train_hip: the reference executor on hip::Runtime. TEST INFRASTRUCTURE.
#include "dropin_train.h"

#include "my_hip/runtime.h"
#include "my_hip/storage.h"

namespace dropin {
Outcome train_hip(hip::Runtime &rt, const std::vector<uint32_t> &tokens,
                  const std::vector<uint32_t> &targets, uint32_t seed, float max_norm) {
  return train<RTensor<hip::HIP, float>, SmallDims>(rt, tokens, targets, seed, max_norm);
}
} // namespace dropin
