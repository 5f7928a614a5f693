// train_hip_bench: the reference executor on hip::Runtime at the
// benchmark model's sizes (BenchDims). TEST INFRASTRUCTURE.
#include "dropin_train.h"

#include "my_hip/runtime.h"
#include "my_hip/storage.h"

namespace dropin {
Outcome train_hip_bench(hip::Runtime &rt, const std::vector<uint32_t> &tokens,
                        const std::vector<uint32_t> &targets, uint32_t seed, float max_norm) {
  return train<RTensor<hip::HIP, float>, BenchDims>(rt, tokens, targets, seed, max_norm);
}
} // namespace dropin
