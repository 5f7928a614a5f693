// Host half of the fused AdamW optimiser: per-parameter state and the call
// into the runtime's adamW op.
//
// Interface of Optimiser::AdamW (reference include/optimiser/AdamW.h:11-107),
// the optimiser passes::Compiled::step() drives through exec::step
// (include/passes/execute.h:492-503):
//   - Shared: learning rate, beta1, beta2 and decay = 1 - lr * weight_decay
//     as 1-element device tensors (so a recorded step reads the current
//     values), epsilon and weight decay on the host; set_lr rewrites lr and
//     decay;
//   - per parameter: moments m, v (zero-filled on first use), a step counter
//     incremented before every update (the update of step t uses t >= 1);
//   - save/load of the moments and the step under "momentum1",
//     "momentum2", "step".
#pragma once

#include "model_utils/archive_concepts.h"

#include <cstdint>
#include <span>
#include <stdexcept>

namespace Optimiser {

template <typename T> class AdamW {
  using value_type = typename T::value_type;

public:
  class Shared {
  public:
    Shared(value_type learning_rate, value_type beta1 = 0.9f, value_type beta2 = 0.999f,
           value_type epsilon = 1e-8f, value_type weight_decay = 0.01f)
        : learning_rate_(learning_rate), beta1_(beta1), beta2_(beta2),
          decay_(value_type{1} - learning_rate * weight_decay), epsilon_(epsilon),
          weight_decay_(weight_decay) {}

    void set_lr(value_type lr) {
      learning_rate_.set(lr, 0);
      decay_.set(value_type{1} - lr * weight_decay_, 0);
    }
    value_type get_lr() { return learning_rate_.get(0); }

  private:
    friend class AdamW;
    T learning_rate_, beta1_, beta2_, decay_;
    value_type epsilon_, weight_decay_;
  };

  static Shared generate_params(value_type learning_rate, value_type beta1 = 0.9f,
                                value_type beta2 = 0.999f, value_type epsilon = 1e-8f,
                                value_type weight_decay = 0.01f) {
    return Shared(learning_rate, beta1, beta2, epsilon, weight_decay);
  }

  void initialise_for(const T &parameter) {
    if (initialised_) {
      if (m1_.shape() != parameter.shape())
        throw std::invalid_argument("AdamW parameter shape changed");
      return;
    }
    m1_ = T::from_zeros(parameter.shape());
    m2_ = T::from_zeros(parameter.shape());
    initialised_ = true;
  }

  template <typename Run>
  void update(Run &runtime, const Shared &s, const T &parameter, const T &gradient,
              T &destination) {
    initialise_for(parameter);
    ++step_;
    runtime.adamW(parameter, gradient, destination, m1_, m2_, s.beta1_, s.beta2_, s.decay_,
                  s.learning_rate_, s.epsilon_, step_);
  }

  uint32_t step() const { return step_; }
  const T &momentum1() const { return m1_; }
  const T &momentum2() const { return m2_; }

  template <WritableArchive Arch> void save(Arch &archive) const {
    if (!initialised_) throw std::logic_error("cannot save uninitialised AdamW state");
    auto a1 = archive.scope("momentum1");
    auto a2 = archive.scope("momentum2");
    m1_.save(a1);
    m2_.save(a2);
    archive.write("step", std::as_bytes(std::span(&step_, 1)));
  }

  template <ReadableArchive Arch> void load(Arch &archive) {
    if (!initialised_) throw std::logic_error("AdamW must be initialised before loading state");
    auto a1 = archive.scope("momentum1");
    auto a2 = archive.scope("momentum2");
    m1_.load(a1);
    m2_.load(a2);
    archive.read("step", std::as_writable_bytes(std::span(&step_, 1)));
  }

private:
  uint32_t step_ = 0;
  T m1_, m2_;
  bool initialised_ = false;
};

} // namespace Optimiser
