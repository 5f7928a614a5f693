// dropin_train.h -- src/train.cpp's loop body over the reference executor,
// templated on the tensor type and runtime (instantiated once per runtime
// in dropin_train_hip.cpp and dropin_train_orc.cpp). TEST INFRASTRUCTURE
// ONLY; the reference headers come from the reference tree.
#pragma once

#include "dropin_gpt.h"

#include "expr/cross-entropy.h"
#include "nn/GPT.h"
#include "optimiser/AdamW.h"
#include "passes/compile.h"

#include <cstring>
#include <map>
#include <random>
#include <span>
#include <string>
#include <vector>

namespace dropin {

// Name -> bytes archive with scoped names, enough for Compiled::save.
struct Archive {
  std::map<std::string, std::vector<std::byte>> *blobs;
  std::string prefix;
  void write(const std::string &name, std::span<const std::byte> v) {
    (*blobs)[prefix + name].assign(v.begin(), v.end());
  }
  void read(const std::string &name, std::span<std::byte> v) const {
    const auto &b = blobs->at(prefix + name);
    if (b.size() != v.size()) throw std::runtime_error("archive size mismatch");
    std::memcpy(v.data(), b.data(), b.size());
  }
  Archive scope(const std::string &name) const { return {blobs, prefix + name + "/"}; }
};

inline Tensors parameters_of(std::map<std::string, std::vector<std::byte>> &blobs) {
  Tensors out;
  for (size_t i = 0;; ++i) {
    auto it = blobs.find("parameters/" + std::to_string(i) + "/data");
    if (it == blobs.end()) break;
    std::vector<float> v(it->second.size() / sizeof(float));
    std::memcpy(v.data(), it->second.data(), it->second.size());
    out.push_back(std::move(v));
  }
  return out;
}

// The optimiser the executor sees: records each gradient it is handed
// (after clipping, in the executor's parameter order) and applies AdamW.
inline Tensors *g_sink = nullptr;
template <typename T> class RecordingAdamW {
public:
  using Shared = typename Optimiser::AdamW<T>::Shared;
  template <typename Run>
  void update(Run &rt, const Shared &s, const T &p, const T &g, T &dst) {
    std::vector<float> h(g.numel());
    g.read(std::span<float>(h));
    g_sink->push_back(std::move(h));
    inner_.update(rt, s, p, g, dst);
  }
  void initialise_for(const T &parameter) { inner_.initialise_for(parameter); }
  template <typename Arch> void save(Arch &archive) const { inner_.save(archive); }
  template <typename Arch> void load(Arch &archive) { inner_.load(archive); }

private:
  Optimiser::AdamW<T> inner_;
};

template <typename Mat, typename Dims, typename Run>
Outcome train(Run &rt, const std::vector<uint32_t> &tokens, const std::vector<uint32_t> &targets,
              uint32_t seed, float max_norm) {
  using IndexMat = typename Mat::template rebind<uint32_t>;
  constexpr uint32_t kBatch = Dims::batch, kSeq = Dims::seq;
  IndexMat in_v({kBatch, kSeq}), tg_v({kBatch, kSeq});
  in_v.set(std::span<const uint32_t>(tokens));
  tg_v.set(std::span<const uint32_t>(targets));
  expr::tensor::Tensor input(std::move(in_v));
  expr::tensor::Tensor target(std::move(tg_v));
  std::mt19937 gen(seed);
  nn::GPT<Mat, Dims::vocab, Dims::seq, Dims::dim, Dims::heads> model(kBatch, kSeq, gen);
  auto graph = model(input);
  auto loss = expr::loss::cross_entropy(graph, target);
  using Opt = RecordingAdamW<Mat>;
  auto compiled = passes::compile<Mat, Opt>(loss, rt,
                                            typename Opt::Shared(kLr, kBeta1, kBeta2, kEps, kWd));
  compiled.prepare();
  Outcome out;
  std::map<std::string, std::vector<std::byte>> blobs;
  Archive archive{&blobs, ""};
  compiled.save(archive);
  out.params0 = parameters_of(blobs);
  Mat root({kBatch, kSeq, 1});
  root.set(std::vector<float>(kBatch * kSeq, 1.0f / float(kBatch * kSeq)));
  for (int s = 0; s < kSteps; ++s) {
    compiled.zero_grad();
    Mat l = compiled.forward();
    std::vector<float> lv(l.numel());
    l.read(std::span<float>(lv));
    out.losses.push_back(lv);
    compiled.backward(root);
    out.grads.emplace_back();
    g_sink = &out.grads.back();
    compiled.step(max_norm);
    g_sink = nullptr;
    blobs.clear();
    compiled.save(archive);
    out.params.push_back(parameters_of(blobs));
  }
  compiled.save_optimisers(archive);
  out.archive = blobs;
  return out;
}

} // namespace dropin
