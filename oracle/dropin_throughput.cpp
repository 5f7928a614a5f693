// dropin_throughput.cpp -- throughput of the reference executor on
// hip::Runtime at the GPT benchmark configuration.
//
// TEST INFRASTRUCTURE: built by oracle/Makefile (target `dropin-throughput`)
// from the reference's frontend headers where they lie (nn/GPT.h,
// passes/compile.h, optimiser/AdamW.h, expr/...) into oracle/_ref/, like
// dropin_gpt, with hip::Runtime compiled in unchanged. It measures what a
// user gets by switching src/train.cpp from metal::Runtime to hip::Runtime:
// nn::GPT<V 2048, T 192, d 384, 6 heads> (4 blocks) at batch 32, AdamW
// (lr 3e-4, betas 0.9/0.95, eps 1e-8, wd 0.1), and train.cpp's loop body
// (train.cpp:148-156): zero_grad, forward, read the per-row losses,
// backward(1/(B*T)), step(1.0). Every phase waits for its work (the runtime's
// start/submit/wait), so wall time per step is the device time plus what the
// host adds between phases.
//
// Usage: dropin_throughput [steps = 20] [modes = 2]  (modes 1: eager only;
// 2: eager, then graph mode). Prints ms per step and tokens/s per mode.
#include "expr/cross-entropy.h"
#include "nn/GPT.h"
#include "optimiser/AdamW.h"
#include "passes/compile.h"

#include "my_hip/runtime.h"
#include "my_hip/storage.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <random>
#include <span>
#include <vector>

namespace {

constexpr uint32_t kB = 32, kT = 192, kV = 2048, kD = 384, kH = 6;

int run(int steps, int modes) {
  hip::init(0);
  {
    hip::Runtime rt;
    using Mat = RTensor<hip::HIP, float>;
    using IndexMat = typename Mat::template rebind<uint32_t>;
    std::vector<uint32_t> tokens(kB * kT), targets(kB * kT);
    std::mt19937 draw(7);
    for (auto &t : tokens) t = draw() % kV;
    for (auto &t : targets) t = draw() % kV;
    IndexMat in_v({kB, kT}), tg_v({kB, kT});
    in_v.set(std::span<const uint32_t>(tokens));
    tg_v.set(std::span<const uint32_t>(targets));
    expr::tensor::Tensor input(std::move(in_v));
    expr::tensor::Tensor target(std::move(tg_v));
    std::mt19937 gen(1);
    nn::GPT<Mat, kV, kT, kD, kH> model(kB, kT, gen);
    auto graph = model(input);
    auto loss = expr::loss::cross_entropy(graph, target);
    using Opt = Optimiser::AdamW<Mat>;
    auto compiled = passes::compile<Mat, Opt>(
        loss, rt, typename Opt::Shared(3e-4f, 0.9f, 0.95f, 1e-8f, 0.1f));
    compiled.prepare();
    Mat root({kB, kT, 1});
    root.set(std::vector<float>(kB * kT, 1.0f / float(kB * kT)));
    std::vector<float> losses(kB * kT);
    auto step = [&] {
      compiled.zero_grad();
      const Mat l = compiled.forward();
      l.read(std::span<float>(losses));
      compiled.backward(root);
      compiled.step(1.0f);
    };
    for (int mode = 0; mode < modes; ++mode) {
      rt.set_graph_mode(mode == 1);
      for (int i = 0; i < 3; ++i) step();
      const auto t0 = std::chrono::steady_clock::now();
      for (int i = 0; i < steps; ++i) step();
      const double s =
          std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() / steps;
      double mean = 0;
      for (float v : losses) mean += v;
      mean /= double(losses.size());
      std::printf("%s: %.3f ms/step, %.0f tokens/s, mean loss %.4f\n",
                  mode ? "graph mode" : "eager", s * 1e3, kB * kT / s, mean);
      std::fflush(stdout);
    }
  }
  hip::shutdown();
  return 0;
}

} // namespace

int main(int argc, char **argv) {
  std::setvbuf(stdout, nullptr, _IOLBF, 0);
  try {
    return run(argc > 1 ? std::atoi(argv[1]) : 20, argc > 2 ? std::atoi(argv[2]) : 2);
  } catch (const std::exception &e) {
    std::printf("error: %s\n", e.what());
    return 2;
  }
}
