// dropin_gpt.cpp -- the reference executor driving hip::Runtime.
//
// TEST INFRASTRUCTURE: built by oracle/Makefile (target `dropin`, with
// dropin_train_hip.cpp and dropin_train_orc.cpp) from the
// reference's own frontend headers where they lie (nn/GPT.h, passes/
// compile.h, optimiser/AdamW.h, expr/...), into oracle/_ref/. Nothing of
// the reference is copied; the product (hip::Runtime, the kernel library)
// is compiled unchanged into the same program, as a maintainer would when
// switching the GPT example from metal::Runtime to hip::Runtime.
//
// It runs src/train.cpp's loop body -- zero_grad, forward, backward(1/(B*T)),
// step(max_norm) with AdamW -- for two steps of the reference nn::GPT (4
// decoder blocks) through passes::Compiled on three runtimes:
//   1. hip::Runtime, eager;
//   2. hip::Runtime, graph mode (each phase recorded as a hipGraph);
//   3. orc::Runtime, the CPU oracle runtime (oracle_runtime.h);
// from the same std::mt19937 initialisation, and compares losses, the
// (clipped) gradients handed to the optimiser and the updated parameters.
// As an independent anchor it also runs the oracle's hand-derived GPT step
// (orc_gpt_train_step) on the same weights, identified by value.
//
// Exit status 0 when every comparison is within tolerance (1 otherwise, 2
// on an error). Prints one line per compared quantity. With --cpu-only it
// runs only the oracle runtime and the anchor (no GPU).
#include "dropin_gpt.h"

#include "my_hip/runtime.h"
#include "my_hip/storage.h"
#include "oracle_runtime.h"

#include <algorithm>
#include <string>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <span>
#include <string>
#include <vector>

namespace {

using namespace dropin;

// ---- comparisons ---------------------------------------------------------------

int g_failures = 0;

double rel_l2(const std::vector<float> &a, const std::vector<float> &b) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    num += (double(a[i]) - b[i]) * (double(a[i]) - b[i]);
    den += double(b[i]) * b[i];
  }
  return den > 0 ? std::sqrt(num / den) : std::sqrt(num);
}

void report(const std::string &what, double err, double tol) {
  const bool ok = err <= tol;
  std::printf("%-72s %.3e (tol %.0e) %s\n", what.c_str(), err, tol, ok ? "ok" : "FAILED");
  if (!ok) ++g_failures;
}

// Tensors whose gradient is zero in exact arithmetic hold only rounding
// noise on both sides: the key-projection biases (a per-row constant added
// to the attention scores cancels in the softmax). They are recognised by
// the reference side's gradient being tiny against the largest gradient,
// and are compared absolutely instead of relatively.
std::vector<bool> degenerate(const Tensors &g) {
  std::vector<double> rms(g.size());
  double top = 0;
  for (size_t t = 0; t < g.size(); ++t) {
    double s = 0;
    for (float x : g[t]) s += double(x) * x;
    rms[t] = std::sqrt(s / std::max<size_t>(1, g[t].size()));
    top = std::max(top, rms[t]);
  }
  std::vector<bool> out(g.size());
  for (size_t t = 0; t < g.size(); ++t) out[t] = rms[t] < 1e-5 * top;
  return out;
}

struct Worst {
  double err = 0;
  size_t tensor = 0;
};

Worst worst(const Tensors &a, const Tensors &b, const std::vector<bool> &skip) {
  Worst w;
  if (a.size() != b.size()) return {INFINITY, 0};
  for (size_t i = 0; i < a.size(); ++i) {
    if (skip[i]) continue;
    const double e = rel_l2(a[i], b[i]);
    if (e > w.err) w = {e, i};
  }
  return w;
}

void report(const std::string &what, const Worst &w, const Tensors &ref, double tol) {
  const std::string where = " [tensor " + std::to_string(w.tensor) + ", " +
                            std::to_string(ref.empty() ? 0 : ref[w.tensor].size()) + " values]";
  report((what + where).c_str(), w.err, tol);
}

// AdamW's update divides by sqrt(v): where a gradient element is at
// rounding-noise level its sign, and so its update, is arbitrary. Compare
// the update only where the gradient is significant for its tensor.
Worst worst_update(const Tensors &p0, const Tensors &pa, const Tensors &pb, const Tensors &g,
                   const std::vector<bool> &skip) {
  Worst w;
  for (size_t t = 0; t < p0.size(); ++t) {
    if (skip[t]) continue;
    double gmax = 0;
    for (float x : g[t]) gmax = std::max(gmax, double(std::fabs(x)));
    double num = 0, den = 0;
    for (size_t i = 0; i < p0[t].size(); ++i) {
      if (std::fabs(g[t][i]) < 1e-3 * gmax) continue;
      const double da = double(pa[t][i]) - p0[t][i], db = double(pb[t][i]) - p0[t][i];
      num += (da - db) * (da - db);
      den += db * db;
    }
    if (den > 0 && std::sqrt(num / den) > w.err) w = {std::sqrt(num / den), t};
  }
  return w;
}

// Largest |a - b| over the degenerate tensors, in units of the learning
// rate: AdamW moves a noise-driven parameter by at most ~lr per step.
double degenerate_drift(const Tensors &a, const Tensors &b, const std::vector<bool> &mask) {
  double d = 0;
  for (size_t t = 0; t < a.size(); ++t)
    if (mask[t])
      for (size_t i = 0; i < a[t].size(); ++i)
        d = std::max(d, std::fabs(double(a[t][i]) - b[t][i]) / kLr);
  return d;
}

// `with_grads` = false when the recorded gradients are not comparable: in
// graph mode the optimiser reads them while the step is being recorded,
// i.e. before the recorded clip has run.
void compare(const char *name, const Outcome &a, const Outcome &b, double loss_tol, double tol,
             bool with_grads = true) {
  std::printf("-- %s\n", name);
  const std::vector<bool> none(b.params0.size(), false);
  report("initial parameters (identical draw)", worst(a.params0, b.params0, none).err, 0.0);
  for (int s = 0; s < kSteps; ++s) {
    const std::string tag = "step " + std::to_string(s + 1) + ": ";
    const std::vector<bool> noise = degenerate(b.grads[s]);
    const size_t n_noise = size_t(std::count(noise.begin(), noise.end(), true));
    report(tag + "per-row losses, rel-L2", rel_l2(a.losses[s], b.losses[s]), loss_tol);
    if (with_grads) {
      report(tag + "gradients, worst tensor rel-L2", worst(a.grads[s], b.grads[s], noise),
             b.grads[s], tol);
      // the degenerate tensors must be noise on this side too
      std::vector<bool> other = degenerate(a.grads[s]);
      size_t agree = 0;
      for (size_t t = 0; t < noise.size(); ++t) agree += noise[t] && other[t];
      report(tag + "zero-gradient tensors (" + std::to_string(n_noise) + ") also ~0 here, missing",
             double(n_noise - agree), 0.0);
    }
    report(tag + "updated parameters, worst tensor rel-L2", worst(a.params[s], b.params[s], noise),
           b.params[s], tol);
    const Tensors &before_a = s ? a.params[s - 1] : a.params0;
    report(tag + "parameter updates (significant grads), rel-L2",
           worst_update(before_a, a.params[s], b.params[s], b.grads[s], noise), b.params[s], 1e-2);
    report(tag + "zero-gradient tensors: parameter drift / lr", 
           degenerate_drift(a.params[s], b.params[s], noise), 2.0 * (s + 1) + 0.01);
  }
}

// ---- independent anchor: the oracle's hand-derived GPT step ---------------------

// The weights the GPT constructor draws, in its member order (GPT.h:42-60,
// decoder_block.h:15-24, multi_head.h:19-30, layer.h:15-30, embedding.h:
// 19-34): each tensor draws from a fresh normal_distribution with Xavier
// scale sqrt(2 / (fan_in + fan_out)).
Tensors canonical_weights(uint32_t seed) {
  std::mt19937 gen(seed);
  Tensors w;
  const auto draw = [&](uint32_t rows, uint32_t cols) {
    std::normal_distribution<float> dis(0.0f, std::sqrt(2.0f / float(rows + cols)));
    std::vector<float> v(size_t(rows) * cols);
    for (auto &x : v) x = dis(gen);
    w.push_back(std::move(v));
  };
  draw(kVocab, kDim);
  draw(kSeq, kDim);
  for (uint32_t l = 0; l < kLayers; ++l) {
    for (int j = 0; j < 4; ++j) draw(kDim, kDim);
    draw(kDim, kFfn);
    draw(kFfn, kDim);
  }
  draw(kDim, kVocab);
  return w;
}

// Returns, for every executor parameter index, the canonical index of the
// same tensor (weights matched by value, biases by gradient), -1 if none.
std::vector<int> anchor(const Outcome &orc_rt, const std::vector<uint32_t> &tokens,
                        const std::vector<uint32_t> &targets, uint32_t seed, float max_norm) {
  std::vector<int> canonical_of(orc_rt.params0.size(), -1);
  std::printf("-- oracle runtime vs the oracle's hand-derived GPT step (weights matched by value)\n");
  const orc_gpt_config cfg{kVocab, kSeq, kDim, kHeads, kLayers, kBatch, kFfn};
  const uint32_t count = orc_gpt_param_count(&cfg);
  // canonical index of every weight tensor; biases are the others
  std::vector<int> weight_slot;
  weight_slot.push_back(0);
  weight_slot.push_back(1);
  for (uint32_t l = 0; l < kLayers; ++l)
    for (int j : {0, 2, 4, 6, 8, 10}) weight_slot.push_back(int(2 + 12 * l + j));
  weight_slot.push_back(int(2 + 12 * kLayers));
  const Tensors drawn = canonical_weights(seed);
  std::vector<int> ref_of(count, -1); // canonical index -> executor index
  std::vector<bool> used(orc_rt.params0.size(), false);
  for (size_t k = 0; k < drawn.size(); ++k)
    for (size_t i = 0; i < orc_rt.params0.size(); ++i)
      if (!used[i] && orc_rt.params0[i] == drawn[k]) {
        ref_of[weight_slot[k]] = int(i);
        used[i] = true;
        break;
      }
  int unmatched = 0;
  for (int s : weight_slot) unmatched += ref_of[s] < 0;
  report("weights identified by value (unmatched count)", unmatched, 0);
  if (unmatched) return canonical_of;
  for (uint32_t c = 0; c < count; ++c)
    if (ref_of[c] >= 0) canonical_of[ref_of[c]] = int(c);
  std::vector<float> params, m, v;
  for (uint32_t c = 0; c < count; ++c) {
    const size_t n = orc_gpt_param_size(&cfg, c);
    if (ref_of[c] >= 0) params.insert(params.end(), orc_rt.params0[ref_of[c]].begin(),
                                      orc_rt.params0[ref_of[c]].end());
    else params.insert(params.end(), n, 0.0f); // biases start at zero
  }
  m.assign(params.size(), 0.0f);
  v.assign(params.size(), 0.0f);
  std::vector<float> losses(kBatch * kSeq), grads(params.size());
  float sq = 0;
  orc_gpt_train_step(&cfg, params.data(), m.data(), v.data(), 1, tokens.data(), targets.data(),
                     1.0f / float(kBatch * kSeq), kLr, kBeta1, kBeta2, kEps, kWd, max_norm,
                     losses.data(), grads.data(), &sq);
  report("step 1: per-row losses, rel-L2", rel_l2(orc_rt.losses[0], losses), 1e-5);
  const float clip = std::min(1.0f, max_norm / std::sqrt(std::max(sq, 1e-12f)));
  // weights: by identity; biases: each executor bias gradient must match a
  // distinct canonical bias gradient of the same size
  double w_err = 0, b_err = 0;
  size_t off = 0;
  std::vector<std::pair<size_t, std::vector<float>>> bias_grads;
  std::vector<uint32_t> bias_slot;
  for (uint32_t c = 0; c < count; ++c) {
    const size_t n = orc_gpt_param_size(&cfg, c);
    std::vector<float> g(grads.begin() + off, grads.begin() + off + n);
    for (auto &x : g) x *= clip;
    if (ref_of[c] >= 0) w_err = std::max(w_err, rel_l2(orc_rt.grads[0][ref_of[c]], g));
    else {
      bias_grads.emplace_back(n, std::move(g));
      bias_slot.push_back(c);
    }
    off += n;
  }
  std::vector<bool> taken(bias_grads.size(), false);
  for (size_t i = 0; i < orc_rt.grads[0].size(); ++i) {
    if (used[i]) continue;
    double best = INFINITY;
    size_t best_j = 0;
    for (size_t j = 0; j < bias_grads.size(); ++j)
      if (!taken[j] && bias_grads[j].first == orc_rt.grads[0][i].size()) {
        const double e = rel_l2(orc_rt.grads[0][i], bias_grads[j].second);
        if (e < best) best = e, best_j = j;
      }
    if (best == INFINITY) {
      b_err = INFINITY;
      continue;
    }
    taken[best_j] = true;
    canonical_of[i] = int(bias_slot[best_j]);
    // the key-projection bias has an exactly-zero gradient in exact
    // arithmetic (softmax shift invariance): judge it absolutely
    double scale = 0;
    for (float x : bias_grads[best_j].second) scale = std::max(scale, double(std::fabs(x)));
    b_err = std::max(b_err, scale < 1e-7 ? 0.0 : best);
  }
  report("step 1: weight gradients, worst tensor rel-L2", w_err, 1e-4);
  report("step 1: bias gradients (matched by value), worst rel-L2", b_err, 1e-4);
  return canonical_of;
}

// The reference checkpoint layout (Compiled::save + save_optimisers,
// include/passes/compile.h:259-299) of this GPT as JSON: per archive index
// the tensor shape and the canonical parameter index (the oracle GPT's
// order). Biases with an exactly-zero gradient (the key projections) match
// among themselves by first come; they stay zero in training.
void print_archive_layout(const Outcome &orc_rt, const std::vector<int> &canonical_of) {
  std::printf("{\"config\": {\"vocab\": %u, \"seq\": %u, \"dim\": %u, \"heads\": %u, "
              "\"layers\": %u, \"ffn\": %u},\n \"parameters\": [",
              kVocab, kSeq, kDim, kHeads, kLayers, kFfn);
  for (size_t i = 0; i < canonical_of.size(); ++i) {
    const auto &b = orc_rt.archive.at("parameters/" + std::to_string(i) + "/size");
    std::vector<uint32_t> shape(b.size() / 4);
    std::memcpy(shape.data(), b.data(), b.size());
    std::printf("%s\n  {\"shape\": [", i ? "," : "");
    for (size_t k = 0; k < shape.size(); ++k) std::printf("%s%u", k ? ", " : "", shape[k]);
    std::printf("], \"canonical\": %d}", canonical_of[i]);
  }
  std::printf("],\n \"names\": [");
  bool first = true;
  for (const auto &[name, blob] : orc_rt.archive) {
    std::printf("%s\n  [\"%s\", %zu]", first ? "" : ",", name.c_str(), blob.size());
    first = false;
  }
  std::printf("]}\n");
}

uint64_t splitmix(uint64_t &s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

} // namespace

int run(bool cpu_only, bool layout) {
  const uint32_t seed = 1;
  const float max_norm = 1.0f;
  std::vector<uint32_t> tokens(kBatch * kSeq), targets(kBatch * kSeq);
  uint64_t s = 7;
  for (auto &t : tokens) t = uint32_t(splitmix(s) % kVocab);
  for (auto &t : targets) t = uint32_t(splitmix(s) % kVocab);
  std::printf("reference nn::GPT<V=%u, T=%u, D=%u, H=%u> (4 blocks), batch %u, clip %.1f, AdamW "
              "lr %.0e b1 %.2f b2 %.2f wd %.1f, %d steps\n",
              kVocab, kSeq, kDim, kHeads, kBatch, max_norm, kLr, kBeta1, kBeta2, kWd, kSteps);
  std::fflush(stdout);

  orc::Runtime cpu;
  const Outcome ref = train_oracle(cpu, tokens, targets, seed, max_norm);
  std::printf("oracle runtime: loss %.6f -> %.6f\n", ref.losses[0][0], ref.losses[1][0]);
  const std::vector<int> canonical_of = anchor(ref, tokens, targets, seed, max_norm);
  if (layout) {
    if (g_failures) return 1;
    std::printf("ARCHIVE LAYOUT\n");
    print_archive_layout(ref, canonical_of);
    return 0;
  }
  if (cpu_only) {
    std::printf("%s\n", g_failures ? "ORACLE ANCHOR FAILED" : "oracle anchor ok");
    return g_failures ? 1 : 0;
  }

  hip::init(0);
  {
    hip::Runtime gpu;
    const Outcome eager = train_hip(gpu, tokens, targets, seed, max_norm);
    compare("hip::Runtime (eager) vs oracle runtime", eager, ref, 1e-4, 1e-3);
    gpu.set_graph_mode(true);
    const Outcome graph = train_hip(gpu, tokens, targets, seed, max_norm);
    compare("hip::Runtime (graph mode) vs oracle runtime", graph, ref, 1e-4, 1e-3, false);
    const auto st = gpu.graph_stats();
    std::printf("graph mode: %zu recordings, %zu instantiations, %zu in-place updates\n",
                st.captures, st.instantiations, st.updates);
  }
  hip::shutdown();
  std::printf("%s\n", g_failures ? "DROP-IN PARITY FAILED" : "drop-in parity ok");
  return g_failures ? 1 : 0;
}

// The same comparison at the benchmark model's sizes (BenchDims: V 2048,
// T 192, d 384, 6 heads, 4 blocks, batch 2), where hip::Runtime's products
// take the large-shape plans (128x128 tiles for the vocabulary projection,
// split-K and tail splits with pool scratch, the tall column sums).
int run_bench_shapes() {
  using D = BenchDims;
  const uint32_t seed = 1;
  const float max_norm = 1.0f;
  std::vector<uint32_t> tokens(D::batch * D::seq), targets(D::batch * D::seq);
  uint64_t s = 7;
  for (auto &t : tokens) t = uint32_t(splitmix(s) % D::vocab);
  for (auto &t : targets) t = uint32_t(splitmix(s) % D::vocab);
  std::printf("reference nn::GPT<V=%u, T=%u, D=%u, H=%u> (4 blocks), batch %u, clip %.1f, AdamW, "
              "%d steps\n",
              D::vocab, D::seq, D::dim, D::heads, D::batch, max_norm, kSteps);
  orc::Runtime cpu;
  const Outcome ref = train_oracle_bench(cpu, tokens, targets, seed, max_norm);
  std::printf("oracle runtime: loss %.6f -> %.6f\n", ref.losses[0][0], ref.losses[1][0]);
  hip::init(0);
  {
    hip::Runtime gpu;
    const Outcome eager = train_hip_bench(gpu, tokens, targets, seed, max_norm);
    compare("hip::Runtime (eager) vs oracle runtime, benchmark shapes", eager, ref, 1e-4, 1e-3);
    gpu.set_graph_mode(true);
    const Outcome graph = train_hip_bench(gpu, tokens, targets, seed, max_norm);
    compare("hip::Runtime (graph mode) vs oracle runtime, benchmark shapes", graph, ref, 1e-4,
            1e-3, false);
    const auto st = gpu.graph_stats();
    std::printf("graph mode: %zu recordings, %zu instantiations, %zu in-place updates\n",
                st.captures, st.instantiations, st.updates);
  }
  hip::shutdown();
  std::printf("%s\n", g_failures ? "DROP-IN PARITY FAILED" : "drop-in parity ok");
  return g_failures ? 1 : 0;
}

// Usage: dropin_gpt [--cpu-only | --archive-layout | --bench-shapes]
//   --cpu-only: only the oracle runtime and its anchor (no GPU needed).
//   --archive-layout: print the reference checkpoint layout of this GPT as
//     JSON after "ARCHIVE LAYOUT" (no GPU needed).
//   --bench-shapes: hip::Runtime vs the oracle runtime at BenchDims.
int main(int argc, char **argv) {
  std::setvbuf(stdout, nullptr, _IOLBF, 0);
  try {
    if (argc > 1 && std::strcmp(argv[1], "--bench-shapes") == 0) return run_bench_shapes();
    const bool layout = argc > 1 && std::strcmp(argv[1], "--archive-layout") == 0;
    return run(layout || (argc > 1 && std::strcmp(argv[1], "--cpu-only") == 0), layout);
  } catch (const std::exception &e) {
    std::printf("error: %s\n", e.what());
    return 2;
  }
}
