// hip::Runtime on the GPU: the known-answer tests the reference holds for
// its Metal runtime (tests/test_metal_runtime.cpp:83-658, values restated
// here), the host-side validation the executor relies on (exception types
// for misuse), in-place use, graph mode, and batched-product layouts
// checked against a double-precision host product.
//
// Usage: test_hip_runtime            run every test (needs a GPU)
//        test_hip_runtime --no-device  only check that hip::init() reports
//                                      a missing GPU as std::runtime_error
#include "harness.h"

#include "RTensor/infer_shape.h"
#include "my_hip/runtime.h"
#include "optimiser/AdamW.h"
#include "templit_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <numeric>
#include <random>
#include <span>
#include <stdexcept>
#include <vector>

using Tensor = RTensor<hip::HIP, hip::kernel_type>;
using IndexTensor = RTensor<hip::HIP, hip::index_type>;

namespace {

constexpr float EPS = 1e-5f; // the reference tests' absolute tolerance

void fill(Tensor &t, std::initializer_list<float> values) {
  CHECK(values.size() == t.numel());
  t.set(std::span<const float>(values.begin(), values.size()));
}

template <typename T> std::vector<T> host(const RTensor<hip::HIP, T> &t) {
  std::vector<T> out(t.numel());
  t.read(std::span<T>(out));
  return out;
}

void expect(const Tensor &t, std::initializer_list<float> values, float tol = EPS) {
  const auto got = host(t);
  CHECK(got.size() == values.size());
  size_t i = 0;
  for (float v : values) {
    if (i < got.size()) CHECK_NEAR(got[i], v, tol);
    ++i;
  }
}

void expect_shape(const Tensor &t, std::initializer_list<uint32_t> shape) {
  CHECK(t.shape() == std::vector<uint32_t>(shape));
}

// One start/submit/wait bracket around `body`, aborting on exceptions
// (the pattern of passes::Compiled, include/passes/compile.h:174-184).
template <typename F> void run(hip::Runtime &rt, F &&body) {
  rt.start();
  try {
    body();
    rt.submit();
    rt.wait();
  } catch (...) {
    rt.abort();
    throw;
  }
}

std::vector<float> random_values(size_t n, uint32_t seed) {
  std::mt19937 gen(seed);
  std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
  std::vector<float> v(n);
  for (auto &x : v) x = dist(gen);
  return v;
}

// ---- the reference's known-answer tests ------------------------------------

void lifecycle(hip::Runtime &rt) { // test_metal_runtime.cpp:83-123
  CHECK_THROWS(std::logic_error, rt.submit());
  rt.start();
  CHECK_THROWS(std::logic_error, rt.start());
  rt.abort();
  rt.start();
  rt.submit();
  CHECK_THROWS(std::logic_error, rt.submit());
  rt.wait();
  CHECK_THROWS(std::logic_error, rt.wait());
}

void binary_and_chained(hip::Runtime &rt) { // 131-158
  Tensor a({2, 2}), b({2, 2});
  fill(a, {1, 2, 3, 4});
  fill(b, {5, 6, 7, 8});
  Tensor added({2, 2}), subtracted({2, 2}), multiplied({2, 2}), divided({2, 2}), chained({2, 2});
  run(rt, [&] {
    rt.add(a, b, added);
    rt.sub(a, b, subtracted);
    rt.hadamard(a, b, multiplied);
    rt.divide(a, b, divided);
    rt.hadamard(added, a, chained);
  });
  expect(added, {6, 8, 10, 12});
  expect(subtracted, {-4, -4, -4, -4});
  expect(multiplied, {5, 12, 21, 32});
  expect(divided, {0.2f, 1.0f / 3.0f, 3.0f / 7.0f, 0.5f});
  expect(chained, {6, 16, 30, 48});
}

void broadcasting(hip::Runtime &rt) { // 160-174
  Tensor m({2, 3}), row({3}), out({2, 3});
  fill(m, {1, 2, 3, 4, 5, 6});
  fill(row, {10, 20, 30});
  run(rt, [&] { rt.add(m, row, out); });
  expect_shape(out, {2, 3});
  expect(out, {11, 22, 33, 14, 25, 36});
}

void scalar_ops(hip::Runtime &rt) { // 176-199
  Tensor in({2, 2}), added({2, 2}), divided({2, 2}), cubed({2, 2}), in_place({2, 2});
  fill(in, {2, 4, 6, 8});
  fill(in_place, {2, 4, 6, 8});
  run(rt, [&] {
    rt.add(in, 3.0f, added);
    rt.divide(in, 2.0f, divided);
    rt.pow(in, 3.0f, cubed);
    rt.divide(in_place, 2.0f, in_place);
    rt.pow(in_place, 2.0f, in_place);
  });
  expect(added, {5, 7, 9, 11});
  expect(divided, {1, 2, 3, 4});
  expect(cubed, {8, 64, 216, 512}, 1e-3f);
  expect(in_place, {1, 4, 9, 16}, 1e-3f);
}

void unary_ops(hip::Runtime &rt) { // 201-226
  Tensor in({4}), squares({4}), sig({4}), ex({4}), root({4});
  fill(in, {0, 1, -1, 2});
  fill(squares, {0, 1, 4, 9});
  run(rt, [&] {
    rt.sigmoid(in, sig);
    rt.exp(in, ex);
    rt.sqrt(squares, root);
  });
  expect(sig, {0.5f, 1.0f / (1.0f + std::exp(-1.0f)), 1.0f / (1.0f + std::exp(1.0f)),
               1.0f / (1.0f + std::exp(-2.0f))});
  expect(ex, {1.0f, std::exp(1.0f), std::exp(-1.0f), std::exp(2.0f)});
  expect(root, {0, 1, 2, 3});
}

void rms_and_rms_norm(hip::Runtime &rt) { // 228-244
  Tensor in({2, 2}), rms({2, 1}), norm({2, 2});
  fill(in, {3, 4, 0, 0});
  run(rt, [&] {
    rt.RMS(in, rms);
    rt.RMSNorm(in, norm);
  });
  const float r = std::sqrt(12.5f + 1e-6f);
  expect(rms, {r, 1e-3f}); // a zero row has rms sqrt(eps) = 1e-3
  expect(norm, {3.0f / r, 4.0f / r, 0, 0});
}

void gelu(hip::Runtime &rt) { // 246-279
  Tensor in({5}), out({5}), der({5});
  fill(in, {-2, -1, 0, 1, 2});
  run(rt, [&] {
    rt.GELU(in, out);
    rt.GELU_derivative(in, der);
  });
  const auto f = [](float x) {
    return 0.5f * x * (1.0f + std::tanh(0.7978845608f * (x + 0.044715f * x * x * x)));
  };
  const auto df = [](float x) {
    const float a = 0.7978845608f, b = 0.044715f, t = std::tanh(a * (x + b * x * x * x));
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * a * (1.0f + 3.0f * b * x * x);
  };
  expect(out, {f(-2), f(-1), f(0), f(1), f(2)});
  expect(der, {df(-2), df(-1), df(0), df(1), df(2)});
}

void matmul(hip::Runtime &rt) { // 281-305
  Tensor a({2, 3}), b({3, 2}), ba({2, 2, 2}), bb({2, 2, 2}), out({2, 2}), bout({2, 2, 2});
  fill(a, {1, 2, 3, 4, 5, 6});
  fill(b, {7, 8, 9, 10, 11, 12});
  fill(ba, {1, 2, 3, 4, 2, 0, 1, 2});
  fill(bb, {5, 6, 7, 8, 1, 3, 4, 2});
  run(rt, [&] {
    rt.mult(a, b, out);
    rt.mult(ba, bb, bout);
  });
  expect(out, {58, 64, 139, 154});
  expect(bout, {19, 22, 43, 50, 2, 6, 9, 7});
}

void tiled_identity_matmul(hip::Runtime &rt) { // 307-342
  constexpr uint32_t n = 64, batches = 2;
  Tensor id({batches, n, n}), vals({batches, n, n}), out({batches, n, n});
  std::vector<float> idv(batches * n * n, 0.0f), v(batches * n * n);
  for (uint32_t b = 0; b < batches; ++b)
    for (uint32_t r = 0; r < n; ++r) idv[b * n * n + r * n + r] = 1.0f;
  for (uint32_t i = 0; i < v.size(); ++i) v[i] = float(i % 31) - 15.0f;
  id.set(idv);
  vals.set(v);
  run(rt, [&] { rt.mult(id, vals, out); });
  const auto got = host(out);
  size_t bad = 0;
  for (size_t i = 0; i < got.size(); ++i) bad += std::fabs(got[i] - v[i]) >= EPS;
  CHECK(bad == 0);
}

void reductions_and_transpose(hip::Runtime &rt) { // 344-374
  Tensor in({2, 3});
  fill(in, {1, 2, 3, 4, 5, 6});
  const std::vector<uint32_t> col = {2, 1}, row = {1, 3};
  Tensor total({1}), row_sums({2, 1}), col_sums(row), row_max(col), tr({3, 2});
  run(rt, [&] {
    rt.sum(in, total);
    rt.sum(in, 1, row_sums);
    rt.sum_to_shape(in, row, col_sums);
    rt.max_to_shape(in, col, row_max);
    rt.transpose(in, tr);
  });
  expect(total, {21});
  expect(row_sums, {6, 15});
  expect(col_sums, {5, 7, 9});
  expect(row_max, {3, 6});
  expect_shape(tr, {3, 2});
  expect(tr, {1, 4, 2, 5, 3, 6});
}

void sum_to_shape_multi(hip::Runtime &rt) { // 376-413
  Tensor in({2, 3, 4});
  std::vector<float> v(24);
  std::iota(v.begin(), v.end(), 1.0f);
  in.set(v);
  const std::vector<uint32_t> s1 = {1, 3, 1}, s2 = {2, 1, 1}, s3 = {1, 1, 1}, s4 = {4};
  Tensor o1(s1), o2(s2), o3(s3), o4(s4);
  run(rt, [&] {
    rt.sum_to_shape(in, s1, o1);
    rt.sum_to_shape(in, s2, o2);
    rt.sum_to_shape(in, s3, o3);
    rt.sum_to_shape(in, s4, o4);
  });
  expect(o1, {68, 100, 132});
  expect(o2, {78, 222});
  expect(o3, {300});
  expect(o4, {66, 72, 78, 84});
}

void sum_to_shape_leading_singletons(hip::Runtime &rt) { // 415-430
  Tensor in({1, 4});
  fill(in, {1, 2, 3, 4});
  const std::vector<uint32_t> s = {4};
  Tensor out(s);
  run(rt, [&] { rt.sum_to_shape(in, s, out); });
  expect_shape(out, {4});
  expect(out, {1, 2, 3, 4});
}

void softmax(hip::Runtime &rt) { // 432-472
  Tensor in({2, 3}), out({2, 3}), r1({3}), r1o({3}), r4({2, 2, 1, 3}), r4o({2, 2, 1, 3}),
      single({2, 1}), singleo({2, 1});
  fill(in, {1, 2, 3, 1, 1, 1});
  fill(r1, {1, 2, 3});
  fill(r4, {1, 2, 3, 3, 2, 1, 1000, 1001, 1002, -1000, -1000, -1000});
  fill(single, {4, -7});
  run(rt, [&] {
    rt.softmax(in, out);
    rt.softmax(r1, r1o);
    rt.softmax(r4, r4o);
    rt.softmax(single, singleo);
  });
  const float d = std::exp(-2.0f) + std::exp(-1.0f) + 1.0f;
  const float lo = std::exp(-2.0f) / d, mid = std::exp(-1.0f) / d, hi = 1.0f / d, t = 1.0f / 3.0f;
  expect(out, {lo, mid, hi, t, t, t});
  expect(r1o, {lo, mid, hi});
  expect(r4o, {lo, mid, hi, hi, mid, lo, lo, mid, hi, t, t, t});
  expect(singleo, {1, 1});
}

void cross_entropy(hip::Runtime &rt) { // 474-507
  Tensor logits({2, 2, 3}), losses({2, 2, 1}), grads({2, 2, 3});
  fill(logits, {1, 2, 3, 1, 1, 1, 1000, 1001, 1002, -1, -2, -3});
  IndexTensor targets({2, 2});
  const std::vector<uint32_t> tv = {2, 0, 1, 2};
  targets.set(tv);
  run(rt, [&] {
    rt.cross_entropy(logits, targets, losses);
    rt.cross_entropy_derivative(logits, targets, grads);
  });
  const float d = std::exp(-2.0f) + std::exp(-1.0f) + 1.0f;
  const float lo = std::exp(-2.0f) / d, mid = std::exp(-1.0f) / d, hi = 1.0f / d, ld = std::log(d);
  expect(losses, {ld, std::log(3.0f), 1.0f + ld, 2.0f + ld}, 1e-4f);
  expect(grads, {lo, mid, hi - 1.0f, -2.0f / 3.0f, 1.0f / 3.0f, 1.0f / 3.0f, lo, mid - 1.0f, hi, hi,
                 mid, lo - 1.0f},
         1e-4f);
}

void cross_entropy_bad_target(hip::Runtime &rt) {
  // A target outside the vocabulary gives +INF loss and a row of +INF
  // gradients (math.metal:893-896, 921-926).
  Tensor logits({2, 3}), loss({2, 1}), grad({2, 3});
  fill(logits, {1, 2, 3, 4, 5, 6});
  IndexTensor targets({2});
  const std::vector<uint32_t> tv = {1, 3};
  targets.set(tv);
  run(rt, [&] {
    rt.cross_entropy(logits, targets, loss);
    rt.cross_entropy_derivative(logits, targets, grad);
  });
  const auto l = host(loss), g = host(grad);
  CHECK(std::isfinite(l[0]));
  CHECK(std::isinf(l[1]) && l[1] > 0);
  for (int i = 3; i < 6; ++i) CHECK(std::isinf(g[i]) && g[i] > 0);
}

void argmax(hip::Runtime &rt) { // 509-531
  Tensor small({2, 3});
  fill(small, {1, 4, 2, 9, 3, 5});
  Tensor large({5000});
  std::vector<float> v(5000, 0.0f);
  v[4097] = 100.0f;
  large.set(v);
  Tensor ties({6});
  fill(ties, {1, 7, 7, 2, 7, 0}); // lowest index of the maximum wins
  IndexTensor so({1, 1}), lo({1, 1}), to({1, 1});
  run(rt, [&] {
    rt.argmax(small, so);
    rt.argmax(large, lo);
    rt.argmax(ties, to);
  });
  CHECK(host(so)[0] == 3);
  CHECK(host(lo)[0] == 4097);
  CHECK(host(to)[0] == 1);
}

void embedding_lookup(hip::Runtime &rt) { // 533-549
  Tensor w({4, 3}), out({2, 2, 3});
  fill(w, {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12});
  IndexTensor ids({2, 2});
  const std::vector<uint32_t> iv = {2, 0, 3, 1};
  ids.set(iv);
  run(rt, [&] { rt.embedding_lookup(w, ids, out); });
  expect(out, {7, 8, 9, 1, 2, 3, 10, 11, 12, 4, 5, 6}, 0.0f);
}

void scatter_index(hip::Runtime &rt) { // 551-569
  Tensor values({2, 2, 3}), out({4, 3});
  fill(values, {1, 2, 3, 4, 5, 6, 10, 20, 30, 7, 8, 9});
  IndexTensor ids({2, 2});
  const std::vector<uint32_t> iv = {2, 0, 2, 1};
  ids.set(iv);
  fill(out, {99, 99, 99, 99, 99, 99, 99, 99, 99, 99, 99, 99});
  run(rt, [&] { rt.scatter_index(values, ids, out); });
  expect(out, {4, 5, 6, 7, 8, 9, 11, 22, 33, 0, 0, 0});
}

void scatter_add_rows(hip::Runtime &rt) { // 571-593
  Tensor base({4, 3}), values({2, 2, 3}), out({4, 3});
  fill(base, {100, 101, 102, 103, 104, 105, 106, 107, 108, 109, 110, 111});
  fill(values, {1, 2, 3, 4, 5, 6, 10, 20, 30, 7, 8, 9});
  IndexTensor ids({2, 2});
  const std::vector<uint32_t> iv = {2, 0, 2, 1};
  ids.set(iv);
  run(rt, [&] { rt.scatter_add_rows(base, ids, values, out); });
  expect(out, {104, 106, 108, 110, 112, 114, 117, 129, 141, 109, 110, 111});
  expect(base, {100, 101, 102, 103, 104, 105, 106, 107, 108, 109, 110, 111}); // base untouched
}

void gradient_clipping(hip::Runtime &rt) { // 595-615
  Tensor first({3}), second({1});
  Tensor s = Tensor::from_zeros({1});
  fill(first, {3, 4, 0});
  fill(second, {12});
  run(rt, [&] {
    rt.accumulate_gradient_squared_norm(first, s);
    rt.accumulate_gradient_squared_norm(second, s);
    rt.clip_gradient(first, s, 1.0f, first);
    rt.clip_gradient(second, s, 1.0f, second);
  });
  expect(s, {169});
  expect(first, {3.0f / 13, 4.0f / 13, 0});
  expect(second, {12.0f / 13});
}

void adamw(hip::Runtime &rt) { // 617-658
  using AdamW = Optimiser::AdamW<Tensor>;
  Tensor p({4}), g({4});
  fill(p, {1, -2, 3, -4});
  fill(g, {0.5f, -0.25f, 1.0f, -0.75f});
  AdamW opt;
  auto params = AdamW::generate_params(0.01f, 0.9f, 0.999f, 1e-8f, 0.01f);
  std::vector<float> e = {1, -2, 3, -4}, m1(4, 0.0f), m2(4, 0.0f);
  const std::vector<float> gv = {0.5f, -0.25f, 1.0f, -0.75f};
  for (uint32_t step = 1; step <= 2; ++step) {
    run(rt, [&] { opt.update(rt, params, p, g, p); });
    const float c1 = 1.0f - std::pow(0.9f, float(step)), c2 = 1.0f - std::pow(0.999f, float(step));
    for (size_t i = 0; i < 4; ++i) {
      m1[i] = 0.9f * m1[i] + 0.1f * gv[i];
      m2[i] = 0.999f * m2[i] + 0.001f * gv[i] * gv[i];
      e[i] = e[i] * 0.9999f - 0.01f * (m1[i] / c1) / (std::sqrt(m2[i] / c2) + 1e-8f);
    }
    expect(p, {e[0], e[1], e[2], e[3]}, 1e-5f);
  }
  CHECK(opt.step() == 2);
}

void cleanup_is_idempotent() { // 125-129
  hip::Runtime rt;
  rt.cleanup();
  rt.cleanup();
}

// ---- validation the executor relies on ----------------------------------------

void validation(hip::Runtime &rt) {
  Tensor a({2, 3}), b({3, 2}), wrong({3, 3}), ok({2, 2});
  // ops outside start..submit
  CHECK_THROWS(std::logic_error, rt.add(a, a, a));
  rt.start();
  CHECK_THROWS(std::invalid_argument, rt.mult(a, b, wrong));
  CHECK_THROWS(std::invalid_argument, rt.mult(a, a, ok)); // inner dims differ
  CHECK_THROWS(std::runtime_error, rt.add(a, b, a));       // cannot broadcast
  CHECK_THROWS(std::invalid_argument, rt.add(a, 1.0f, wrong));
  CHECK_THROWS(std::invalid_argument, rt.transpose(a, a));
  CHECK_THROWS(std::out_of_range, rt.transpose(a, b, 0, 2));
  CHECK_THROWS(std::out_of_range, rt.sum(a, 2, ok));
  CHECK_THROWS(std::invalid_argument, rt.softmax(a, b));
  Tensor g({4}), p({4}), m({4}), v({4}), s1({1}), bad({2});
  CHECK_THROWS(std::invalid_argument, rt.adamW(p, g, p, m, v, s1, s1, s1, s1, 1e-8f, 0));
  CHECK_THROWS(std::invalid_argument, rt.adamW(p, g, p, m, v, bad, s1, s1, s1, 1e-8f, 1));
  CHECK_THROWS(std::invalid_argument, rt.clip_gradient(g, s1, 0.0f, g));
  CHECK_THROWS(std::invalid_argument, rt.clip_gradient(g, s1, NAN, g));
  Tensor w({4, 3}), emb_bad({2, 3});
  IndexTensor ids({2, 2});
  CHECK_THROWS(std::invalid_argument, rt.embedding_lookup(w, ids, emb_bad));
  Tensor logits({2, 3}), loss_bad({2});
  IndexTensor targets({2});
  CHECK_THROWS(std::invalid_argument, rt.cross_entropy(logits, targets, loss_bad));
  Tensor r({2, 3}), rms_bad({2, 3});
  CHECK_THROWS(std::invalid_argument, rt.RMS(r, rms_bad));
  const std::vector<uint32_t> two_shrinks = {1, 1};
  Tensor mx({1, 1});
  CHECK_THROWS(std::invalid_argument, rt.max_to_shape(a, two_shrinks, mx));
  rt.abort();
}

void max_to_shape_alias(hip::Runtime &rt) {
  // Nothing to shrink: the destination becomes the input (runtime.cpp:629-632).
  Tensor a({2, 3}), out({2, 3});
  fill(a, {1, 2, 3, 4, 5, 6});
  const std::vector<uint32_t> same = {2, 3};
  run(rt, [&] { rt.max_to_shape(a, same, out); });
  CHECK(out.get_storage() == a.get_storage());
  CHECK(a.get_storage()->ref_count == 2);
}

void in_place_and_split_merge(hip::Runtime &rt) {
  Tensor x({2, 4}), bias({1, 4}), split({2, 2, 2}), merged({2, 4});
  fill(x, {1, 2, 3, 4, 5, 6, 7, 8});
  fill(bias, {10, 20, 30, 40});
  run(rt, [&] {
    rt.add(x, bias, x); // the executor's LINEAR bias add (execute.h:249)
    rt.split_last_dim(x, split, 2, 2);
    rt.merge_last_dims(split, merged, 2, 2);
  });
  expect(x, {11, 22, 33, 44, 15, 26, 37, 48});
  expect(split, {11, 22, 33, 44, 15, 26, 37, 48});
  expect(merged, {11, 22, 33, 44, 15, 26, 37, 48});
  // split / merge are reshapes: the destinations become views of the input,
  // as in the reference CPU runtime (CPU/runtime.h:53-75)
  CHECK(split.get_storage() == x.get_storage());
  CHECK(merged.get_storage() == x.get_storage());
}

// Double-precision host product for the batched layouts of the GPT:
// weight broadcast [B,T,D].[D,F], attention [B,H,T,d].[B,H,d,T] and a rank-3
// by rank-4 broadcast of the batch dims.
void batched_matmul_layouts(hip::Runtime &rt) {
  struct Case {
    std::vector<uint32_t> a, b;
  };
  const Case cases[] = {{{4, 24, 32}, {32, 40}},
                        {{2, 3, 17, 64}, {2, 3, 64, 19}},
                        {{3, 1, 8, 16}, {1, 2, 16, 8}},
                        {{5, 33, 7}, {5, 7, 65}}};
  uint32_t seed = 1;
  for (const Case &c : cases) {
    const auto shape = rtensor::infer_mult(c.a, c.b);
    Tensor a(c.a), b(c.b), out(shape);
    const auto av = random_values(a.numel(), seed++), bv = random_values(b.numel(), seed++);
    a.set(av);
    b.set(bv);
    run(rt, [&] { rt.mult(a, b, out); });
    const auto got = host(out);
    const size_t r = shape.size();
    const uint32_t M = shape[r - 2], N = shape[r - 1], K = c.a.back();
    // decode each output batch index into the operands' broadcast offsets
    const size_t batches = out.numel() / (size_t(M) * N);
    double max_err = 0, max_ref = 0;
    for (size_t bi = 0; bi < batches; ++bi) {
      size_t rem = bi, off_a = 0, off_b = 0, sa = 1, sb = 1;
      for (size_t d = r - 2; d-- > 0;) {
        const uint32_t dim = shape[d];
        const uint32_t idx = uint32_t(rem % dim);
        rem /= dim;
        const size_t da = d + c.a.size() >= r ? d + c.a.size() - r : size_t(-1);
        const size_t db = d + c.b.size() >= r ? d + c.b.size() - r : size_t(-1);
        if (da != size_t(-1)) {
          if (c.a[da] != 1) off_a += idx * sa;
          sa *= c.a[da];
        }
        if (db != size_t(-1)) {
          if (c.b[db] != 1) off_b += idx * sb;
          sb *= c.b[db];
        }
      }
      for (uint32_t m = 0; m < M; ++m)
        for (uint32_t n = 0; n < N; ++n) {
          double acc = 0;
          for (uint32_t k = 0; k < K; ++k)
            acc += double(av[off_a * M * K + m * K + k]) * bv[off_b * K * N + k * N + n];
          max_err = std::max(max_err, std::fabs(acc - got[bi * M * N + m * N + n]));
          max_ref = std::max(max_ref, std::fabs(acc));
        }
    }
    CHECK(max_err <= 1e-3 * max_ref); // matmul tolerance: rel 1e-3
  }
}

// Graph mode: the same recording replayed from the cache gives the eager
// result, and a repeat refreshes the cached graph instead of rebuilding it.
void graph_mode(hip::Runtime &rt) {
  Tensor x({64, 96}), w({96, 128}), bias({1, 128}), y({64, 128}), z({64, 128});
  x.set(random_values(x.numel(), 11));
  w.set(random_values(w.numel(), 12));
  bias.set(random_values(bias.numel(), 13));
  const auto step = [&] {
    Tensor tmp({64, 128}); // a per-call temporary like the executor's
    rt.mult(x, w, tmp);
    rt.add(tmp, bias, tmp);
    rt.GELU(tmp, y);
    rt.softmax(y, z);
  };
  run(rt, step);
  const auto eager = host(z);
  rt.set_graph_mode(true);
  for (int i = 0; i < 3; ++i) {
    z.get_storage()->fill(0.0f);
    run(rt, step);
    const auto got = host(z);
    double err = 0;
    for (size_t k = 0; k < got.size(); ++k) err = std::max(err, double(std::fabs(got[k] - eager[k])));
    CHECK(err == 0.0);
  }
  const auto stats = rt.graph_stats();
  CHECK(stats.captures == 3);
  CHECK(stats.instantiations == 1);
  CHECK(stats.updates == 2);
  // Host writes while recording land at record time (EXPR_CONSTANT,
  // include/passes/execute.h:458-466).
  Tensor c({1, 1}), out({1, 1});
  run(rt, [&] {
    const float v = 2.5f;
    c.set(std::span<const float>(&v, 1));
    rt.add(c, 1.0f, out);
  });
  expect(out, {3.5f});
  rt.set_graph_mode(false);
}

// Graph mode with pool scratch: a split-K product releases its K-chunk
// partials during the capture; a tensor of the same size class created
// later in that capture and written from the host at record time must keep
// its contents when the graph runs the product.
void graph_mode_scratch_is_not_reused_within_a_capture(hip::Runtime &rt) {
  constexpr uint32_t M = 384, K = 6144, N = 384; // 36 tiles: split over K
  const uint32_t one = 1, none = 0;
  size_t ws = 0;
  hip::detail::check(tlh_matmul_workspace_size(M, K, N, K, 1, N, 1, N, 1, 1, &one, &none, &none,
                                               &none, &ws),
                     "workspace size");
  CHECK(ws > 0);
  Tensor a({M, K}), b({K, N}), prod({M, N}), out({uint32_t(ws)});
  a.set(random_values(a.numel(), 21));
  b.set(random_values(b.numel(), 22));
  const auto values = random_values(ws, 23);
  rt.set_graph_mode(true);
  for (int i = 0; i < 2; ++i) {
    run(rt, [&] {
      rt.mult(a, b, prod);
      Tensor c({uint32_t(ws)}); // same size class as the released partials
      c.set(values);            // lands at record time (EXPR_CONSTANT)
      rt.add(c, 1.0f, out);
    });
    const auto got = host(out);
    size_t bad = 0;
    for (size_t k = 0; k < ws; ++k) bad += got[k] != values[k] + 1.0f;
    CHECK(bad == 0);
  }
  rt.set_graph_mode(false);
}

// sqe = (prediction - target)^2 elementwise (runtime.cpp:843-848), with
// the executor's broadcasting and in place.
// transpose / copy / identity sum_to_shape results are views filled on
// demand: every way to observe them gives the materialised values.
void deferred_views(hip::Runtime &rt) {
  const std::vector<float> av = random_values(6 * 4, 11), bv = random_values(6 * 5, 12);
  Tensor a({6, 4}), b({6, 5});
  a.set(std::span<const float>(av));
  b.set(std::span<const float>(bv));
  auto at = [&](size_t r, size_t c) { return av[r * 4 + c]; };
  // 1. host read of a transpose
  Tensor t1({4, 6});
  run(rt, [&] { rt.transpose(a, t1); });
  {
    const auto got = host(t1);
    for (size_t i = 0; i < 4; ++i)
      for (size_t j = 0; j < 6; ++j) CHECK(got[i * 6 + j] == at(j, i));
  }
  // 2. the transposed operand of a product (read through its strides), then
  // the source overwritten while a second view of it is pending
  Tensor t2({4, 6}), p({4, 5}), c({6, 4});
  run(rt, [&] {
    rt.transpose(a, t2);
    rt.mult(t2, b, p);       // A^T . B
    rt.add(a, a, a);         // the source changes: t2 must keep the old values
  });
  {
    const auto got = host(p);
    for (size_t i = 0; i < 4; ++i)
      for (size_t j = 0; j < 5; ++j) {
        double e = 0;
        for (size_t k = 0; k < 6; ++k) e += double(at(k, i)) * bv[k * 5 + j];
        CHECK_NEAR(got[i * 5 + j], e, 1e-5);
      }
    const auto t2h = host(t2), ah = host(a);
    for (size_t i = 0; i < 4; ++i)
      for (size_t j = 0; j < 6; ++j) {
        CHECK(t2h[i * 6 + j] == at(j, i));
        CHECK(ah[j * 4 + i] == at(j, i) + at(j, i));
      }
  }
  a.set(std::span<const float>(av));
  // 3. copy then in-place accumulation (GradientContext::accumulate), a host
  // write to the source of a pending copy, and a transpose into a reused
  // destination
  Tensor g({6, 4}), h({6, 4}), s({6, 4}), r({4, 6});
  run(rt, [&] {
    rt.copy(a, g);
    rt.add(g, a, g); // g = 2a
    rt.copy(a, h);
    rt.transpose(a, r);
    rt.transpose(g, r); // r is overwritten before its first view was filled
    rt.sum_to_shape(a, std::vector<uint32_t>{6, 4}, s);
  });
  std::vector<float> zeros(24, 0.0f);
  a.set(std::span<const float>(zeros)); // the pending copy h keeps a's old values
  {
    const auto gh = host(g), hh = host(h), rh = host(r), sh = host(s);
    for (size_t i = 0; i < 24; ++i) {
      CHECK(gh[i] == av[i] + av[i]);
      CHECK(hh[i] == av[i]);
      CHECK(sh[i] == av[i]);
    }
    for (size_t i = 0; i < 4; ++i)
      for (size_t j = 0; j < 6; ++j) CHECK(rh[i * 6 + j] == at(j, i) + at(j, i));
  }
  // 4. an elementwise consumer (not a product or broadcast op) fills the view
  Tensor e({4, 6});
  a.set(std::span<const float>(av));
  run(rt, [&] {
    rt.transpose(a, t1);
    rt.exp(t1, e);
  });
  {
    const auto got = host(e);
    for (size_t i = 0; i < 4; ++i)
      for (size_t j = 0; j < 6; ++j) CHECK_NEAR(got[i * 6 + j], std::exp(at(j, i)), 1e-5);
  }
  // 5. views of views: a transpose of a pending transpose and a copy of it
  // view the first source; the intermediate is then overwritten whole (its
  // view is dropped, never filled) and the source changes afterwards
  const std::vector<float> xv = random_values(2 * 3 * 4, 13);
  Tensor x({2, 3, 4}), x1({3, 2, 4}), x2({3, 4, 2}), x3({3, 4, 2}), y({3, 2, 4});
  x.set(std::span<const float>(xv));
  y.set(std::span<const float>(xv));
  run(rt, [&] {
    rt.transpose(x, x1, 0, 1);
    rt.transpose(x1, x2, 1, 2);
    rt.copy(x2, x3);
    rt.divide(y, 0.5f, x1); // x1 = 2y: its pending view is dead
    rt.add(x, x, x);       // x changes: x2 and x3 keep its old values
  });
  {
    const auto h1 = host(x1), h2 = host(x2), h3 = host(x3), hx = host(x);
    for (size_t i = 0; i < 2; ++i)
      for (size_t j = 0; j < 3; ++j)
        for (size_t k = 0; k < 4; ++k) {
          const float v = xv[(i * 3 + j) * 4 + k];
          CHECK(h1[(i * 3 + j) * 4 + k] == 2.0f * v); // y holds xv in the same order
          CHECK(h2[(j * 4 + k) * 2 + i] == v);
          CHECK(h3[(j * 4 + k) * 2 + i] == v);
          CHECK(hx[(i * 3 + j) * 4 + k] == v + v);
        }
  }
  // 6. the squared norm reads a pending copy's source, and an in-place clip
  // of the copy writes it without the copy being made; the source keeps its
  // values
  Tensor gsrc({3}), gslot({3});
  Tensor sq = Tensor::from_zeros({1});
  fill(gsrc, {3, 4, 12});
  run(rt, [&] {
    rt.copy(gsrc, gslot);
    rt.accumulate_gradient_squared_norm(gslot, sq);
    rt.clip_gradient(gslot, sq, 1.0f, gslot);
  });
  expect(sq, {169});
  expect(gslot, {3.0f / 13, 4.0f / 13, 12.0f / 13});
  expect(gsrc, {3, 4, 12});
  // 7. a source overwritten whole while views of it are pending (the
  // executor's next step rewriting a node buffer): the views keep the old
  // values, the source and its aliases see the new ones, and a view of the
  // new values can be taken again
  a.set(std::span<const float>(av));
  Tensor v1({4, 6}), v2({6, 4}), v3({4, 6}), alias({6, 2, 2});
  run(rt, [&] {
    rt.transpose(a, v1);
    rt.copy(a, v2);
    rt.split_last_dim(a, alias, 2, 2); // alias shares a's storage
    rt.divide(v2, 0.25f, a);           // a = 4 * old a, read from the pending copy
    rt.transpose(a, v3);
  });
  {
    const auto h1 = host(v1), h2 = host(v2), h3 = host(v3), ha = host(a), hal = host(alias);
    for (size_t i = 0; i < 4; ++i)
      for (size_t j = 0; j < 6; ++j) {
        CHECK(h1[i * 6 + j] == at(j, i));
        CHECK(h3[i * 6 + j] == 4.0f * at(j, i));
      }
    for (size_t i = 0; i < 24; ++i) {
      CHECK(h2[i] == av[i]);
      CHECK(ha[i] == 4.0f * av[i]);
      CHECK(hal[i] == 4.0f * av[i]);
    }
  }
  // 8. a transposed view of a split alias of a pending copy (the executor's
  // head split of a reused product: split_last_dim, then transpose<1,2>)
  // reads the copy's source through the alias's layout
  a.set(std::span<const float>(av));
  Tensor cp({6, 4}), heads({6, 2, 2}), ht({2, 6, 2});
  run(rt, [&] {
    rt.copy(a, cp);                     // pending copy of a ([6, 4])
    rt.split_last_dim(cp, heads, 2, 2); // [6, 2, 2], aliasing cp
    rt.transpose(heads, ht, 0, 1);      // [2, 6, 2]
  });
  {
    const auto h = host(ht), hc = host(cp);
    for (size_t p = 0; p < 2; ++p)
      for (size_t r = 0; r < 6; ++r)
        for (size_t q = 0; q < 2; ++q) CHECK(h[(p * 6 + r) * 2 + q] == av[r * 4 + p * 2 + q]);
    for (size_t k = 0; k < 24; ++k) CHECK(hc[k] == av[k]);
  }
}

// The executor evaluates a gradient expression once per path, so the same
// op runs again on the same values (include/passes/execute.h): the runtime
// hands back the earlier result. Whatever it reuses, every result must be
// what running the op gives, also after inputs, cached blocks or
// destinations change.
void repeated_results(hip::Runtime &rt) {
  const std::vector<float> av = random_values(8 * 16, 31), bv = random_values(16 * 4, 32);
  Tensor a({8, 16}), b({16, 4}), w({8, 4});
  a.set(std::span<const float>(av));
  b.set(std::span<const float>(bv));
  w.set(std::vector<float>(32, 0.0f));
  auto prod = [&](const std::vector<float> &x, const std::vector<float> &y, size_t i, size_t j) {
    double e = 0;
    for (size_t k = 0; k < 16; ++k) e += double(x[i * 16 + k]) * y[k * 4 + j];
    return e;
  };
  auto expect_prod = [&](const Tensor &t, const std::vector<float> &x, const std::vector<float> &y,
                         double scale, double shift) {
    const auto got = host(t);
    for (size_t i = 0; i < 8; ++i)
      for (size_t j = 0; j < 4; ++j)
        CHECK_NEAR(got[i * 4 + j], scale * prod(x, y, i, j) + shift, 1e-4);
  };
  // 1. the same chain twice into other destinations, a third time into the
  // first ones, and once with a changed input
  Tensor p1({8, 4}), p2({8, 4}), e1({8, 4}), e2({8, 4}), q({8, 4});
  run(rt, [&] {
    rt.mult(a, b, p1);
    rt.add(p1, 1.0f, e1);
    rt.mult(a, b, p2);   // reused: p2 = p1
    rt.add(p2, 1.0f, e2); // reused through p2's identity
    rt.mult(a, b, p1);   // p1 already holds it
    rt.add(p1, 1.0f, e1);
    rt.divide(p2, 0.5f, q);
  });
  expect_prod(p1, av, bv, 1, 0);
  expect_prod(p2, av, bv, 1, 0);
  expect_prod(e1, av, bv, 1, 1);
  expect_prod(e2, av, bv, 1, 1);
  expect_prod(q, av, bv, 2, 0);
  // 2. an input changes (kernel write, host write): the op runs again
  std::vector<float> a2(av);
  for (auto &x : a2) x *= 3.0f;
  Tensor p3({8, 4}), p4({8, 4});
  run(rt, [&] {
    rt.divide(a, 1.0f / 3.0f, a); // in place: a = 3a
    rt.mult(a, b, p3);
  });
  expect_prod(p3, a2, bv, 1, 0);
  a.set(std::span<const float>(av));
  run(rt, [&] { rt.mult(a, b, p4); });
  expect_prod(p4, av, bv, 1, 0);
  // 3. the cached block is overwritten in place, then whole: later reuses
  // of the product it held still see the product
  Tensor p5({8, 4}), p6({8, 4}), p7({8, 4});
  run(rt, [&] {
    rt.mult(a, b, p5);
    rt.add(p5, p5, p5); // in place: p5 = 2ab; the cached product keeps the old block
    rt.mult(a, b, p6);  // reused from that block
    rt.exp(w, p6);      // p6 overwritten whole
    rt.mult(a, b, p7);  // reused again
  });
  expect_prod(p5, av, bv, 2, 0);
  expect_prod(p7, av, bv, 1, 0);
  // 4. a reused result read by a kernel that needs bytes (fills the copy)
  Tensor s1({8, 1}), s2({8, 1}), r1({8, 4}), r2({8, 4});
  run(rt, [&] {
    rt.sum_to_shape(p7, std::vector<uint32_t>{8, 1}, s1);
    rt.mult(a, b, r1);
    rt.sum_to_shape(r1, std::vector<uint32_t>{8, 1}, s2); // r1 and p7 hold one value
    rt.softmax(r1, r2);
  });
  {
    const auto g1 = host(s1), g2 = host(s2), gr = host(r2);
    for (size_t i = 0; i < 8; ++i) {
      double e = 0, mx = -1e30, z = 0;
      for (size_t j = 0; j < 4; ++j) {
        e += prod(av, bv, i, j);
        mx = std::max(mx, prod(av, bv, i, j));
      }
      CHECK_NEAR(g1[i], e, 1e-4);
      CHECK(g1[i] == g2[i]);
      for (size_t j = 0; j < 4; ++j) z += std::exp(prod(av, bv, i, j) - mx);
      for (size_t j = 0; j < 4; ++j)
        CHECK_NEAR(gr[i * 4 + j], std::exp(prod(av, bv, i, j) - mx) / z, 1e-5);
    }
  }
  // 5. an expression evaluated once per path, whose evaluation writes a
  // product in place over a difference it just computed (the softmax
  // derivative p * (g - m)): the difference stays cached in its own block,
  // later evaluations reuse it, and each product sees the difference
  Tensor g({8, 4}), m({8, 1}), pw({8, 4}), d1({8, 4}), d2({8, 4}), d3({8, 4});
  const std::vector<float> gv = random_values(32, 33), mv = random_values(8, 34),
                           pv = random_values(32, 35);
  g.set(std::span<const float>(gv));
  m.set(std::span<const float>(mv));
  pw.set(std::span<const float>(pv));
  run(rt, [&] {
    rt.sub(g, m, d1);
    rt.hadamard(pw, d1, d1); // in place over the cached difference
    rt.sub(g, m, d2);        // reused
    rt.hadamard(pw, d2, d2); // reused as well: the same inputs again
    rt.sub(g, m, d3);
  });
  {
    const auto h1 = host(d1), h2 = host(d2), h3 = host(d3);
    for (size_t i = 0; i < 8; ++i)
      for (size_t j = 0; j < 4; ++j) {
        const float diff = gv[i * 4 + j] - mv[i];
        CHECK(h3[i * 4 + j] == diff);
        CHECK(h1[i * 4 + j] == pv[i * 4 + j] * diff);
        CHECK(h2[i * 4 + j] == h1[i * 4 + j]);
      }
  }
  // 6. the same for an op on one input: a row sum divided in place (the
  // RMSNorm derivative's mean, execute.h:343-348), then the sum again
  Tensor m1({8, 1}), m2({8, 1});
  run(rt, [&] {
    rt.sum_to_shape(g, std::vector<uint32_t>{8, 1}, m1);
    rt.divide(m1, 4.0f, m1); // in place over the cached sum
    rt.sum_to_shape(g, std::vector<uint32_t>{8, 1}, m2); // reused
  });
  {
    const auto h1 = host(m1), h2 = host(m2);
    for (size_t i = 0; i < 8; ++i) {
      double e = 0;
      for (size_t j = 0; j < 4; ++j) e += gv[i * 4 + j];
      CHECK_NEAR(h2[i], e, 1e-5);
      CHECK(h1[i] == h2[i] / 4.0f);
    }
  }
}

// Squared norms accumulated into one scalar are collected and run together
// (Compiled::step(max_norm), include/passes/compile.h:241-245): the scalar
// keeps its starting value, a gradient written after its accumulation still
// counts with its old values, and host reads and later ops see the sum.
void collected_norms(hip::Runtime &rt) {
  Tensor a({3}), b({2, 2}), c({1}), s({1}), t({1}), scaled({2, 2});
  fill(a, {1, 2, 3});       // 14
  fill(b, {1, 1, 1, 1});    // 4
  fill(c, {5});             // 25
  fill(s, {100});
  fill(t, {0});
  run(rt, [&] {
    rt.accumulate_gradient_squared_norm(a, s);
    rt.accumulate_gradient_squared_norm(b, s);
    rt.add(b, b, b);        // b = 2: written after its accumulation
    rt.accumulate_gradient_squared_norm(c, t);
    rt.accumulate_gradient_squared_norm(b, t); // 25 + 16
    rt.divide(b, s, scaled); // reads s: 2 / 118
  });
  expect(s, {118});
  expect(t, {41});
  expect(scaled, {2.0f / 118, 2.0f / 118, 2.0f / 118, 2.0f / 118});
  // collected at submit, then read by the host
  run(rt, [&] {
    rt.accumulate_gradient_squared_norm(c, s);
    rt.accumulate_gradient_squared_norm(c, s);
  });
  expect(s, {168});
}

// A graph-mode recording that is aborted never runs: a later identical op
// must compute its result, not take the dropped graph's as done, and
// collected optimiser calls of the aborted phase are dropped with it.
void aborted_capture_forgets_results(hip::Runtime &rt) {
  Tensor a({2, 3}), b({3, 2}), o({2, 2}), s({1}), g({3});
  fill(a, {1, 2, 3, 4, 5, 6});
  fill(b, {7, 8, 9, 10, 11, 12});
  fill(o, {0, 0, 0, 0});
  fill(s, {1});
  fill(g, {1, 1, 1});
  rt.set_graph_mode(true);
  rt.start();
  rt.mult(a, b, o);
  rt.accumulate_gradient_squared_norm(g, s);
  rt.abort();
  rt.set_graph_mode(false);
  run(rt, [&] { rt.mult(a, b, o); });
  expect(o, {58, 64, 139, 154});
  expect(s, {1});
}

// In-place AdamW updates are collected and run as one multi-tensor launch
// (exec::step's per-parameter update calls): the same values as the
// per-tensor kernel, a read of a parameter in between and a write to a
// gradient after its update was queued see the right values.
void collected_adamw(hip::Runtime &rt) {
  Tensor b1({1}), b2({1}), dec({1}), lr({1});
  fill(b1, {0.9f});
  fill(b2, {0.999f});
  fill(dec, {1.0f - 0.01f * 0.1f});
  fill(lr, {0.01f});
  const std::vector<uint32_t> sizes = {4, 7, 5};
  std::vector<Tensor> p, g, m1, m2, q, qo, n1, n2;
  for (size_t i = 0; i < sizes.size(); ++i) {
    const uint32_t n = sizes[i];
    const auto pv = random_values(n, 40 + uint32_t(i)), gv = random_values(n, 50 + uint32_t(i));
    for (auto *v : {&p, &q}) v->emplace_back(std::vector<uint32_t>{n}).set(std::span<const float>(pv));
    g.emplace_back(std::vector<uint32_t>{n}).set(std::span<const float>(gv));
    for (auto *v : {&m1, &m2, &n1, &n2}) v->push_back(Tensor::from_zeros({n}));
    qo.emplace_back(std::vector<uint32_t>{n});
  }
  Tensor peek({7});
  for (uint32_t step = 1; step <= 2; ++step) {
    run(rt, [&] {
      for (size_t i = 0; i < sizes.size(); ++i) {
        rt.adamW(p[i], g[i], p[i], m1[i], m2[i], b1, b2, dec, lr, 1e-8f, step); // collected
        rt.adamW(q[i], g[i], qo[i], n1[i], n2[i], b1, b2, dec, lr, 1e-8f, step); // direct
      }
      rt.copy(p[1], peek);    // reads an updated parameter
      rt.add(g[0], g[0], g[0]); // writes a gradient an update reads
      for (size_t i = 0; i < sizes.size(); ++i) rt.copy(qo[i], q[i]);
    });
    for (size_t i = 0; i < sizes.size(); ++i) {
      const auto a = host(p[i]), b = host(q[i]), ma = host(m1[i]), mb = host(n1[i]);
      for (size_t j = 0; j < a.size(); ++j) {
        CHECK_NEAR(a[j], b[j], 1e-6);
        CHECK_NEAR(ma[j], mb[j], 1e-6);
      }
    }
    const auto pk = host(peek), p1 = host(p[1]);
    for (size_t j = 0; j < 7; ++j) CHECK(pk[j] == p1[j]);
  }
}

// In-place clips by one norm are batched into one launch that runs before
// anything else (Compiled::step(max_norm), include/passes/compile.h:246-249).
// Checked against out-of-place clips, which run directly: the gradients, an
// op reading one of them, a host read in the middle of the recording, a
// gradient clipped twice and the AdamW updates that follow all agree.
void batched_clips(hip::Runtime &rt) {
  Tensor b1({1}), b2({1}), dec({1}), lr({1});
  fill(b1, {0.9f});
  fill(b2, {0.95f});
  fill(dec, {1.0f - 0.01f * 0.1f});
  fill(lr, {0.01f});
  const std::vector<uint32_t> sizes = {4, 7, 4101}; // 4101: a partial chunk
  std::vector<Tensor> p, g, m1, m2, q, h, hc, n1, n2, qo;
  for (size_t i = 0; i < sizes.size(); ++i) {
    const uint32_t n = sizes[i];
    const auto pv = random_values(n, 80 + uint32_t(i));
    auto gv = random_values(n, 90 + uint32_t(i));
    for (auto &x : gv) x *= 3.0f; // a norm above the bound: the clip scales
    for (auto *v : {&p, &q}) v->emplace_back(std::vector<uint32_t>{n}).set(std::span<const float>(pv));
    for (auto *v : {&g, &h}) v->emplace_back(std::vector<uint32_t>{n}).set(std::span<const float>(gv));
    for (auto *v : {&m1, &m2, &n1, &n2}) v->push_back(Tensor::from_zeros({n}));
    hc.emplace_back(std::vector<uint32_t>{n});
    qo.emplace_back(std::vector<uint32_t>{n});
  }
  Tensor s({1}), s2({1}), peek({7}), peek2({7});
  fill(s, {0.0f});
  fill(s2, {0.0f});
  std::vector<float> mid;
  run(rt, [&] {
    for (size_t i = 0; i < sizes.size(); ++i) {
      rt.accumulate_gradient_squared_norm(g[i], s);
      rt.accumulate_gradient_squared_norm(h[i], s2);
    }
    for (size_t i = 0; i < sizes.size(); ++i) rt.clip_gradient(g[i], s, 1.0f, g[i]); // batched
    for (size_t i = 0; i < sizes.size(); ++i) rt.clip_gradient(h[i], s2, 1.0f, hc[i]); // direct
    mid = host(g[0]); // a host read runs the batch
    rt.clip_gradient(g[2], s, 1.0f, g[2]);   // clipped twice: a new batch
    rt.clip_gradient(hc[2], s2, 1.0f, hc[2]); // the same on the other side (another norm)
    rt.copy(g[1], peek); // the op after the clips sees them done
    rt.copy(hc[1], peek2);
    for (size_t i = 0; i < sizes.size(); ++i) {
      rt.adamW(p[i], g[i], p[i], m1[i], m2[i], b1, b2, dec, lr, 1e-8f, 1);
      rt.adamW(q[i], hc[i], qo[i], n1[i], n2[i], b1, b2, dec, lr, 1e-8f, 1);
    }
    for (size_t i = 0; i < sizes.size(); ++i) rt.copy(qo[i], q[i]);
  });
  const auto hc0 = host(hc[0]);
  for (size_t j = 0; j < hc0.size(); ++j) CHECK(mid[j] == hc0[j]);
  for (size_t i = 0; i < sizes.size(); ++i) {
    const auto ga = host(g[i]), gb = host(hc[i]), a = host(p[i]), b = host(q[i]);
    for (size_t j = 0; j < ga.size(); ++j) {
      CHECK(ga[j] == gb[j]); // the same clips of the same values
      CHECK_NEAR(a[j], b[j], 1e-6); // and the updates (multi-tensor vs single kernel)
    }
  }
  const auto k1 = host(peek), k2 = host(peek2);
  for (size_t j = 0; j < 7; ++j) CHECK(k1[j] == k2[j]);
  // gradient slots that are still pending copies (a slot's one contribution,
  // context.h:73-89) are clipped from the copy's source, which keeps its
  // values; a clip of a tensor that a pending copy reads runs before that
  // copy's own clip can read it
  auto xv = random_values(4101, 95);
  for (auto &v : xv) v *= 3.0f;
  Tensor x({4101}), y({4101}), slot1({4101}), slot2({4101}), slot3({4101}), want({4101});
  x.set(std::span<const float>(xv));
  y.set(std::span<const float>(xv));
  fill(s, {2500.0f}); // factor 1/50
  run(rt, [&] {
    rt.copy(x, slot1);
    rt.copy(slot1, slot2); // a copy of a copy: reads x too
    rt.copy(y, slot3);
    rt.clip_gradient(slot1, s, 1.0f, slot1); // from x
    rt.clip_gradient(slot2, s, 1.0f, slot2); // from x
    rt.clip_gradient(y, s, 1.0f, y);         // y in place
    rt.clip_gradient(slot3, s, 1.0f, slot3); // reads y, which the batch writes: runs it first
    rt.clip_gradient(x, s, 1.0f, want);      // direct, out of place
  });
  const auto hx = host(x), h1 = host(slot1), h2 = host(slot2), h3 = host(slot3), hy = host(y),
             hw = host(want);
  for (size_t j = 0; j < xv.size(); ++j) {
    CHECK(hx[j] == xv[j]); // the copies' source is not clipped
    CHECK(h1[j] == hw[j]);
    CHECK(h2[j] == hw[j]);
    CHECK(hy[j] == hw[j]);
    CHECK(h3[j] == hw[j]); // slot3 took y before y's clip
  }
}

// The executor's LINEAR, mult(x, W, y) then add(y, bias, y)
// (include/passes/execute.h:242-253): the product waits for the next call
// and takes the bias in its epilogue. The same bits as the product and the
// add run apart (an op in between launches the product first), with and
// without K splits, batched, and with a host read in between.
void linear_bias(hip::Runtime &rt) {
  struct Case {
    std::vector<uint32_t> x, w;
  };
  for (const Case &c : {Case{{6, 40, 24}, {24, 33}}, Case{{96, 2048}, {2048, 64}},
                        Case{{3, 16, 8}, {3, 8, 12}}, Case{{4, 32, 48}, {48, 48}}}) {
    const uint32_t N = c.w.back();
    Tensor x(c.x), w(c.w), bias({N}), bias2({1, N});
    size_t nx = 1, nw = 1;
    for (uint32_t d : c.x) nx *= d;
    for (uint32_t d : c.w) nw *= d;
    x.set(random_values(nx, 41));
    w.set(random_values(nw, 42));
    const auto bv = random_values(N, 43);
    bias.set(std::span<const float>(bv));
    bias2.set(std::span<const float>(bv));
    std::vector<uint32_t> ys = c.x;
    ys.back() = N;
    if (c.w.size() == 3) ys[0] = std::max(c.x[0], c.w[0]);
    Tensor y1(ys), y2(ys), y3(ys), z(ys), other(ys);
    other.set(std::vector<float>(y1.numel(), 0.5f));
    std::vector<float> mid;
    run(rt, [&] {
      rt.mult(x, w, y1);
      rt.add(y1, bias, y1); // the product's epilogue
      rt.mult(x, w, y2);    // (the cached product: no launch)
      rt.mult(x, w, y3);
      rt.copy(y3, z);       // launches the product first
      rt.add(y3, bias2, y3); // apart
    });
    const auto h1 = host(y1), h3 = host(y3), hz = host(z);
    for (size_t i = 0; i < h1.size(); ++i) {
      CHECK(h1[i] == h3[i]);
      CHECK(hz[i] + bv[i % N] == h3[i]); // z: the product before the add
    }
    // a host read between the product and the add; an add of a full tensor
    Tensor y4(ys), y5(ys);
    run(rt, [&] {
      rt.mult(x, w, y4);
      mid = host(y4);
      rt.add(y4, bias, y4);
      rt.mult(x, w, y5);
      rt.add(y5, other, y5); // not a bias row: the ordinary add
    });
    const auto h4 = host(y4), h5 = host(y5);
    for (size_t i = 0; i < h4.size(); ++i) {
      CHECK(h4[i] == h1[i]);
      CHECK(h5[i] == mid[i] + 0.5f);
    }
    // GELU of the product with its bias (execute.h:477-482): one launch
    // writes the pre-activation and GELU of it, the same bits as apart; a
    // GELU into the product's own input stays apart
    Tensor ya(ys), yb(ys), ga(ys), gb(ys), yc(ys), held(ys);
    Tensor xc(c.x);
    run(rt, [&] {
      rt.mult(x, w, ya);
      rt.add(ya, bias, ya);
      rt.GELU(ya, ga);      // fused
      rt.mult(x, w, yb);
      rt.add(yb, bias, yb);
      rt.copy(yb, held);    // launches the product with its bias
      rt.GELU(yb, gb);      // apart
      rt.copy(x, xc);
    });
    if (ys == c.x) {
      run(rt, [&] {
        rt.mult(xc, w, yc);
        rt.add(yc, bias, yc);
        rt.GELU(yc, xc); // writes the product's input: not fused
      });
      const auto hyc = host(yc), hxc = host(xc), hgb = host(gb);
      for (size_t i = 0; i < hyc.size(); ++i) {
        CHECK(hyc[i] == h1[i]);
        CHECK(hxc[i] == hgb[i]);
      }
    }
    const auto hya = host(ya), hyb = host(yb), hga = host(ga), hgb = host(gb);
    for (size_t i = 0; i < hya.size(); ++i) {
      CHECK(hya[i] == h1[i]);
      CHECK(hyb[i] == h1[i]);
      CHECK(hga[i] == hgb[i]);
    }
  }
}

// A per-entry weight gradient as the executor forms it
// (MULT_RHS_DERIVATIVE, include/passes/execute.h:210-232): transpose the
// input, a batched product with the output gradient, then sum_to_shape over
// the batch. The product is kept pending and the sum runs as one product
// over K * entries; the product's own values are still there when read.
void deferred_products(hip::Runtime &rt) {
  constexpr uint32_t B = 3, T = 5, I = 4, O = 6;
  const std::vector<float> xv = random_values(B * T * I, 21), gv = random_values(B * T * O, 22);
  Tensor x({B, T, I}), g({B, T, O}), xt({B, I, T}), prod({B, I, O}), w({I, O}), w1({1, I, O});
  x.set(std::span<const float>(xv));
  g.set(std::span<const float>(gv));
  auto per = [&](size_t b, size_t i, size_t o) {
    double e = 0;
    for (size_t t = 0; t < T; ++t) e += double(xv[(b * T + t) * I + i]) * gv[(b * T + t) * O + o];
    return e;
  };
  auto check_sum = [&](const Tensor &t) {
    const auto got = host(t);
    for (size_t i = 0; i < I; ++i)
      for (size_t o = 0; o < O; ++o) {
        double e = 0;
        for (size_t b = 0; b < B; ++b) e += per(b, i, o);
        CHECK_NEAR(got[i * O + o], e, 1e-5);
      }
  };
  // 1. summed twice (rank-dropping and rank-keeping targets), then the
  // batched values read after the sources changed
  Tensor zeros_x({B, T, I}), zeros_g({B, T, O});
  zeros_x.set(std::vector<float>(B * T * I, 0.0f));
  zeros_g.set(std::vector<float>(B * T * O, 0.0f));
  run(rt, [&] {
    rt.transpose(x, xt);
    rt.mult(xt, g, prod);
    rt.sum_to_shape(prod, std::vector<uint32_t>{I, O}, w);
    rt.sum_to_shape(prod, std::vector<uint32_t>{1, I, O}, w1);
    rt.copy(zeros_x, x); // the product must keep the old operands
    rt.copy(zeros_g, g);
  });
  check_sum(w);
  check_sum(w1);
  {
    const auto got = host(prod);
    for (size_t b = 0; b < B; ++b)
      for (size_t i = 0; i < I; ++i)
        for (size_t o = 0; o < O; ++o) CHECK_NEAR(got[(b * I + i) * O + o], per(b, i, o), 1e-5);
  }
  // 2. a pending product read by another kernel, then overwritten whole
  x.set(std::span<const float>(xv));
  g.set(std::span<const float>(gv));
  Tensor e({B, I, O}), other({B, I, O});
  other.set(std::vector<float>(B * I * O, 1.0f));
  run(rt, [&] {
    rt.transpose(x, xt);
    rt.mult(xt, g, prod);
    rt.exp(prod, e);
    rt.mult(xt, g, prod);
    rt.copy(other, prod); // the second product is dead
  });
  {
    const auto ge = host(e), gp = host(prod);
    for (size_t b = 0; b < B; ++b)
      for (size_t i = 0; i < I; ++i)
        for (size_t o = 0; o < O; ++o) {
          CHECK_NEAR(ge[(b * I + i) * O + o], std::exp(per(b, i, o)), 1e-4);
          CHECK(gp[(b * I + i) * O + o] == 1.0f);
        }
  }
  // 3. a partial sum (one of two batch dims) runs the batched product first
  Tensor x4({2, B, T, I}), g4({2, B, T, O}), xt4({2, B, I, T}), p4({2, B, I, O}), s4({B, I, O});
  std::vector<float> x4v(xv), g4v(gv);
  x4v.insert(x4v.end(), xv.begin(), xv.end());
  g4v.insert(g4v.end(), gv.begin(), gv.end());
  x4.set(std::span<const float>(x4v));
  g4.set(std::span<const float>(g4v));
  run(rt, [&] {
    rt.transpose(x4, xt4);
    rt.mult(xt4, g4, p4);
    rt.sum_to_shape(p4, std::vector<uint32_t>{B, I, O}, s4);
  });
  {
    const auto got = host(s4);
    for (size_t b = 0; b < B; ++b)
      for (size_t i = 0; i < I; ++i)
        for (size_t o = 0; o < O; ++o) CHECK_NEAR(got[(b * I + i) * O + o], 2 * per(b, i, o), 1e-5);
  }
}

void sqe(hip::Runtime &rt) {
  Tensor p({2, 3}), t({2, 3}), row({3}), o({2, 3}), ob({2, 3});
  fill(p, {1, -2, 3.5f, 0, 10, -7});
  fill(t, {4, -2, 1, 0.25f, -10, 7});
  fill(row, {1, 2, 3});
  run(rt, [&] {
    rt.sqe(p, t, o);
    rt.sqe(p, row, ob);
    rt.sqe(p, t, p); // in place: destination is the prediction
  });
  expect(o, {9, 0, 6.25f, 0.0625f, 400, 196});
  expect(ob, {0, 16, 0.25f, 1, 64, 100});
  expect(p, {9, 0, 6.25f, 0.0625f, 400, 196});
  // a larger random case against sub-then-square on the host
  Tensor x({6144, 384}), y({6144, 384}), z({6144, 384});
  const auto xv = random_values(x.numel(), 31), yv = random_values(y.numel(), 32);
  x.set(xv);
  y.set(yv);
  run(rt, [&] { rt.sqe(x, y, z); });
  const auto got = host(z);
  size_t bad = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const float d = xv[i] - yv[i];
    bad += std::fabs(got[i] - d * d) > 1e-5f + 1e-4f * d * d;
  }
  CHECK(bad == 0);
}

void memory_pool_reuse(hip::Runtime &) {
  const auto before = hip::memory_stats();
  for (int i = 0; i < 10; ++i) {
    Tensor t({256, 1024});
    t.get_storage()->fill(1.0f);
  }
  const auto after = hip::memory_stats();
  CHECK(after.device_allocations - before.device_allocations <= 1);
  CHECK(after.in_use_bytes == before.in_use_bytes);
}

void storage_semantics(hip::Runtime &) {
  Tensor a = Tensor::from_values({{1, 2}, {3, 4}});
  Tensor b = a.clone();
  CHECK(a == b);
  b.set(9.0f, 1, 1);
  CHECK(!(a == b));
  CHECK(b.get(1, 1) == 9.0f);
  CHECK(a.get(1, 0) == 3.0f);
  std::vector<float> big(4);
  CHECK_THROWS(std::out_of_range, a.get_storage()->read(std::span<float>(big.data(), 3), 2));
  const std::vector<uint32_t> flat = {4};
  Tensor v = a.view(flat);
  CHECK(v.get_storage() == a.get_storage());
  CHECK(a.get_storage()->ref_count == 2);
  Tensor z = Tensor::from_zeros({3, 5});
  for (float x : host(z)) CHECK(x == 0.0f);
}

} // namespace

int main(int argc, char **argv) {
  if (argc > 1 && std::strcmp(argv[1], "--no-device") == 0) {
    harness::run("init_without_device_throws", [] {
      CHECK_THROWS(std::runtime_error, hip::init(0));
      CHECK(!hip::initialised());
      CHECK_THROWS(std::logic_error, hip::Runtime());
    });
    return harness::failures();
  }
  hip::init(0);
  {
    hip::Runtime rt;
    harness::run("lifecycle", [&] { lifecycle(rt); });
    harness::run("binary_and_chained_operations", [&] { binary_and_chained(rt); });
    harness::run("broadcasting", [&] { broadcasting(rt); });
    harness::run("scalar_operations", [&] { scalar_ops(rt); });
    harness::run("unary_operations", [&] { unary_ops(rt); });
    harness::run("rms_and_rms_norm", [&] { rms_and_rms_norm(rt); });
    harness::run("gelu", [&] { gelu(rt); });
    harness::run("matmul", [&] { matmul(rt); });
    harness::run("tiled_identity_matmul", [&] { tiled_identity_matmul(rt); });
    harness::run("reductions_and_transpose", [&] { reductions_and_transpose(rt); });
    harness::run("sum_to_shape_multiple_dimensions", [&] { sum_to_shape_multi(rt); });
    harness::run("sum_to_shape_leading_singletons", [&] { sum_to_shape_leading_singletons(rt); });
    harness::run("softmax", [&] { softmax(rt); });
    harness::run("cross_entropy", [&] { cross_entropy(rt); });
    harness::run("cross_entropy_bad_target", [&] { cross_entropy_bad_target(rt); });
    harness::run("argmax", [&] { argmax(rt); });
    harness::run("embedding_lookup", [&] { embedding_lookup(rt); });
    harness::run("scatter_index", [&] { scatter_index(rt); });
    harness::run("scatter_add_rows", [&] { scatter_add_rows(rt); });
    harness::run("gradient_clipping", [&] { gradient_clipping(rt); });
    harness::run("adamw", [&] { adamw(rt); });
    harness::run("validation", [&] { validation(rt); });
    harness::run("max_to_shape_alias", [&] { max_to_shape_alias(rt); });
    harness::run("in_place_and_split_merge", [&] { in_place_and_split_merge(rt); });
    harness::run("batched_matmul_layouts", [&] { batched_matmul_layouts(rt); });
    harness::run("graph_mode", [&] { graph_mode(rt); });
    harness::run("graph_mode_scratch_is_not_reused_within_a_capture",
                 [&] { graph_mode_scratch_is_not_reused_within_a_capture(rt); });
    harness::run("sqe", [&] { sqe(rt); });
    harness::run("deferred_views", [&] { deferred_views(rt); });
    harness::run("deferred_products", [&] { deferred_products(rt); });
    harness::run("repeated_results", [&] { repeated_results(rt); });
    harness::run("collected_norms", [&] { collected_norms(rt); });
    harness::run("collected_adamw", [&] { collected_adamw(rt); });
    harness::run("batched_clips", [&] { batched_clips(rt); });
    harness::run("linear_bias", [&] { linear_bias(rt); });
    harness::run("aborted_capture_forgets_results",
                 [&] { aborted_capture_forgets_results(rt); });
    harness::run("memory_pool_reuse", [&] { memory_pool_reuse(rt); });
    harness::run("storage_semantics", [&] { storage_semantics(rt); });
  }
  harness::run("cleanup_is_idempotent", cleanup_is_idempotent);
  hip::shutdown();
  std::printf("%s\n", harness::failures() ? "SOME TESTS FAILED" : "all hip::Runtime tests passed");
  return harness::failures();
}
