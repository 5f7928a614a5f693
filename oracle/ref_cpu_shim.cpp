// C ABI over the reference CPU runtime -- TEST INFRASTRUCTURE ONLY.
//
// Compiled by oracle/Makefile together with the reference's own
// src/CPU/cpu.cpp (read in place from the reference tree, never copied)
// into oracle/_ref/libref_cpu.so. The tests use it to check the oracle's
// restatement against the real reference CPU runtime on random inputs,
// and bench.py may time it as the "reference" CPU baseline for the matmul.
// Only the rank-2 surface of cpu::Runtime exists (src/CPU/cpu.cpp:39-43).
#include "CPU/runtime.h"

#include <cstdint>
#include <span>
#include <vector>

namespace {
using Mat = RTensor<cpu::CPU, float>;

Mat make(const float *data, uint32_t rows, uint32_t cols) {
  Mat m({rows, cols});
  m.set(std::span<const float>(data, size_t(rows) * cols));
  return m;
}

void take(const Mat &m, float *out) {
  m.read(std::span<float>(out, m.numel()));
}

template <typename F>
int guarded(F &&f) {
  try {
    f();
    return 0;
  } catch (...) {
    return 1;
  }
}
} // namespace

extern "C" {

int ref_mult(const float *a, const float *b, float *c, uint32_t M, uint32_t K, uint32_t N) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat A = make(a, M, K), B = make(b, K, N), C({M, N});
    rt.mult(A, B, C);
    take(C, c);
  });
}

// op: 0 add, 1 sub, 2 hadamard, 3 divide. Rank-2 broadcasting as
// binary_transform supports it.
int ref_binary(int op, const float *a, uint32_t ar, uint32_t ac, const float *b, uint32_t br,
               uint32_t bc, float *out) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat A = make(a, ar, ac), B = make(b, br, bc);
    Mat O({std::max(ar, br), std::max(ac, bc)});
    if (op == 0) rt.add(A, B, O);
    else if (op == 1) rt.sub(A, B, O);
    else if (op == 2) rt.hadamard(A, B, O);
    else rt.divide(A, B, O);
    take(O, out);
  });
}

int ref_softmax(const float *x, float *out, uint32_t rows, uint32_t cols) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat X = make(x, rows, cols), O({rows, cols});
    rt.softmax(X, O);
    take(O, out);
  });
}

int ref_transpose(const float *a, float *out, uint32_t rows, uint32_t cols) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat A = make(a, rows, cols), O({cols, rows});
    rt.transpose(A, O);
    take(O, out);
  });
}

int ref_sum_to_shape(const float *a, uint32_t rows, uint32_t cols, float *out, uint32_t orows,
                     uint32_t ocols) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat A = make(a, rows, cols), O({orows, ocols});
    const std::vector<uint32_t> shape{orows, ocols};
    rt.sum_to_shape(A, shape, O);
    take(O, out);
  });
}

int ref_sum(const float *a, uint32_t rows, uint32_t cols, float *out) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat A = make(a, rows, cols), O({1});
    rt.sum(A, O);
    take(O, out);
  });
}

int ref_unary(int op, const float *a, float *out, uint32_t rows, uint32_t cols) {
  return guarded([&] {
    cpu::Runtime rt;
    Mat A = make(a, rows, cols), O({rows, cols});
    if (op == 0) rt.sqrt(A, O);
    else rt.sigmoid(A, O);
    take(O, out);
  });
}

int ref_argmax(const float *a, uint32_t rows, uint32_t cols, uint32_t *out) {
  return guarded([&] {
    Mat A = make(a, rows, cols);
    Mat idx = cpu::argmax(A);
    float v = 0.0f;
    idx.read(std::span<float>(&v, 1));
    *out = uint32_t(v);
  });
}

} // extern "C"
