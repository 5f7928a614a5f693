// CPU oracle for the TempLit runtime hot path -- TEST INFRASTRUCTURE ONLY.
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
// this library, and only as the checker (or the timed CPU baseline). See
// oracle.h for what it restates; each function cites the reference lines.
// Single-threaded fp32 throughout, like the reference CPU runtime
// (src/CPU/cpu.cpp has no threading).
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// Portable synthetic data: SplitMix64 stream, Box-Muller in double.
// ---------------------------------------------------------------------------
struct SplitMix64 {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform_open() { // (0, 1]
    return (double((next() >> 11) + 1)) * (1.0 / 9007199254740992.0);
  }
};

// Row-major decode of a linear index into per-dimension coordinates and the
// dot product with a stride vector (the index loop of math.metal:401-426).
inline size_t strided_offset(size_t index, uint32_t ndim, const uint32_t *shape,
                             const uint32_t *strides) {
  size_t off = 0;
  for (int d = int(ndim) - 1; d >= 0; --d) {
    const size_t c = index % shape[d];
    index /= shape[d];
    off += c * strides[d];
  }
  return off;
}

inline size_t product(const uint32_t *shape, uint32_t ndim) {
  size_t n = 1;
  for (uint32_t i = 0; i < ndim; ++i) n *= shape[i];
  return n;
}

// GELU as the Metal kernels evaluate it (math.metal:821-855): the forward
// constant is sqrt(2.0f / 3.14159265f) in fp32, the derivative's is the
// literal 0.7978845608f.
inline float gelu_fwd(float x) {
  const float a = std::sqrt(2.0f / 3.14159265f);
  return 0.5f * x * (1.0f + std::tanh(a * (x + 0.044715f * x * x * x)));
}

inline float gelu_grad(float x) {
  constexpr float a = 0.7978845608f;
  constexpr float b = 0.044715f;
  const float x2 = x * x;
  const float u = a * (x + b * x2 * x);
  const float t = std::tanh(u);
  return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * a * (1.0f + 3.0f * b * x2);
}

// i-k-j product into a zeroed C (src/CPU/cpu.cpp:245-274), row-major,
// with leading dimensions.
void mm_ikj(const float *a, const float *b, float *c, size_t M, size_t K, size_t N) {
  std::fill(c, c + M * N, 0.0f);
  for (size_t i = 0; i < M; ++i) {
    for (size_t k = 0; k < K; ++k) {
      const float value = a[i * K + k];
      float *crow = c + i * N;
      const float *brow = b + k * N;
      for (size_t j = 0; j < N; ++j) crow[j] += value * brow[j];
    }
  }
}

void transpose2(const float *a, float *out, size_t rows, size_t cols) {
  for (size_t i = 0; i < rows; ++i)
    for (size_t j = 0; j < cols; ++j) out[j * rows + i] = a[i * cols + j];
}

// Reduction of one 256-wide threadgroup exactly as the Metal kernel does it
// (math.metal:955-983: stride-halving tree over squares).
float tree256_squares(const float *g, size_t n) {
  float partial[256];
  for (size_t i = 0; i < 256; ++i) {
    const float v = i < n ? g[i] : 0.0f;
    partial[i] = v * v;
  }
  for (size_t stride = 128; stride > 0; stride /= 2)
    for (size_t i = 0; i < stride; ++i) partial[i] += partial[i + stride];
  return partial[0];
}

} // namespace

extern "C" {

void orc_fill_normal(float *out, size_t n, uint64_t seed, float mean, float std) {
  SplitMix64 rng{seed};
  const double two_pi = 6.283185307179586;
  for (size_t i = 0; i < n; i += 2) {
    const double u1 = rng.uniform_open();
    const double u2 = rng.uniform_open();
    const double r = std::sqrt(-2.0 * std::log(u1));
    out[i] = float(mean + std * r * std::cos(two_pi * u2));
    if (i + 1 < n) out[i + 1] = float(mean + std * r * std::sin(two_pi * u2));
  }
}

void orc_fill_uniform_u32(uint32_t *out, size_t n, uint64_t seed, uint32_t bound) {
  SplitMix64 rng{seed};
  for (size_t i = 0; i < n; ++i) out[i] = uint32_t(rng.next() % bound);
}

// Broadcast binary ops: rank-N restatement of binary_transform
// (src/CPU/cpu.cpp:37-147) with the index decode of the Metal kernels
// add/sub/hadamard/divide (math.metal:401-510).
void orc_binary(int op, const float *a, const float *b, float *out, uint32_t ndim,
                const uint32_t *out_shape, const uint32_t *stride_a,
                const uint32_t *stride_b) {
  const size_t n = product(out_shape, ndim);
  std::vector<float> tmp(n);
  for (size_t i = 0; i < n; ++i) {
    const float x = a[strided_offset(i, ndim, out_shape, stride_a)];
    const float y = b[strided_offset(i, ndim, out_shape, stride_b)];
    float r = 0.0f;
    switch (op) {
    case ORC_ADD: r = x + y; break;
    case ORC_SUB: r = x - y; break;
    case ORC_MUL: r = x * y; break;
    default: r = x / y; break;
    }
    tmp[i] = r;
  }
  std::memcpy(out, tmp.data(), n * sizeof(float));
}

// Unary ops: sqrt/exp/sigmoid (cpu.cpp:209-235, math.metal:519-548),
// GELU/GELU_derivative (math.metal:821-855), copy (math.metal:1045-1050).
void orc_unary(int op, const float *a, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float x = a[i];
    float r = x;
    switch (op) {
    case ORC_SQRT: r = std::sqrt(x); break;
    case ORC_EXP: r = std::exp(x); break;
    case ORC_SIGMOID: r = 1.0f / (1.0f + std::exp(-x)); break;
    case ORC_GELU: r = gelu_fwd(x); break;
    case ORC_GELU_DERIVATIVE: r = gelu_grad(x); break;
    default: break;
    }
    out[i] = r;
  }
}

// add_scalar / divide_scalar / pow_scalar (math.metal:427-434, 511-534).
void orc_scalar(int op, const float *a, float s, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    switch (op) {
    case ORC_ADD_SCALAR: out[i] = a[i] + s; break;
    case ORC_DIVIDE_SCALAR: out[i] = a[i] / s; break;
    default: out[i] = std::pow(a[i], s); break;
    }
  }
}

// transpose through swapped input strides (cpu.cpp:365-401, math.metal:566-584).
void orc_transpose(const float *a, float *out, uint32_t ndim, const uint32_t *out_shape,
                   const uint32_t *in_strides) {
  const size_t n = product(out_shape, ndim);
  std::vector<float> tmp(n);
  for (size_t i = 0; i < n; ++i) tmp[i] = a[strided_offset(i, ndim, out_shape, in_strides)];
  std::memcpy(out, tmp.data(), n * sizeof(float));
}

// Batched broadcasting matmul (runtime.cpp:375-505 semantics) with the
// i-k-j loop of cpu.cpp:245-274 per batch element. C is contiguous.
void orc_matmul(const float *a, const float *b, float *c, uint32_t M, uint32_t K,
                uint32_t N, uint32_t batch_ndim, const uint32_t *batch_shape,
                const uint32_t *batch_stride_a, const uint32_t *batch_stride_b) {
  const size_t batch = batch_ndim ? product(batch_shape, batch_ndim) : 1;
  std::vector<float> tmp(size_t(M) * N);
  for (size_t z = 0; z < batch; ++z) {
    const size_t oa = batch_ndim ? strided_offset(z, batch_ndim, batch_shape, batch_stride_a) : 0;
    const size_t ob = batch_ndim ? strided_offset(z, batch_ndim, batch_shape, batch_stride_b) : 0;
    mm_ikj(a + oa, b + ob, tmp.data(), M, K, N);
    std::memcpy(c + z * size_t(M) * N, tmp.data(), tmp.size() * sizeof(float));
  }
}

// Serial sum (math.metal:549-564; cpu.cpp reduce 149-160).
float orc_sum(const float *a, size_t n) {
  float total = 0.0f;
  for (size_t i = 0; i < n; ++i) total += a[i];
  return total;
}

// sum_to_shape / max_to_shape over a rank-aligned output shape
// (runtime.cpp:595-739; math.metal:618-714): one output element at a time,
// reduced coordinates visited in row-major order (last reduced dim fastest).
static void reduce_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                            const uint32_t *out_shape, bool is_max) {
  std::vector<uint32_t> a_strides(ndim);
  size_t s = 1;
  for (int d = int(ndim) - 1; d >= 0; --d) {
    a_strides[d] = uint32_t(s);
    s *= a_shape[d];
  }
  std::vector<uint32_t> red_dims, red_sizes;
  for (uint32_t d = 0; d < ndim; ++d)
    if (a_shape[d] != out_shape[d]) {
      red_dims.push_back(d);
      red_sizes.push_back(a_shape[d]);
    }
  size_t red_count = 1;
  for (uint32_t r : red_sizes) red_count *= r;
  const size_t n_out = product(out_shape, ndim);
  for (size_t o = 0; o < n_out; ++o) {
    const size_t base = strided_offset(o, ndim, out_shape, a_strides.data());
    float acc = is_max ? -std::numeric_limits<float>::infinity() : 0.0f;
    for (size_t i = 0; i < red_count; ++i) {
      size_t rem = i, off = 0;
      for (int j = int(red_dims.size()) - 1; j >= 0; --j) {
        off += (rem % red_sizes[j]) * a_strides[red_dims[j]];
        rem /= red_sizes[j];
      }
      const float v = a[base + off];
      if (is_max) {
        if (v > acc) acc = v;
      } else {
        acc += v;
      }
    }
    out[o] = acc;
  }
}

void orc_sum_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                      const uint32_t *out_shape) {
  reduce_to_shape(a, out, ndim, a_shape, out_shape, false);
}

void orc_max_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                      const uint32_t *out_shape) {
  reduce_to_shape(a, out, ndim, a_shape, out_shape, true);
}

// argmax: first index of the maximum (strict '>' from -INF,
// math.metal:715-777; cpu.cpp:528-532 max_element is also first-maximum).
uint32_t orc_argmax(const float *a, size_t n) {
  float best = -std::numeric_limits<float>::infinity();
  uint32_t index = 0;
  for (size_t i = 0; i < n; ++i)
    if (a[i] > best) {
      best = a[i];
      index = uint32_t(i);
    }
  return index;
}

// Top-k sampling, inference::sample_top_k (include/inference.h:14-43): the
// candidates (logit, token) are ordered by logit, descending (partial_sort
// with a.first > b.first; its order of equal logits is unspecified, here the
// lower token comes first), weights are std::exp((logit - maximum) /
// temperature) in fp32 (the exponential taken in double and rounded to fp32,
// the correctly rounded expf), and std::discrete_distribution picks one:
// libstdc++ normalises each weight by the double sum, takes partial sums,
// sets the last to 1.0 and returns the lower_bound of one
// generate_canonical<double, 53> draw. The EOS re-draw loop is
// inference::autoregression's (inference.h:80-84), bounded by max_draws.
void orc_sample_top_k(const float *logits, uint32_t rows, uint32_t vocab, uint32_t row_stride,
                      uint32_t top_k, float temperature, uint64_t seed, uint64_t counter,
                      const double *uniforms, uint32_t eos_token, int resample_eos,
                      uint32_t max_draws, uint32_t *tokens, uint32_t *draws) {
  const uint32_t k = std::min(std::max(top_k, 1u), vocab);
  std::vector<std::pair<float, uint32_t>> cand(vocab);
  std::vector<float> w(k);
  for (uint32_t r = 0; r < rows; ++r) {
    const float *row = logits + size_t(r) * row_stride;
    for (uint32_t t = 0; t < vocab; ++t) {
      const float x = row[t];
      cand[t] = {std::isnan(x) ? -std::numeric_limits<float>::infinity() : x, t};
    }
    std::sort(cand.begin(), cand.end(), [](const auto &a, const auto &b) {
      return a.first > b.first || (a.first == b.first && a.second < b.second);
    });
    const float maximum = cand[0].first;
    double total = 0.0;
    for (uint32_t i = 0; i < k; ++i) {
      w[i] = float(std::exp(double((cand[i].first - maximum) / temperature)));
      total += double(w[i]);
    }
    uint32_t token = 0, d = 0;
    for (; d < max_draws; ++d) {
      double u;
      if (uniforms) {
        u = uniforms[size_t(r) * max_draws + d];
      } else {
        SplitMix64 g{seed + (counter + uint64_t(r) * max_draws + d) * 0x9E3779B97F4A7C15ull};
        u = double(g.next() >> 11) * (1.0 / 9007199254740992.0);
      }
      uint32_t pick = k - 1;
      double c = 0.0;
      for (uint32_t i = 0; i + 1 < k; ++i) {
        c += double(w[i]) / total;
        if (c >= u) {
          pick = i;
          break;
        }
      }
      token = cand[pick].second;
      if (!(resample_eos && token == eos_token)) {
        ++d;
        break;
      }
    }
    tokens[r] = token;
    if (draws) draws[r] = std::min(d, max_draws);
  }
}

// softmax per row: max, shift, exp, serial sum, divide (cpu.cpp:501-519).
void orc_softmax(const float *x, float *out, size_t rows, uint32_t cols) {
  std::vector<float> e(cols);
  for (size_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    float m = std::numeric_limits<float>::lowest();
    for (uint32_t j = 0; j < cols; ++j) m = std::max(m, row[j]);
    float sum = 0.0f;
    for (uint32_t j = 0; j < cols; ++j) {
      e[j] = std::exp(row[j] - m);
      sum += e[j];
    }
    for (uint32_t j = 0; j < cols; ++j) out[r * cols + j] = e[j] / sum;
  }
}

// EXPR_SFTMX_DERIVATIVE (execute.h:291-308): d = g*y; s = sum(d);
// d = g - s; d = y*d.
void orc_softmax_backward(const float *g, const float *y, float *out, size_t rows,
                          uint32_t cols) {
  std::vector<float> d(cols);
  for (size_t r = 0; r < rows; ++r) {
    const float *gr = g + r * cols;
    const float *yr = y + r * cols;
    float s = 0.0f;
    for (uint32_t j = 0; j < cols; ++j) {
      d[j] = gr[j] * yr[j];
      s += d[j];
    }
    for (uint32_t j = 0; j < cols; ++j) out[r * cols + j] = yr[j] * (gr[j] - s);
  }
}

// cross_entropy_rows (math.metal:884-910).
void orc_cross_entropy_rows(const float *logits, const uint32_t *targets, float *losses,
                            size_t rows, uint32_t vocab) {
  for (size_t r = 0; r < rows; ++r) {
    const float *row = logits + r * vocab;
    const uint32_t t = targets[r];
    if (t >= vocab) {
      losses[r] = std::numeric_limits<float>::infinity();
      continue;
    }
    float m = -std::numeric_limits<float>::infinity();
    for (uint32_t j = 0; j < vocab; ++j) m = std::max(m, row[j]);
    float s = 0.0f;
    for (uint32_t j = 0; j < vocab; ++j) s += std::exp(row[j] - m);
    losses[r] = m + std::log(s) - row[t];
  }
}

// cross_entropy_rows_backward (math.metal:912-953).
void orc_cross_entropy_rows_backward(const float *logits, const uint32_t *targets,
                                     float *grad, size_t rows, uint32_t vocab) {
  for (size_t r = 0; r < rows; ++r) {
    const float *row = logits + r * vocab;
    float *gr = grad + r * vocab;
    const uint32_t t = targets[r];
    if (t >= vocab) {
      for (uint32_t j = 0; j < vocab; ++j) gr[j] = std::numeric_limits<float>::infinity();
      continue;
    }
    float m = -std::numeric_limits<float>::infinity();
    for (uint32_t j = 0; j < vocab; ++j) m = std::max(m, row[j]);
    float s = 0.0f;
    for (uint32_t j = 0; j < vocab; ++j) s += std::exp(row[j] - m);
    for (uint32_t j = 0; j < vocab; ++j) gr[j] = std::exp(row[j] - m) / s;
    gr[t] -= 1.0f;
  }
}

// RMS (runtime.cpp:1031-1052): hadamard(x,x) -> sum(last) -> /D -> +eps -> sqrt.
void orc_rms(const float *x, float *rms, size_t rows, uint32_t cols, float eps) {
  const float hidden = float(cols);
  for (size_t r = 0; r < rows; ++r) {
    float s = 0.0f;
    for (uint32_t j = 0; j < cols; ++j) {
      const float v = x[r * cols + j];
      s += v * v;
    }
    s = s / hidden;
    s = s + eps;
    rms[r] = std::sqrt(s);
  }
}

// RMSNorm (runtime.cpp:1060-1072): y = x / rms, optional gain extension.
void orc_rms_norm(const float *x, const float *gain, float *y, float *rms_out, size_t rows,
                  uint32_t cols, float eps) {
  std::vector<float> rms(rows);
  orc_rms(x, rms.data(), rows, cols, eps);
  for (size_t r = 0; r < rows; ++r) {
    for (uint32_t j = 0; j < cols; ++j) {
      float v = x[r * cols + j] / rms[r];
      if (gain) v = v * gain[j];
      y[r * cols + j] = v;
    }
    if (rms_out) rms_out[r] = rms[r];
  }
}

// EXPR_RMSN_DERIVATIVE (execute.h:330-356): rms = RMS(x); d = g*y;
// m = sum(d)/D; d = y*m; d = g - d; d = d/rms. With a gain, g is first
// multiplied by gain and y is the un-gained x/rms; grad_gain = sum_r g*n.
void orc_rms_norm_backward(const float *g, const float *x, const float *gain, float *dx,
                           float *grad_gain, size_t rows, uint32_t cols, float eps) {
  std::vector<float> rms(rows), n(cols), gy(cols);
  orc_rms(x, rms.data(), rows, cols, eps);
  if (grad_gain) std::fill(grad_gain, grad_gain + cols, 0.0f);
  const float hidden = float(cols);
  for (size_t r = 0; r < rows; ++r) {
    float s = 0.0f;
    for (uint32_t j = 0; j < cols; ++j) {
      n[j] = x[r * cols + j] / rms[r];
      gy[j] = gain ? g[r * cols + j] * gain[j] : g[r * cols + j];
      if (grad_gain) grad_gain[j] += g[r * cols + j] * n[j];
      s += gy[j] * n[j];
    }
    const float m = s / hidden;
    for (uint32_t j = 0; j < cols; ++j) dx[r * cols + j] = (gy[j] - n[j] * m) / rms[r];
  }
}

// embedding_lookup (math.metal:778-793).
void orc_embedding_lookup(const float *w, uint32_t dim, const uint32_t *ids, size_t n_ids,
                          float *out) {
  for (size_t i = 0; i < n_ids; ++i)
    std::memcpy(out + i * dim, w + size_t(ids[i]) * dim, dim * sizeof(float));
}

// scatter_add_rows (math.metal:794-820) in increasing i.
void orc_scatter_add_rows(const float *values, const uint32_t *ids, size_t n_ids,
                          uint32_t dim, float *dst) {
  for (size_t i = 0; i < n_ids; ++i)
    for (uint32_t j = 0; j < dim; ++j) dst[size_t(ids[i]) * dim + j] += values[i * dim + j];
}

// accumulate_gradient_squared_norm (math.metal:955-983): 256-wide tree per
// threadgroup, threadgroup partials added in order.
void orc_accumulate_gradient_squared_norm(const float *g, size_t n, float *squared_norm) {
  for (size_t base = 0; base < n; base += 256)
    *squared_norm += tree256_squares(g + base, std::min<size_t>(256, n - base));
}

// clip_gradient (math.metal:985-1006).
void orc_clip_gradient(const float *g, const float *squared_norm, float max_norm, float *out,
                       size_t n) {
  const float scale =
      std::min(1.0f, max_norm * (1.0f / std::sqrt(std::max(*squared_norm, 1e-12f))));
  for (size_t i = 0; i < n; ++i) out[i] = g[i] * scale;
}

// adamW (math.metal:1008-1043).
void orc_adamw(const float *param, const float *grad, float *out, float *m1, float *m2,
               float beta1, float beta2, float decay, float lr, float eps, uint32_t step,
               size_t n) {
  const float c1 = 1.0f - std::pow(beta1, float(step));
  const float c2 = 1.0f - std::pow(beta2, float(step));
  for (size_t i = 0; i < n; ++i) {
    const float g = grad[i];
    m1[i] = beta1 * m1[i] + (1.0f - beta1) * g;
    m2[i] = beta2 * m2[i] + (1.0f - beta2) * g * g;
    out[i] = param[i] * decay - lr * (m1[i] / c1) / (std::sqrt(m2[i] / c2) + eps);
  }
}

// Attention forward as the reference chain computes it
// (include/nn/multi_head.h:37-52): S = Q.K^T (via transpose + i-k-j mult),
// S / sqrt(D), + causal mask (include/nn/attention.h:9-22), softmax, P.V.
// q,k,v,o: [B,H,T,D]; probs: [B,H,T,T] (kept for the backward).
void orc_attention_forward(const float *q, const float *k, const float *v, float *o,
                           float *probs, uint32_t B, uint32_t H, uint32_t T, uint32_t D,
                           int causal) {
  const float root = std::sqrt(float(D));
  std::vector<float> kt(size_t(D) * T), s(size_t(T) * T);
  for (size_t bh = 0; bh < size_t(B) * H; ++bh) {
    const float *qb = q + bh * T * D, *kb = k + bh * T * D, *vb = v + bh * T * D;
    transpose2(kb, kt.data(), T, D);
    mm_ikj(qb, kt.data(), s.data(), T, D, T);
    for (uint32_t i = 0; i < T; ++i)
      for (uint32_t j = 0; j < T; ++j) {
        float x = s[size_t(i) * T + j] / root;
        if (causal && j > i) x = x + -std::numeric_limits<float>::infinity();
        else x = x + 0.0f;
        s[size_t(i) * T + j] = x;
      }
    float *pb = probs + bh * T * T;
    orc_softmax(s.data(), pb, T, T);
    mm_ikj(pb, vb, o + bh * T * D, T, T, D);
  }
}

// Backward of the same chain as the reference autograd composes it:
// dP = dO.V^T, dV = P^T.dO, dS = softmax'(dP, P) (execute.h:291-308),
// divide' = dS / sqrt(D), dQ = dS.K, dK = dS^T.Q.
void orc_attention_backward(const float *q, const float *k, const float *v,
                            const float *probs, const float *dout, float *dq, float *dk,
                            float *dv, uint32_t B, uint32_t H, uint32_t T, uint32_t D) {
  const float root = std::sqrt(float(D));
  std::vector<float> vt(size_t(D) * T), dp(size_t(T) * T), pt(size_t(T) * T),
      ds(size_t(T) * T), dst(size_t(T) * T);
  for (size_t bh = 0; bh < size_t(B) * H; ++bh) {
    const size_t o1 = bh * T * D, o2 = bh * T * T;
    transpose2(v + o1, vt.data(), T, D);
    mm_ikj(dout + o1, vt.data(), dp.data(), T, D, T);
    transpose2(probs + o2, pt.data(), T, T);
    mm_ikj(pt.data(), dout + o1, dv + o1, T, T, D);
    orc_softmax_backward(dp.data(), probs + o2, ds.data(), T, T);
    for (auto &x : ds) x = x / root;
    mm_ikj(ds.data(), k + o1, dq + o1, T, T, D);
    transpose2(ds.data(), dst.data(), T, T);
    mm_ikj(dst.data(), q + o1, dk + o1, T, T, D);
  }
}

} // extern "C"
