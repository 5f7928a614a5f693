// GPT training-step program over the C-ABI of libtemplit_hip.so.
//
// The reference runs this model through passes::Compiled
// (include/passes/compile.h:148-258): ~1,269 runtime calls per step, every
// op writing a fresh temporary, the backward re-evaluating shared gradient
// expressions, explicit transposes before every matmul derivative, and 52
// clip + 52 AdamW launches. Here the same mathematics is a fixed list of
// ~170 fused launches on one stream:
//   forward   embed(+pos) | per layer: RMSNorm, Q/K/V GEMMs storing the
//             [B,H,T,64] head layout, fused causal attention, O GEMM
//             (+bias +residual), RMSNorm, W1 GEMM (+bias, GELU), W2 GEMM
//             (+bias +residual) | RMSNorm, vocab GEMM, fused CE fwd+bwd
//   backward  transposed-operand GEMMs (no materialised transposes),
//             GELU' fused into the dG GEMM epilogue, fused RMSNorm',
//             attention backward, split-K weight gradients that also emit
//             the bias gradients
//   step      one multi-tensor squared norm, one multi-tensor clip+AdamW.
// Every buffer is allocated once in tlg_create (lifetime planned by hand:
// activations kept for the backward, one shared scratch set), so the whole
// step can be captured as a hipGraph and replayed.
#include "templit_gpt.h"
#include "templit_hip.h"

#include "model_utils/Dataset.h"
#include "model_utils/archive.h"
#include "model_utils/loader.h"

#include <algorithm>
#include <array>
#include <span>
#include <cmath>
#include <cstring>
#include <fstream>
#include <new>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

struct Tensor {
  float *ptr = nullptr;
  size_t size = 0;
};

constexpr uint32_t kHeadDim = 64;
constexpr float kRmsEps = 1e-6f; // src/my_metal/runtime.cpp:1044
constexpr size_t kAlign = 64;    // floats: every tensor starts 256-byte aligned
constexpr int kInvalidValue = 1; // hipErrorInvalidValue
// EOS re-draws per sampled token before the last draw stands (the reference
// draws until a non-EOS token comes, inference.h:80-84)
constexpr uint32_t kMaxSampleDraws = 1024;

struct Program {
  tlg_config cfg{};
  void *stream = nullptr;
  size_t R = 0; // rows = B*T

  // parameters / gradients / moments: one allocation each, same offsets
  std::vector<size_t> offset, size;
  size_t padded_total = 0, total = 0;
  float *params = nullptr, *grads = nullptr, *m1 = nullptr, *m2 = nullptr;
  // device tables for the multi-tensor kernels
  void *tab_params = nullptr, *tab_grads = nullptr, *tab_m1 = nullptr, *tab_m2 = nullptr;
  uint64_t *tab_sizes = nullptr;
  uint32_t *steps = nullptr;
  // optimiser scalars (device): beta1, beta2, decay, lr
  float *scalars = nullptr;
  float eps = 1e-8f, weight_decay = 0.01f, lr = 1e-3f;
  float *norm_partials = nullptr, *sqnorm = nullptr;

  // io
  uint32_t *tokens = nullptr, *targets = nullptr;
  float *losses = nullptr, *logits = nullptr, *dlogits = nullptr;
  uint32_t *argmax_out = nullptr;

  // activations (per layer) and scratch
  std::vector<float *> x;        // L+1 residual-stream inputs [R,D]
  std::vector<float *> n1, q, k, v, o, lse, x_mid, n2, u, g;
  float *nf = nullptr;
  float *dx = nullptr, *tmp = nullptr, *dgf = nullptr, *dq = nullptr, *dk = nullptr,
        *dv = nullptr, *delta = nullptr, *workspace = nullptr;
  size_t workspace_elems = 0;

  // Weight gradients run on a second stream, concurrently with the chain of
  // input gradients; fork/join events order the two (a recorded graph keeps
  // them as dependencies). While profiling everything runs on `stream`, so
  // kernel durations are measured in isolation.
  void *side = nullptr;
  float *workspace_side = nullptr;
  bool two_streams = true; // see auto_two_streams
  std::vector<void *> sync; // 2 + 8 per layer, see backward()

  std::vector<void *> allocations;
  void *graph = nullptr;

  // profiling (eager steps only): event pairs around GEMM / attention launches
  bool profiling = false;
  std::vector<void *> events;
  size_t next_event = 0;
  std::vector<std::pair<void *, void *>> gemm_spans, attn_spans;
  double gemm_flops = 0.0, gemm_bytes = 0.0;
  std::vector<tlh_gemm_desc> gemm_descs; // the profiled step's GEMMs, in launch order

  // K-contiguous copies of the weight matrices ([out, in], at the weights'
  // own offsets) for the forward products, rebuilt from the weights at the
  // start of every forward by one tlh_transpose_multi launch; see
  // auto_forward_copies.
  float *wt = nullptr;
  void *wt_jobs = nullptr;
  uint32_t wt_count = 0, wt_tiles = 0;
  bool forward_copies = false;

  float *P(uint32_t i) const { return params + offset[i]; }
  float *PT(uint32_t i) const { return wt + offset[i]; }
  float *G(uint32_t i) const { return grads + offset[i]; }
};

int alloc(Program &p, void **ptr, size_t bytes) {
  const int st = tlh_malloc(ptr, bytes < 256 ? 256 : bytes);
  if (st == 0) p.allocations.push_back(*ptr);
  return st;
}

int allocf(Program &p, float **ptr, size_t elems) {
  return alloc(p, reinterpret_cast<void **>(ptr), elems * sizeof(float));
}

// Parameter shapes in canonical order.
void layout(Program &p) {
  const size_t V = p.cfg.vocab, T = p.cfg.seq, D = p.cfg.dim, F = p.cfg.ffn;
  std::vector<size_t> sizes = {V * D, T * D};
  for (uint32_t l = 0; l < p.cfg.layers; ++l) {
    const size_t layer[12] = {D * D, D, D * D, D, D * D, D, D * D, D, D * F, F, F * D, D};
    sizes.insert(sizes.end(), layer, layer + 12);
  }
  sizes.push_back(D * V);
  sizes.push_back(V);
  size_t off = 0;
  p.total = 0;
  for (size_t s : sizes) {
    p.offset.push_back(off);
    p.size.push_back(s);
    off += (s + kAlign - 1) / kAlign * kAlign;
    p.total += s;
  }
  p.padded_total = off;
}

tlh_gemm_desc desc(const float *a, const float *b, float *c, int m, int n, int k, bool ta,
                   bool tb) {
  tlh_gemm_desc d;
  std::memset(&d, 0, sizeof(d));
  d.a = a;
  d.b = b;
  d.c = c;
  d.m = m;
  d.n = n;
  d.k = k;
  d.trans_a = ta;
  d.trans_b = tb;
  d.lda = ta ? m : k;
  d.ldb = tb ? k : n;
  d.ldc = n;
  return d;
}

// The forward product rows x weight w ([k, n]): on the K-contiguous copy
// (B transposed) when the program keeps copies, else on the weight itself.
tlh_gemm_desc wdesc(const Program &p, bool copies, const float *a, uint32_t w, float *c, int m,
                    int n, int k) {
  return copies ? desc(a, p.PT(w), c, m, n, k, false, true)
                : desc(a, p.P(w), c, m, n, k, false, false);
}

#define TRY(x)                                                                                 \
  do {                                                                                         \
    const int st_ = (x);                                                                       \
    if (st_) return st_;                                                                       \
  } while (0)

void *event(Program &p) {
  if (p.next_event == p.events.size()) {
    void *e = nullptr;
    if (tlh_event_create(&e)) return nullptr;
    p.events.push_back(e);
  }
  return p.events[p.next_event++];
}

// Records an event pair around `launch` when profiling.
template <typename F>
int timed(Program &p, std::vector<std::pair<void *, void *>> &spans, F &&launch) {
  if (!p.profiling) return launch();
  void *a = event(p), *b = event(p);
  if (!a || !b) return 1;
  TRY(tlh_event_record(a, p.stream));
  TRY(launch());
  TRY(tlh_event_record(b, p.stream));
  spans.emplace_back(a, b);
  return 0;
}

// Weight and bias gradient of y = x.W + b: dW = x^T.dy (x stored [rows, in])
// with db = column sums of dy computed inside the same GEMM.
tlh_gemm_desc wgrad(const float *x, const float *dy, float *dw, float *db, int in, int out,
                    int rows) {
  tlh_gemm_desc d = desc(x, dy, dw, in, out, rows, true, false);
  d.bias_grad = db;
  return d;
}

// The three Q/K/V products of a layer as one batched descriptor: entry j
// uses plane j of the activations (stride `act`) and the j-th of wq, wk, wv
// in the parameter or gradient buffer (stride `weights`; each bias sits at
// the same stride after its weight).
void qkv_batch(tlh_gemm_desc &d, uint32_t act, ptrdiff_t weights) {
  d.batch = 3;
  if (d.trans_a) { // weight gradient: A = activations shared, B = dq/dk/dv planes
    d.batch_stride_a = 0;
    d.batch_stride_b = act;
    d.batch_stride_c = uint32_t(weights);
  } else { // dX: A = dq/dk/dv planes, B = the weights
    d.batch_stride_a = act;
    d.batch_stride_b = uint32_t(weights);
    d.batch_stride_c = 0;
  }
  d.bias_batch_stride = uint32_t(weights);
}

bool concurrent(const Program &p) { return p.side != nullptr && p.two_streams && !p.profiling; }

// A second stream pays while the input-gradient chain leaves CUs idle: its
// [rows, dim] products then have fewer than 4 tiles of 64x64 per CU (rows
// 6144, dim 384: 576 tiles on 256 CUs, where the weight gradients beside
// the chain save 11% of the step). Once the chain fills the device on its
// own (rows 8192, dim 1024: 2048 tiles) the two streams only contend for
// CUs and L2, and one stream is 3% faster.
bool auto_two_streams(const Program &p) {
  int cus = 0;
  if (tlh_device_cu_count(&cus) || cus <= 0) return true;
  const size_t tiles = ((p.R + 63) / 64) * ((size_t(p.cfg.dim) + 63) / 64);
  return tiles < 4 * size_t(cus);
}

// Forward products on K-contiguous weight copies (B transposed) instead of
// the [in, out] weights: the GEMM reads a K-contiguous operand tile from LDS
// with one ds_read_b128 per fragment instead of four ds_read_b32, and one
// launch per forward rebuilds the copies. Measured on MI355X: rows 6144 x
// dim 384 (64x64 tiles, fewer than 4 per CU) 3.697 -> 3.679 ms per step;
// rows 8192 x dim 1024 unchanged (77.7 ms), so the copies are used below 4
// tiles per CU only, the same rule as the second stream.
bool auto_forward_copies(const Program &p) { return p.wt != nullptr && auto_two_streams(p); }

// The side stream continues from the main stream's current point.
int fork(Program &p, void *ev) {
  if (!concurrent(p)) return 0;
  TRY(tlh_event_record(ev, p.stream));
  return tlh_stream_wait_event(p.side, ev);
}

// The side stream's work so far completes before what the main stream queues next.
int join(Program &p, void *ev) {
  if (!concurrent(p)) return 0;
  TRY(tlh_event_record(ev, p.side));
  return tlh_stream_wait_event(p.stream, ev);
}

// Waits on the main stream for an event that join-style recording left on
// the side stream earlier in the step.
int after(Program &p, void *ev) {
  if (!concurrent(p)) return 0;
  return tlh_stream_wait_event(p.stream, ev);
}

int record_side(Program &p, void *ev) {
  if (!concurrent(p)) return 0;
  return tlh_event_record(ev, p.side);
}

int gemm(Program &p, tlh_gemm_desc d, bool side = false) {
  const bool on_side = side && concurrent(p);
  // partials of split-K and tail-split products; each stream has its own
  d.workspace = on_side ? p.workspace_side : p.workspace;
  d.workspace_elems = p.workspace_elems;
  if (p.profiling) {
    const double e = d.batch > 1 ? d.batch : 1, mn = double(d.m) * d.n;
    const double a = (e > 1 && d.batch_stride_a == 0) ? 1 : e;
    const double b = (e > 1 && d.batch_stride_b == 0) ? 1 : e;
    const double c = d.sum_batches ? 1 : e;
    p.gemm_flops += 2.0 * mn * d.k * e;
    p.gemm_descs.push_back(d);
    p.gemm_bytes += 4.0 * (a * d.m * d.k + b * double(d.k) * d.n + c * mn * (d.beta != 0.0f ? 2 : 1) +
                           (d.residual ? mn : 0) + (d.aux ? mn : 0) + (d.bias ? c * d.n : 0) +
                           (d.bias_grad ? c * d.n : 0));
  }
  return timed(p, p.gemm_spans, [&] { return tlh_gemm(&d, on_side ? p.side : p.stream); });
}

// Forward over the first `seq` <= cfg.seq positions of every sequence (the
// whole window in training; a shorter prefix is exact for causal decoding,
// where position t only sees positions <= t).
int forward(Program &p, uint32_t seq) {
  const tlg_config &c = p.cfg;
  const size_t rows = size_t(c.batch) * seq;
  const int R = int(rows), D = int(c.dim), F = int(c.ffn), V = int(c.vocab);
  // (one-row products keep the weights: the GEMV path reads B row-major)
  const bool copies = p.forward_copies && rows > 1;
  if (copies) {
    TRY(tlh_transpose_multi(p.params, p.wt, static_cast<const tlh_transpose_job *>(p.wt_jobs),
                            p.wt_count, p.wt_tiles, p.stream));
  }
  TRY(tlh_embedding_add_positions(p.P(0), c.vocab, p.P(1), p.tokens, c.batch, seq, c.dim,
                                  p.x[0], p.stream));
  for (uint32_t l = 0; l < c.layers; ++l) {
    const uint32_t w = 2 + 12 * l;
    TRY(tlh_rms_norm(p.x[l], nullptr, p.n1[l], nullptr, rows, c.dim, kRmsEps, p.stream));
    {
      // Q, K and V in one batched launch: the three weights (and biases)
      // sit at a constant stride in the parameter buffer and q, k, v are
      // consecutive planes of one allocation.
      tlh_gemm_desc d = wdesc(p, copies, p.n1[l], w, p.q[l], R, D, D);
      d.bias = p.P(w + 1);
      d.remap_t = int(seq);
      d.remap_h = int(c.heads);
      d.remap_d = int(kHeadDim);
      d.batch = 3;
      d.batch_stride_a = 0;
      d.batch_stride_b = uint32_t(p.P(w + 2) - p.P(w));
      d.batch_stride_c = uint32_t(p.k[l] - p.q[l]);
      d.bias_batch_stride = uint32_t(p.P(w + 3) - p.P(w + 1));
      TRY(gemm(p, d));
    }
    TRY(timed(p, p.attn_spans, [&] {
      return tlh_attention_forward(p.q[l], p.k[l], p.v[l], p.o[l], p.lse[l], c.batch, c.heads,
                                   seq, kHeadDim, 1.0f / std::sqrt(float(kHeadDim)), 1, 1,
                                   p.stream);
    }));
    {
      tlh_gemm_desc d = wdesc(p, copies, p.o[l], w + 6, p.x_mid[l], R, D, D);
      d.bias = p.P(w + 7);
      d.residual = p.x[l];
      TRY(gemm(p, d));
    }
    TRY(tlh_rms_norm(p.x_mid[l], nullptr, p.n2[l], nullptr, rows, c.dim, kRmsEps, p.stream));
    {
      tlh_gemm_desc d = wdesc(p, copies, p.n2[l], w + 8, p.g[l], R, F, D);
      d.bias = p.P(w + 9);
      d.epilogue = TLH_EPI_GELU;
      d.aux = p.u[l];
      TRY(gemm(p, d));
    }
    {
      tlh_gemm_desc d = wdesc(p, copies, p.g[l], w + 10, p.x[l + 1], R, D, F);
      d.bias = p.P(w + 11);
      d.residual = p.x_mid[l];
      TRY(gemm(p, d));
    }
  }
  TRY(tlh_rms_norm(p.x[c.layers], nullptr, p.nf, nullptr, rows, c.dim, kRmsEps, p.stream));
  const uint32_t last = 2 + 12 * c.layers;
  tlh_gemm_desc d = wdesc(p, copies, p.nf, last, p.logits, R, V, D);
  d.bias = p.P(last + 1);
  return gemm(p, d);
}

// One position of the forward for incremental decoding (batch 1): the token
// at position t (already in tokens[t]) through every block, extending and
// reading the K/V planes that a forward over the window left (their T
// stride is cfg.seq, so position t's keys and values land where the
// window's forward put them). Row 0 of the activation buffers is scratch;
// logits row 0 receives position t's logits. The same arithmetic as row t of
// the window's forward: causal attention never lets row t see later rows.
int decode_step(Program &p, uint32_t t) {
  const tlg_config &c = p.cfg;
  const int D = int(c.dim), F = int(c.ffn), V = int(c.vocab);
  TRY(tlh_embedding_add_positions(p.P(0), c.vocab, p.P(1) + size_t(t) * c.dim, p.tokens + t, 1,
                                  1, c.dim, p.x[0], p.stream));
  for (uint32_t l = 0; l < c.layers; ++l) {
    const uint32_t w = 2 + 12 * l;
    TRY(tlh_rms_norm(p.x[l], nullptr, p.n1[l], nullptr, 1, c.dim, kRmsEps, p.stream));
    {
      // Q, K, V of position t, written into the planes at row t: the head
      // remap of row 0 with a T stride of cfg.seq, offset by t rows.
      tlh_gemm_desc d =
          desc(p.n1[l], p.P(w), p.q[l] + size_t(t) * kHeadDim, 1, D, D, false, false);
      d.bias = p.P(w + 1);
      d.remap_t = int(c.seq);
      d.remap_h = int(c.heads);
      d.remap_d = int(kHeadDim);
      d.batch = 3;
      d.batch_stride_a = 0;
      d.batch_stride_b = uint32_t(p.P(w + 2) - p.P(w));
      d.batch_stride_c = uint32_t(p.k[l] - p.q[l]);
      d.bias_batch_stride = uint32_t(p.P(w + 3) - p.P(w + 1));
      TRY(gemm(p, d));
    }
    TRY(tlh_attention_decode(p.q[l], p.k[l], p.v[l], p.o[l], c.heads, c.seq, t, kHeadDim,
                             1.0f / std::sqrt(float(kHeadDim)), p.stream));
    {
      tlh_gemm_desc d = desc(p.o[l], p.P(w + 6), p.x_mid[l], 1, D, D, false, false);
      d.bias = p.P(w + 7);
      d.residual = p.x[l];
      TRY(gemm(p, d));
    }
    TRY(tlh_rms_norm(p.x_mid[l], nullptr, p.n2[l], nullptr, 1, c.dim, kRmsEps, p.stream));
    {
      tlh_gemm_desc d = desc(p.n2[l], p.P(w + 8), p.g[l], 1, F, D, false, false);
      d.bias = p.P(w + 9);
      d.epilogue = TLH_EPI_GELU;
      d.aux = p.u[l];
      TRY(gemm(p, d));
    }
    {
      tlh_gemm_desc d = desc(p.g[l], p.P(w + 10), p.x[l + 1], 1, D, F, false, false);
      d.bias = p.P(w + 11);
      d.residual = p.x_mid[l];
      TRY(gemm(p, d));
    }
  }
  TRY(tlh_rms_norm(p.x[c.layers], nullptr, p.nf, nullptr, 1, c.dim, kRmsEps, p.stream));
  const uint32_t last = 2 + 12 * c.layers;
  tlh_gemm_desc d = desc(p.nf, p.P(last), p.logits, 1, V, D, false, false);
  d.bias = p.P(last + 1);
  return gemm(p, d);
}

// Input gradients run on the main stream; each weight gradient forks to the
// side stream as soon as its upstream gradient exists, and the main stream
// waits for it only before overwriting that gradient's buffer: dx is updated
// in place twice per block, dgf and dq/dk/dv are rewritten one block later.
int backward(Program &p) {
  const tlg_config &c = p.cfg;
  const int R = int(p.R), D = int(c.dim), F = int(c.ffn), V = int(c.vocab);
  const uint32_t last = 2 + 12 * c.layers;
  auto ev = [&](int l, int i) { return p.sync[2 + 8 * size_t(l) + size_t(i)]; };
  // vocab projection
  TRY(fork(p, p.sync[0]));
  TRY(gemm(p, wgrad(p.nf, p.dlogits, p.G(last), p.G(last + 1), D, V, R), true));
  TRY(gemm(p, desc(p.dlogits, p.P(last), p.tmp, R, D, V, false, true)));
  TRY(tlh_rms_norm_backward(p.tmp, p.x[c.layers], nullptr, p.dx, nullptr, p.R, c.dim, kRmsEps,
                            0.0f, p.stream));
  for (int l = int(c.layers) - 1; l >= 0; --l) {
    const uint32_t w = 2 + 12 * uint32_t(l);
    const bool top = l + 1 == int(c.layers);
    // FFN: x[l+1] = x_mid + W2.GELU(W1.n2 + b1) + b2
    TRY(fork(p, ev(l, 0)));
    TRY(gemm(p, wgrad(p.g[l], p.dx, p.G(w + 10), p.G(w + 11), F, D, R), true));
    TRY(record_side(p, ev(l, 1)));
    if (!top) TRY(after(p, ev(l + 1, 3))); // the block above's dW1 has read dgf
    {
      tlh_gemm_desc d = desc(p.dx, p.P(w + 10), p.dgf, R, F, D, false, true);
      d.epilogue = TLH_EPI_GELU_BWD;
      d.aux = p.u[l];
      TRY(gemm(p, d));
    }
    TRY(fork(p, ev(l, 2)));
    TRY(gemm(p, wgrad(p.n2[l], p.dgf, p.G(w + 8), p.G(w + 9), D, F, R), true));
    TRY(record_side(p, ev(l, 3)));
    TRY(gemm(p, desc(p.dgf, p.P(w + 8), p.tmp, R, D, F, false, true)));
    TRY(after(p, ev(l, 1))); // dW2 has read dx
    TRY(tlh_rms_norm_backward(p.tmp, p.x_mid[l], nullptr, p.dx, nullptr, p.R, c.dim, kRmsEps,
                              1.0f, p.stream));
    // attention: x_mid = x + Wo.attn(n1) + bo
    TRY(fork(p, ev(l, 4)));
    TRY(gemm(p, wgrad(p.o[l], p.dx, p.G(w + 6), p.G(w + 7), D, D, R), true));
    TRY(record_side(p, ev(l, 5)));
    TRY(gemm(p, desc(p.dx, p.P(w + 6), p.tmp, R, D, D, false, true)));
    if (!top) TRY(after(p, ev(l + 1, 7))); // the block above's dWq/k/v have read dq/dk/dv
    TRY(timed(p, p.attn_spans, [&] {
      return tlh_attention_backward(p.q[l], p.k[l], p.v[l], p.o[l], p.tmp, p.lse[l], p.delta,
                                    p.dq, p.dk, p.dv, c.batch, c.heads, c.seq, kHeadDim,
                                    1.0f / std::sqrt(float(kHeadDim)), 1, 1, 1, p.stream);
    }));
    // dWq, dWk, dWv (+ bias gradients) as one batched product over the
    // consecutive dq, dk, dv planes; dX = dq.Wq^T + dk.Wk^T + dv.Wv^T as one
    // product whose K range runs through the three (dq_j, W_j) pairs.
    TRY(fork(p, ev(l, 6)));
    {
      tlh_gemm_desc d = wgrad(p.n1[l], p.dq, p.G(w), p.G(w + 1), D, D, R);
      qkv_batch(d, uint32_t(p.dk - p.dq), p.G(w + 2) - p.G(w));
      TRY(gemm(p, d, true));
    }
    TRY(record_side(p, ev(l, 7)));
    {
      tlh_gemm_desc d = desc(p.dq, p.P(w), p.tmp, R, D, D, false, true);
      qkv_batch(d, uint32_t(p.dk - p.dq), p.P(w + 2) - p.P(w));
      d.batch_stride_c = 0;
      d.sum_batches = 1;
      TRY(gemm(p, d));
    }
    TRY(after(p, ev(l, 5))); // dWo has read dx
    TRY(tlh_rms_norm_backward(p.tmp, p.x[l], nullptr, p.dx, nullptr, p.R, c.dim, kRmsEps, 1.0f,
                              p.stream));
  }
  // embeddings: scatter_index for tokens (zero + scatter_add_rows), positions
  // as a column sum over the batch of the [B, T*D] view.
  TRY(tlh_fill_f32(p.G(0), 0.0f, p.size[0], p.stream));
  TRY(tlh_scatter_add_rows(p.dx, p.tokens, p.R, c.dim, p.G(0), c.vocab, p.stream));
  TRY(tlh_column_sum(p.dx, c.batch, c.seq * c.dim, p.G(1), 0.0f, p.stream));
  return join(p, p.sync[1]); // every weight gradient is complete
}

int optimizer_step(Program &p, float max_norm) {
  const uint32_t count = uint32_t(p.size.size());
  TRY(tlh_gradient_squared_norm_multi(reinterpret_cast<const float *const *>(p.tab_grads),
                                      p.tab_sizes, count, p.norm_partials, p.sqnorm, p.stream));
  TRY(tlh_increment_u32(p.steps, count, 1, p.stream));
  return tlh_adamw_multi(reinterpret_cast<float *const *>(p.tab_params),
                         reinterpret_cast<const float *const *>(p.tab_grads),
                         reinterpret_cast<float *const *>(p.tab_m1),
                         reinterpret_cast<float *const *>(p.tab_m2), p.tab_sizes, p.steps, count,
                         p.scalars, p.scalars + 1, p.scalars + 2, p.scalars + 3, p.eps,
                         max_norm > 0.0f ? p.sqnorm : nullptr, max_norm, p.stream);
}

int train_step(Program &p, float root_grad, float max_norm, int update) {
  TRY(forward(p, p.cfg.seq));
  TRY(tlh_cross_entropy_rows_fused(p.logits, p.targets, p.losses, p.dlogits, p.R, p.cfg.vocab,
                                   root_grad, p.stream));
  TRY(backward(p));
  if (!update) {
    const uint32_t count = uint32_t(p.size.size());
    return tlh_gradient_squared_norm_multi(reinterpret_cast<const float *const *>(p.tab_grads),
                                           p.tab_sizes, count, p.norm_partials, p.sqnorm,
                                           p.stream);
  }
  return optimizer_step(p, max_norm);
}

int write_scalars(Program &p, float beta1, float beta2) {
  const float decay = 1.0f - p.lr * p.weight_decay; // AdamW.h:28-29, fp32 on the host
  const float host[4] = {beta1, beta2, decay, p.lr};
  TRY(tlh_memcpy_h2d(p.scalars, host, sizeof(host), p.stream));
  return tlh_stream_synchronize(p.stream);
}

int create(Program &p) {
  const tlg_config &c = p.cfg;
  const size_t R = p.R, D = c.dim, F = c.ffn, V = c.vocab, B = c.batch, H = c.heads,
               T = c.seq, L = c.layers;
  layout(p);
  TRY(allocf(p, &p.params, p.padded_total));
  TRY(allocf(p, &p.grads, p.padded_total));
  TRY(allocf(p, &p.m1, p.padded_total));
  TRY(allocf(p, &p.m2, p.padded_total));
  const size_t count = p.size.size();
  TRY(alloc(p, &p.tab_params, count * sizeof(void *)));
  TRY(alloc(p, &p.tab_grads, count * sizeof(void *)));
  TRY(alloc(p, &p.tab_m1, count * sizeof(void *)));
  TRY(alloc(p, &p.tab_m2, count * sizeof(void *)));
  TRY(alloc(p, reinterpret_cast<void **>(&p.tab_sizes), count * sizeof(uint64_t)));
  TRY(alloc(p, reinterpret_cast<void **>(&p.steps), count * sizeof(uint32_t)));
  TRY(allocf(p, &p.scalars, 4));
  TRY(allocf(p, &p.norm_partials, TLH_NORM_PARTIALS));
  TRY(allocf(p, &p.sqnorm, 1));
  {
    std::vector<void *> tp(count), tg(count), t1(count), t2(count);
    std::vector<uint64_t> sz(count);
    for (size_t i = 0; i < count; ++i) {
      tp[i] = p.params + p.offset[i];
      tg[i] = p.grads + p.offset[i];
      t1[i] = p.m1 + p.offset[i];
      t2[i] = p.m2 + p.offset[i];
      sz[i] = p.size[i];
    }
    TRY(tlh_memcpy_h2d(p.tab_params, tp.data(), count * sizeof(void *), p.stream));
    TRY(tlh_memcpy_h2d(p.tab_grads, tg.data(), count * sizeof(void *), p.stream));
    TRY(tlh_memcpy_h2d(p.tab_m1, t1.data(), count * sizeof(void *), p.stream));
    TRY(tlh_memcpy_h2d(p.tab_m2, t2.data(), count * sizeof(void *), p.stream));
    TRY(tlh_memcpy_h2d(p.tab_sizes, sz.data(), count * sizeof(uint64_t), p.stream));
    TRY(tlh_stream_synchronize(p.stream));
  }
  {
    // the weight matrices [in, out]: per layer wq, wk, wv, wo, w1, w2, then wp
    std::vector<tlh_transpose_job> jobs;
    std::vector<uint32_t> weights;
    for (uint32_t l = 0; l < c.layers; ++l)
      for (uint32_t k : {0u, 2u, 4u, 6u, 8u, 10u}) weights.push_back(2 + 12 * l + k);
    weights.push_back(2 + 12 * uint32_t(L));
    uint32_t tiles = 0;
    for (uint32_t w : weights) {
      const uint32_t in = w == 2 + 12 * uint32_t(L) ? uint32_t(D)
                          : (w - 2) % 12 == 10  ? uint32_t(F)
                                                : uint32_t(D);
      const uint32_t out = uint32_t(p.size[w] / in);
      tlh_transpose_job j{};
      j.src_offset = j.dst_offset = p.offset[w];
      j.rows = in;
      j.cols = out;
      j.first_tile = tiles;
      tiles += ((in + 63) / 64) * ((out + 63) / 64);
      jobs.push_back(j);
    }
    if (jobs.size() <= 256) {
      TRY(allocf(p, &p.wt, p.padded_total));
      TRY(alloc(p, &p.wt_jobs, jobs.size() * sizeof(tlh_transpose_job)));
      TRY(tlh_memcpy_h2d(p.wt_jobs, jobs.data(), jobs.size() * sizeof(tlh_transpose_job),
                         p.stream));
      TRY(tlh_stream_synchronize(p.stream));
      p.wt_count = uint32_t(jobs.size());
      p.wt_tiles = tiles;
    }
  }
  TRY(tlh_fill_u32(p.steps, 0, count, p.stream));
  TRY(tlh_fill_f32(p.params, 0.0f, p.padded_total, p.stream));
  TRY(tlh_fill_f32(p.grads, 0.0f, p.padded_total, p.stream));
  TRY(tlh_fill_f32(p.m1, 0.0f, p.padded_total, p.stream));
  TRY(tlh_fill_f32(p.m2, 0.0f, p.padded_total, p.stream));

  TRY(alloc(p, reinterpret_cast<void **>(&p.tokens), R * sizeof(uint32_t)));
  TRY(alloc(p, reinterpret_cast<void **>(&p.targets), R * sizeof(uint32_t)));
  TRY(tlh_fill_u32(p.tokens, 0, R, p.stream));
  TRY(tlh_fill_u32(p.targets, 0, R, p.stream));
  TRY(allocf(p, &p.losses, R));
  TRY(alloc(p, reinterpret_cast<void **>(&p.argmax_out), 2 * sizeof(uint32_t)));
  TRY(allocf(p, &p.logits, R * V));
  TRY(allocf(p, &p.dlogits, R * V));
  p.x.resize(L + 1);
  for (auto &b : p.x) TRY(allocf(p, &b, R * D));
  for (auto *vec : {&p.n1, &p.o, &p.x_mid, &p.n2}) {
    vec->resize(L);
    for (auto &b : *vec) TRY(allocf(p, &b, R * D));
  }
  // q, k, v of a layer: three consecutive [B,H,T,64] planes (one batched GEMM)
  p.q.resize(L);
  p.k.resize(L);
  p.v.resize(L);
  for (size_t l = 0; l < L; ++l) {
    TRY(allocf(p, &p.q[l], 3 * R * D));
    p.k[l] = p.q[l] + R * D;
    p.v[l] = p.q[l] + 2 * R * D;
  }
  p.lse.resize(L);
  for (auto &b : p.lse) TRY(allocf(p, &b, B * H * T));
  p.u.resize(L);
  p.g.resize(L);
  for (size_t l = 0; l < L; ++l) {
    TRY(allocf(p, &p.u[l], R * F));
    TRY(allocf(p, &p.g[l], R * F));
  }
  TRY(allocf(p, &p.nf, R * D));
  TRY(allocf(p, &p.dx, R * D));
  TRY(allocf(p, &p.tmp, R * D));
  TRY(allocf(p, &p.dgf, R * F));
  // dq, dk, dv: consecutive planes (the batched Q/K/V backward products)
  TRY(allocf(p, &p.dq, 3 * R * D));
  p.dk = p.dq + R * D;
  p.dv = p.dq + 2 * R * D;
  TRY(allocf(p, &p.delta, B * H * T));
  // workspace: the largest any GEMM of the step asks for (split-K weight
  // gradients; tail splits of the others)
  size_t ws = 0;
  const int shapes[4][2] = {{int(D), int(V)}, {int(F), int(D)}, {int(D), int(F)},
                            {int(D), int(D)}};
  std::vector<tlh_gemm_desc> uses;
  for (auto &s : shapes) uses.push_back(desc(nullptr, nullptr, nullptr, s[0], s[1], int(R), true, false));
  {
    tlh_gemm_desc d = desc(nullptr, nullptr, nullptr, int(D), int(D), int(R), true, false);
    qkv_batch(d, uint32_t(R * D), ptrdiff_t(D * D + D));
    uses.push_back(d);
    d = desc(nullptr, nullptr, nullptr, int(R), int(D), int(D), false, true);
    qkv_batch(d, uint32_t(R * D), ptrdiff_t(D * D + D));
    d.sum_batches = 1;
    uses.push_back(d);
  }
  // linears (out, in): forward x.W and input gradient dY.W^T
  const int linears[4][2] = {{int(D), int(D)}, {int(F), int(D)}, {int(D), int(F)},
                             {int(V), int(D)}};
  for (auto &s : linears) {
    uses.push_back(desc(nullptr, nullptr, nullptr, int(R), s[0], s[1], false, false));
    uses.push_back(desc(nullptr, nullptr, nullptr, int(R), s[1], s[0], false, true));
  }
  if (c.batch == 1) {
    // decode_step: one row through every linear (split K: a single row
    // gives only N/64 output tiles), Q/K/V batched
    for (auto &s : linears) uses.push_back(desc(nullptr, nullptr, nullptr, 1, s[0], s[1], false, false));
    tlh_gemm_desc d = desc(nullptr, nullptr, nullptr, 1, int(D), int(D), false, false);
    d.batch = 3;
    d.batch_stride_a = 0;
    d.batch_stride_b = uint32_t(D * D + D);
    d.batch_stride_c = uint32_t(R * D);
    uses.push_back(d);
  }
  for (auto &d : uses) {
    size_t e = 0;
    tlh_gemm_workspace_size(&d, &e);
    if (e > ws) ws = e;
  }
  p.workspace_elems = ws;
  // The batched Q/K/V GEMM needs wq->wk->wv (and bq->bk->bv) at one stride;
  // every tensor is padded to kAlign floats and D is a multiple of 64.
  for (size_t l = 0; l < L; ++l) {
    const uint32_t w = 2 + 12 * uint32_t(l);
    if (p.offset[w + 2] - p.offset[w] != p.offset[w + 4] - p.offset[w + 2] ||
        p.offset[w + 3] - p.offset[w + 1] != p.offset[w + 5] - p.offset[w + 3])
      return kInvalidValue;
  }
  if (ws) {
    TRY(allocf(p, &p.workspace, ws));
    TRY(allocf(p, &p.workspace_side, ws));
  }
  TRY(tlh_stream_create(&p.side));
  p.two_streams = auto_two_streams(p);
  p.forward_copies = auto_forward_copies(p);
  p.sync.resize(2 + 8 * L);
  for (auto &e : p.sync) TRY(tlh_event_create(&e));
  p.lr = 1e-3f;
  TRY(write_scalars(p, 0.9f, 0.999f));
  return tlh_stream_synchronize(p.stream);
}

void release(Program &p) {
  if (p.graph) tlh_graph_destroy(p.graph);
  for (void *e : p.events) tlh_event_destroy(e);
  p.events.clear();
  for (void *e : p.sync)
    if (e) tlh_event_destroy(e);
  p.sync.clear();
  if (p.side) tlh_stream_destroy(p.side);
  p.side = nullptr;
  for (void *a : p.allocations) tlh_free(a);
  p.allocations.clear();
}

int copy_params(Program &p, float *dev_base, const float *host, bool to_device) {
  // flat canonical host vector <-> padded device layout
  size_t flat = 0;
  for (size_t i = 0; i < p.size.size(); ++i) {
    const size_t bytes = p.size[i] * sizeof(float);
    if (to_device) {
      TRY(tlh_memcpy_h2d(dev_base + p.offset[i], host + flat, bytes, p.stream));
    } else {
      TRY(tlh_memcpy_d2h(const_cast<float *>(host) + flat, dev_base + p.offset[i], bytes,
                         p.stream));
    }
    flat += p.size[i];
  }
  return tlh_stream_synchronize(p.stream);
}

// Archive entry `index` of the reference checkpoint layout (the reference's
// gradient-path order over nn::GPT: the blocks from the last to the first,
// each w1 b1 w2 b2 wq bq wk bk wv bv wo bo, then the token and position
// tables, then wp, bp) -> canonical parameter index and [rows, cols] shape.
bool archive_entry(const tlg_config &c, uint32_t index, uint32_t &canonical, uint32_t shape[2]) {
  const uint32_t L = c.layers, D = c.dim, F = c.ffn, V = c.vocab, T = c.seq;
  static const uint32_t block_slot[12] = {8, 9, 10, 11, 0, 1, 2, 3, 4, 5, 6, 7};
  const uint32_t last = 2 + 12 * L;
  if (index < 12 * L) canonical = 2 + 12 * (L - 1 - index / 12) + block_slot[index % 12];
  else if (index < 12 * L + 4) canonical = std::array<uint32_t, 4>{0, 1, last, last + 1}[index - 12 * L];
  else return false;
  if (canonical == 0) shape[0] = V, shape[1] = D;
  else if (canonical == 1) shape[0] = T, shape[1] = D;
  else if (canonical == last) shape[0] = D, shape[1] = V;
  else if (canonical == last + 1) shape[0] = 1, shape[1] = V;
  else {
    const uint32_t s = (canonical - 2) % 12;
    if (s == 8) shape[0] = D, shape[1] = F;       // w1
    else if (s == 10) shape[0] = F, shape[1] = D; // w2
    else if (s % 2 == 0) shape[0] = D, shape[1] = D;
    else shape[0] = 1, shape[1] = (s == 9 ? F : D); // biases
  }
  return true;
}

template <typename T> std::span<const std::byte> bytes_of(const std::vector<T> &v) {
  return std::as_bytes(std::span<const T>(v));
}

// A token file's dataset and a loader over one of its splits.
struct TokenLoader {
  Dataset dataset;
  std::optional<Loader> loader;
};

bool is_bias(const Program &p, uint32_t i) {
  if (i < 2) return false;
  const uint32_t last = 2 + 12 * p.cfg.layers;
  if (i == last) return false;
  if (i == last + 1) return true;
  return ((i - 2) % 12) % 2 == 1;
}

} // namespace

extern "C" {

int tlg_create(const tlg_config *cfg, void *stream, void **program) {
  *program = nullptr;
  if (!cfg || cfg->heads == 0 || cfg->dim != cfg->heads * kHeadDim || cfg->vocab == 0 ||
      cfg->seq == 0 || cfg->batch == 0 || cfg->layers == 0 || cfg->ffn == 0)
    return 1; // hipErrorInvalidValue
  Program *p = new (std::nothrow) Program();
  if (!p) return 2; // hipErrorOutOfMemory
  p->cfg = *cfg;
  p->stream = stream;
  p->R = size_t(cfg->batch) * cfg->seq;
  const int st = create(*p);
  if (st) {
    release(*p);
    delete p;
    return st;
  }
  *program = p;
  return 0;
}

int tlg_destroy(void *program) {
  if (!program) return 0;
  Program *p = static_cast<Program *>(program);
  tlh_stream_synchronize(p->stream);
  release(*p);
  delete p;
  return 0;
}

int tlg_param_count(void *program, uint32_t *count) {
  *count = uint32_t(static_cast<Program *>(program)->size.size());
  return 0;
}

int tlg_param_info(void *program, uint32_t index, uint64_t *size, float **param, float **grad,
                   float **m1, float **m2) {
  Program *p = static_cast<Program *>(program);
  if (index >= p->size.size()) return 1;
  if (size) *size = p->size[index];
  if (param) *param = p->params + p->offset[index];
  if (grad) *grad = p->grads + p->offset[index];
  if (m1) *m1 = p->m1 + p->offset[index];
  if (m2) *m2 = p->m2 + p->offset[index];
  return 0;
}

int tlg_total_params(void *program, uint64_t *total) {
  *total = static_cast<Program *>(program)->total;
  return 0;
}

int tlg_set_params(void *program, const float *host_params) {
  Program *p = static_cast<Program *>(program);
  return copy_params(*p, p->params, host_params, true);
}

int tlg_get_params(void *program, float *host_params) {
  Program *p = static_cast<Program *>(program);
  return copy_params(*p, p->params, host_params, false);
}

int tlg_get_grads(void *program, float *host_grads) {
  Program *p = static_cast<Program *>(program);
  return copy_params(*p, p->grads, host_grads, false);
}

int tlg_get_moments(void *program, float *host_m1, float *host_m2) {
  Program *p = static_cast<Program *>(program);
  TRY(copy_params(*p, p->m1, host_m1, false));
  return copy_params(*p, p->m2, host_m2, false);
}

int tlg_get_steps(void *program, uint32_t *host_steps) {
  Program *p = static_cast<Program *>(program);
  TRY(tlh_memcpy_d2h(host_steps, p->steps, p->size.size() * sizeof(uint32_t), p->stream));
  return tlh_stream_synchronize(p->stream);
}

int tlg_get_scalars(void *program, float *host_scalars4) {
  Program *p = static_cast<Program *>(program);
  TRY(tlh_memcpy_d2h(host_scalars4, p->scalars, 4 * sizeof(float), p->stream));
  return tlh_stream_synchronize(p->stream);
}

int tlg_init_params(void *program, uint64_t seed, float std) {
  Program *p = static_cast<Program *>(program);
  for (uint32_t i = 0; i < p->size.size(); ++i) {
    float *dst = p->params + p->offset[i];
    if (is_bias(*p, i)) {
      TRY(tlh_fill_f32(dst, 0.0f, p->size[i], p->stream));
    } else {
      TRY(tlh_fill_normal(dst, p->size[i], seed + 7919ull * i, 0.0f, std, p->stream));
    }
  }
  TRY(tlh_fill_f32(p->m1, 0.0f, p->padded_total, p->stream));
  TRY(tlh_fill_f32(p->m2, 0.0f, p->padded_total, p->stream));
  TRY(tlh_fill_u32(p->steps, 0, p->size.size(), p->stream));
  return tlh_stream_synchronize(p->stream);
}

int tlg_set_optimizer(void *program, float lr, float beta1, float beta2, float eps,
                      float weight_decay) {
  Program *p = static_cast<Program *>(program);
  p->lr = lr;
  p->eps = eps;
  p->weight_decay = weight_decay;
  return write_scalars(*p, beta1, beta2);
}

int tlg_set_lr(void *program, float lr) {
  Program *p = static_cast<Program *>(program);
  p->lr = lr;
  const float host[2] = {1.0f - lr * p->weight_decay, lr};
  TRY(tlh_memcpy_h2d(p->scalars + 2, host, sizeof(host), p->stream));
  return tlh_stream_synchronize(p->stream);
}

int tlg_set_concurrency(void *program, int mode) {
  Program *p = static_cast<Program *>(program);
  if (mode < -1 || mode > 1) return kInvalidValue;
  TRY(tlh_stream_synchronize(p->stream));
  TRY(tlh_stream_synchronize(p->side));
  p->two_streams = mode < 0 ? auto_two_streams(*p) : mode == 1;
  return 0;
}

int tlg_set_forward_copies(void *program, int mode) {
  Program *p = static_cast<Program *>(program);
  if (mode < -1 || mode > 1) return kInvalidValue;
  if (mode == 1 && !p->wt) return kInvalidValue;
  TRY(tlh_stream_synchronize(p->stream));
  p->forward_copies = mode < 0 ? auto_forward_copies(*p) : mode == 1;
  return 0;
}

int tlg_get_forward_copies(void *program, int *copies) {
  *copies = static_cast<Program *>(program)->forward_copies ? 1 : 0;
  return 0;
}

int tlg_get_concurrency(void *program, int *two_streams) {
  *two_streams = static_cast<Program *>(program)->two_streams ? 1 : 0;
  return 0;
}

int tlg_io(void *program, uint32_t **tokens, uint32_t **targets, float **losses,
           float **logits) {
  Program *p = static_cast<Program *>(program);
  if (tokens) *tokens = p->tokens;
  if (targets) *targets = p->targets;
  if (losses) *losses = p->losses;
  if (logits) *logits = p->logits;
  return 0;
}

int tlg_train_step(void *program, float root_grad, float max_norm, int update) {
  return train_step(*static_cast<Program *>(program), root_grad, max_norm, update);
}

int tlg_forward(void *program) {
  Program &p = *static_cast<Program *>(program);
  return forward(p, p.cfg.seq);
}

extern "C++" {
namespace {
// inference::autoregression's loop (include/inference.h:45-99): the window
// holds the prompt, EOS-padded; each step computes the logits at the last
// valid position, `choose` launches the kernel that writes the next token
// (and the draws it used) to p.argmax_out[0..1], and the token is appended
// (the window slides once full). With stop_at_eos generation ends after an
// EOS is emitted (inference.h:86-90). prefix_only: 0 recomputes the padded
// window as the reference does, 1 only the valid prefix (the same logits:
// attention is causal), 2 keeps the window's K/V planes and runs each new
// position alone through decode_step while the window has room. `picked`
// sees each step's token and draw count. Returns the tokens generated in
// *count.
template <typename Choose, typename Picked>
int generate(Program &p, const uint32_t *host_prompt, uint32_t prompt_len, uint32_t n_new,
             uint32_t eos_token, int prefix_only, bool stop_at_eos, Choose &&choose,
             Picked &&picked, uint32_t *host_out, uint32_t *count) {
  const tlg_config &c = p.cfg;
  *count = 0;
  if (c.batch != 1 || prompt_len == 0 || prompt_len > c.seq || prefix_only < 0 ||
      prefix_only > 2)
    return kInvalidValue;
  for (uint32_t i = 0; i < prompt_len; ++i)
    if (host_prompt[i] >= c.vocab) return kInvalidValue;
  std::vector<uint32_t> context(c.seq, eos_token);
  std::copy(host_prompt, host_prompt + prompt_len, context.begin());
  uint32_t valid = prompt_len;
  bool cached = false;
  for (uint32_t g = 0; g < n_new; ++g) {
    const float *row;
    if (cached) {
      const uint32_t t = valid - 1; // the newest token's position
      TRY(tlh_memcpy_h2d(p.tokens + t, &context[t], sizeof(uint32_t), p.stream));
      TRY(decode_step(p, t));
      row = p.logits;
    } else {
      const uint32_t seq = prefix_only == 1 ? valid : c.seq;
      TRY(tlh_memcpy_h2d(p.tokens, context.data(), size_t(seq) * sizeof(uint32_t), p.stream));
      TRY(forward(p, seq));
      row = p.logits + size_t(valid - 1) * c.vocab;
    }
    TRY(choose(row, g));
    uint32_t out[2] = {0, 0};
    TRY(tlh_memcpy_d2h(out, p.argmax_out, sizeof(out), p.stream));
    TRY(tlh_stream_synchronize(p.stream));
    const uint32_t token = out[0];
    host_out[g] = token;
    *count = g + 1;
    picked(token, out[1]);
    if (stop_at_eos && token == eos_token) break;
    if (valid < c.seq) {
      context[valid++] = token;
      // the window's K/V planes now serve decode_step (or keep serving it)
      cached = prefix_only == 2;
    } else {
      std::move(context.begin() + 1, context.end(), context.begin());
      context.back() = token;
      cached = false; // the window slid: every position moved
    }
  }
  return 0;
}
} // namespace
} // extern "C++"

int tlg_generate_greedy(void *program, const uint32_t *host_prompt, uint32_t prompt_len,
                        uint32_t n_new, uint32_t eos_token, int prefix_only,
                        uint32_t *host_out) {
  Program &p = *static_cast<Program *>(program);
  uint32_t count = 0;
  // greedy = the lowest-index maximum of the logits (sample_top_k with
  // top_k 1); EOS does not stop it
  return generate(
      p, host_prompt, prompt_len, n_new, eos_token, prefix_only, false,
      [&](const float *row, uint32_t) { return tlh_argmax(row, p.cfg.vocab, p.argmax_out, p.stream); },
      [](uint32_t, uint32_t) {}, host_out, &count);
}

int tlg_generate_sample(void *program, const uint32_t *host_prompt, uint32_t prompt_len,
                        uint32_t n_new, uint32_t eos_token, uint32_t top_k, float temperature,
                        uint32_t minimum_length, uint64_t seed, int prefix_only,
                        uint32_t *host_out, uint32_t *host_count) {
  Program &p = *static_cast<Program *>(program);
  if (!host_count || !(temperature > 0.0f)) return kInvalidValue;
  // inference.h:68, 80-84: EOS is drawn again while fewer than
  // min(minimum_length, window) tokens were generated
  const uint32_t min_len = std::min(minimum_length, p.cfg.seq);
  uint64_t counter = 0; // SplitMix64 outputs used so far
  return generate(
      p, host_prompt, prompt_len, n_new, eos_token, prefix_only, true,
      [&](const float *row, uint32_t g) {
        return tlh_sample_top_k(row, 1, p.cfg.vocab, p.cfg.vocab, top_k, temperature, seed,
                                counter, nullptr, eos_token, g < min_len ? 1 : 0,
                                kMaxSampleDraws, p.argmax_out, p.argmax_out + 1, p.stream);
      },
      [&](uint32_t, uint32_t used) { counter += used; }, host_out, host_count);
}

int tlg_last_squared_norm(void *program, float *host_value) {
  Program *p = static_cast<Program *>(program);
  TRY(tlh_memcpy_d2h(host_value, p->sqnorm, sizeof(float), p->stream));
  return tlh_stream_synchronize(p->stream);
}

int tlg_profile_step(void *program, float root_grad, float max_norm, float *host_gemm_ms,
                     double *host_gemm_flops, double *host_gemm_bytes,
                     uint32_t *host_gemm_launches,
                     float *host_attention_ms, float *host_step_ms) {
  Program *p = static_cast<Program *>(program);
  TRY(tlh_stream_synchronize(p->stream));
  p->profiling = true;
  p->next_event = 0;
  p->gemm_spans.clear();
  p->attn_spans.clear();
  p->gemm_flops = 0.0;
  p->gemm_bytes = 0.0;
  p->gemm_descs.clear();
  void *start = event(*p), *end = event(*p);
  int st = (start && end) ? tlh_event_record(start, p->stream) : 1;
  if (!st) st = train_step(*p, root_grad, max_norm, 1);
  if (!st) st = tlh_event_record(end, p->stream);
  p->profiling = false;
  TRY(st);
  TRY(tlh_stream_synchronize(p->stream));
  float total = 0.0f, ms = 0.0f;
  for (auto &s : p->gemm_spans) {
    TRY(tlh_event_elapsed_ms(s.first, s.second, &ms));
    total += ms;
  }
  float attn = 0.0f;
  for (auto &s : p->attn_spans) {
    TRY(tlh_event_elapsed_ms(s.first, s.second, &ms));
    attn += ms;
  }
  TRY(tlh_event_elapsed_ms(start, end, &ms));
  *host_gemm_ms = total;
  *host_gemm_flops = p->gemm_flops;
  *host_gemm_bytes = p->gemm_bytes;
  *host_gemm_launches = uint32_t(p->gemm_spans.size());
  *host_attention_ms = attn;
  *host_step_ms = ms;
  return 0;
}

int tlg_time_gemms(void *program, uint32_t iters, float *host_ms) {
  Program *p = static_cast<Program *>(program);
  if (iters == 0 || p->gemm_descs.empty()) return kInvalidValue;
  TRY(tlh_stream_synchronize(p->stream));
  void *a = nullptr, *b = nullptr;
  TRY(tlh_event_create(&a));
  int st = tlh_event_create(&b);
  float total = 0.0f;
  for (size_t i = 0; !st && i < p->gemm_descs.size(); ++i) {
    const tlh_gemm_desc &d = p->gemm_descs[i];
    st = tlh_gemm(&d, p->stream); // warm-up
    if (!st) st = tlh_event_record(a, p->stream);
    for (uint32_t r = 0; !st && r < iters; ++r) st = tlh_gemm(&d, p->stream);
    if (!st) st = tlh_event_record(b, p->stream);
    if (!st) st = tlh_event_synchronize(b);
    float ms = 0.0f;
    if (!st) st = tlh_event_elapsed_ms(a, b, &ms);
    total += ms / float(iters);
  }
  tlh_event_destroy(a);
  if (b) tlh_event_destroy(b);
  TRY(st);
  *host_ms = total;
  return 0;
}

int tlg_archive_entry(const tlg_config *cfg, uint32_t index, uint32_t *canonical,
                      uint32_t *shape2) {
  if (!cfg || !canonical || !shape2) return kInvalidValue;
  return archive_entry(*cfg, index, *canonical, shape2) ? 0 : kInvalidValue;
}

int tlg_save_archive(void *program, const char *path, int optimiser) {
  Program *p = static_cast<Program *>(program);
  if (!path) return kInvalidValue;
  const uint32_t count = uint32_t(p->size.size());
  std::vector<uint32_t> steps(count);
  TRY(tlh_stream_synchronize(p->stream));
  TRY(tlh_memcpy_d2h(steps.data(), p->steps, count * sizeof(uint32_t), p->stream));
  TRY(tlh_stream_synchronize(p->stream));
  try {
    Archive archive;
    auto params = archive.scope("parameters");
    auto optimisers = archive.scope("optimisers");
    for (uint32_t i = 0; i < count; ++i) {
      uint32_t c = 0;
      std::vector<uint32_t> shape(2);
      if (!archive_entry(p->cfg, i, c, shape.data())) return kInvalidValue;
      std::vector<float> host(p->size[c]);
      auto put = [&](ArchiveView view, const float *dev) {
        TRY(tlh_memcpy_d2h(host.data(), dev + p->offset[c], host.size() * sizeof(float),
                           p->stream));
        TRY(tlh_stream_synchronize(p->stream));
        view.write("size", bytes_of(shape));
        view.write("data", bytes_of(host));
        return 0;
      };
      TRY(put(params.scope(std::to_string(i)), p->params));
      if (optimiser) {
        auto state = optimisers.scope(std::to_string(i));
        TRY(put(state.scope("momentum1"), p->m1));
        TRY(put(state.scope("momentum2"), p->m2));
        state.write("step", std::as_bytes(std::span<const uint32_t>(&steps[c], 1)));
      }
    }
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    archive.commit(out);
    out.close();
    return out.good() ? 0 : kInvalidValue;
  } catch (const std::exception &) {
    return kInvalidValue;
  }
}

int tlg_load_archive(void *program, const char *path, int optimiser) {
  Program *p = static_cast<Program *>(program);
  if (!path) return kInvalidValue;
  const uint32_t count = uint32_t(p->size.size());
  // everything is read and checked before anything reaches the device
  std::vector<float> params(p->total), m1, m2;
  std::vector<uint32_t> steps(count);
  if (optimiser) {
    m1.resize(p->total);
    m2.resize(p->total);
  }
  try {
    std::ifstream in(path, std::ios::binary);
    if (!in) return kInvalidValue;
    Archive archive;
    archive.restore(in);
    const auto ps = archive.scope("parameters");
    const auto os = archive.scope("optimisers");
    std::vector<size_t> flat(count + 1, 0); // canonical flat offsets
    for (uint32_t c = 0; c < count; ++c) flat[c + 1] = flat[c] + p->size[c];
    for (uint32_t i = 0; i < count; ++i) {
      uint32_t c = 0, want[2];
      if (!archive_entry(p->cfg, i, c, want)) return kInvalidValue;
      auto get = [&](const ArchiveView &view, std::vector<float> &dst) {
        uint32_t shape[2] = {0, 0};
        view.read("size", std::as_writable_bytes(std::span<uint32_t>(shape, 2)));
        if (shape[0] != want[0] || shape[1] != want[1])
          throw std::runtime_error("tensor shape differs from the program's");
        view.read("data", std::as_writable_bytes(
                              std::span<float>(dst.data() + flat[c], p->size[c])));
      };
      get(ps.scope(std::to_string(i)), params);
      if (optimiser) {
        const auto state = os.scope(std::to_string(i));
        get(state.scope("momentum1"), m1);
        get(state.scope("momentum2"), m2);
        state.read("step", std::as_writable_bytes(std::span<uint32_t>(&steps[c], 1)));
      }
    }
  } catch (const std::exception &) {
    return kInvalidValue;
  }
  TRY(copy_params(*p, p->params, params.data(), true));
  if (optimiser) {
    TRY(copy_params(*p, p->m1, m1.data(), true));
    TRY(copy_params(*p, p->m2, m2.data(), true));
    TRY(tlh_memcpy_h2d(p->steps, steps.data(), count * sizeof(uint32_t), p->stream));
  }
  return tlh_stream_synchronize(p->stream);
}

int tlg_set_batch(void *program, const uint32_t *host_tokens, const uint32_t *host_targets) {
  Program *p = static_cast<Program *>(program);
  if (!host_tokens || !host_targets) return kInvalidValue;
  TRY(tlh_memcpy_h2d(p->tokens, host_tokens, p->R * sizeof(uint32_t), p->stream));
  TRY(tlh_memcpy_h2d(p->targets, host_targets, p->R * sizeof(uint32_t), p->stream));
  return tlh_stream_synchronize(p->stream);
}

int tlg_loader_open(const char *tokens_path, double training_fraction, int validation,
                    uint32_t seed, void **loader) {
  if (!tokens_path || !loader) return kInvalidValue;
  *loader = nullptr;
  try {
    std::ifstream in(tokens_path, std::ios::binary);
    auto *l = new TokenLoader{Dataset::load_tokens(in, training_fraction), {}};
    const Dataset &d = l->dataset;
    l->loader.emplace(validation ? d.validation_split() : d.training_split(), seed);
    *loader = l;
    return 0;
  } catch (const std::exception &) {
    return kInvalidValue;
  }
}

int tlg_loader_batch(void *loader, uint32_t batch, uint32_t seq, uint32_t *host_inputs,
                     uint32_t *host_targets) {
  auto *l = static_cast<TokenLoader *>(loader);
  if (!l || !host_inputs || !host_targets) return kInvalidValue;
  try {
    const Loader::Batch &b = l->loader->get_batch(batch, seq);
    std::copy(b.inputs.begin(), b.inputs.end(), host_inputs);
    std::copy(b.targets.begin(), b.targets.end(), host_targets);
    return 0;
  } catch (const std::exception &) {
    return kInvalidValue;
  }
}

int tlg_loader_next(void *loader, void *program) {
  auto *l = static_cast<TokenLoader *>(loader);
  Program *p = static_cast<Program *>(program);
  if (!l || !p) return kInvalidValue;
  try {
    const Loader::Batch &b = l->loader->get_batch(p->cfg.batch, p->cfg.seq);
    return tlg_set_batch(program, b.inputs.data(), b.targets.data());
  } catch (const std::exception &) {
    return kInvalidValue;
  }
}

int tlg_loader_close(void *loader) {
  delete static_cast<TokenLoader *>(loader);
  return 0;
}

int tlg_capture_train_step(void *program, float root_grad, float max_norm) {
  Program *p = static_cast<Program *>(program);
  if (p->graph) {
    tlh_graph_destroy(p->graph);
    p->graph = nullptr;
  }
  TRY(tlh_stream_synchronize(p->stream));
  TRY(tlh_graph_begin_capture(p->stream));
  const int st = train_step(*p, root_grad, max_norm, 1);
  void *exec = nullptr;
  const int st2 = tlh_graph_end_capture(p->stream, &exec);
  if (st) {
    if (exec) tlh_graph_destroy(exec);
    return st;
  }
  if (st2) return st2;
  p->graph = exec;
  return 0;
}

int tlg_replay(void *program) {
  Program *p = static_cast<Program *>(program);
  if (!p->graph) return 1;
  return tlh_graph_launch(p->graph, p->stream);
}

} // extern "C"
