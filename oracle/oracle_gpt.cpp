// GPT training step for the CPU oracle -- TEST INFRASTRUCTURE ONLY.
//
// Restates the model of include/nn/GPT.h:62-68 (token + position embedding,
// `layers` pre-RMSNorm decoder blocks of include/nn/decoder_block.h:27-43
// with the attention of include/nn/multi_head.h:33-55 and a GELU FFN, a final
// RMSNorm and the projection Layer), the cross-entropy loss
// (include/expr/cross-entropy.h:16-21), the backward pass the reference
// autograd produces for it (written out by hand, composed of the oracle ops
// of oracle.cpp), Compiled::step(max_norm) (include/passes/compile.h:236-258)
// and Optimiser::AdamW::update (include/optimiser/AdamW.h:73-82).
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace {

using Vec = std::vector<float>;

struct Shapes {
  uint32_t V, T, D, H, L, B, F;
  size_t rows() const { return size_t(B) * T; }
};

struct ParamView {
  std::vector<float *> p;
  std::vector<size_t> n;
};

uint32_t param_count(const orc_gpt_config &c) { return 2 + 12 * c.layers + 2; }

size_t param_size(const orc_gpt_config &c, uint32_t i) {
  const size_t V = c.vocab, T = c.seq, D = c.dim, F = c.ffn;
  if (i == 0) return V * D;
  if (i == 1) return T * D;
  const uint32_t last = 2 + 12 * c.layers;
  if (i == last) return D * V;
  if (i == last + 1) return V;
  switch ((i - 2) % 12) {
  case 0: case 2: case 4: case 6: return D * D;
  case 1: case 3: case 5: case 7: return D;
  case 8: return D * F;
  case 9: return F;
  case 10: return F * D;
  default: return D;
  }
}

ParamView view(const orc_gpt_config &c, float *base) {
  ParamView v;
  size_t off = 0;
  for (uint32_t i = 0; i < param_count(c); ++i) {
    v.p.push_back(base + off);
    v.n.push_back(param_size(c, i));
    off += param_size(c, i);
  }
  return v;
}

// y[r,:] = x[r,:] . W + b  (EXPR_LINEAR: mult then in-place bias add,
// execute.h:241-252).
void linear(const float *x, const float *w, const float *b, float *y, size_t rows, size_t in,
            size_t out) {
  orc_matmul(x, w, y, uint32_t(rows), uint32_t(in), uint32_t(out), 0, nullptr, nullptr,
             nullptr);
  for (size_t r = 0; r < rows; ++r)
    for (size_t j = 0; j < out; ++j) y[r * out + j] = y[r * out + j] + b[j];
}

// Weight gradient X^T.dY (MULT_RHS_DERIVATIVE, execute.h:209-232: transpose
// the left operand, then mult).
void weight_grad(const float *x, const float *dy, float *dw, size_t rows, size_t in,
                 size_t out) {
  Vec xt(in * rows);
  for (size_t r = 0; r < rows; ++r)
    for (size_t i = 0; i < in; ++i) xt[i * rows + r] = x[r * in + i];
  orc_matmul(xt.data(), dy, dw, uint32_t(in), uint32_t(rows), uint32_t(out), 0, nullptr,
             nullptr, nullptr);
}

// Input gradient dY.W^T (MULT_LHS_DERIVATIVE, execute.h:186-208).
void input_grad(const float *dy, const float *w, float *dx, size_t rows, size_t in,
                size_t out) {
  Vec wt(out * in);
  for (size_t i = 0; i < in; ++i)
    for (size_t j = 0; j < out; ++j) wt[j * in + i] = w[i * out + j];
  orc_matmul(dy, wt.data(), dx, uint32_t(rows), uint32_t(out), uint32_t(in), 0, nullptr,
             nullptr, nullptr);
}

// Bias gradient: sum_to_shape([rows, out] -> [1, out]) (cpu.cpp reduce axis 0).
void bias_grad(const float *dy, float *db, size_t rows, size_t out) {
  for (size_t j = 0; j < out; ++j) db[j] = 0.0f;
  for (size_t r = 0; r < rows; ++r)
    for (size_t j = 0; j < out; ++j) db[j] += dy[r * out + j];
}

// [B,T,H,dh] (merged rows) <-> [B,H,T,dh] (split_last_dim + transpose<1,2>).
void to_heads(const float *x, float *h, const Shapes &s) {
  const size_t dh = s.D / s.H;
  for (size_t b = 0; b < s.B; ++b)
    for (size_t t = 0; t < s.T; ++t)
      for (size_t hh = 0; hh < s.H; ++hh)
        std::memcpy(h + ((b * s.H + hh) * s.T + t) * dh, x + (b * s.T + t) * s.D + hh * dh,
                    dh * sizeof(float));
}

void from_heads(const float *h, float *x, const Shapes &s) {
  const size_t dh = s.D / s.H;
  for (size_t b = 0; b < s.B; ++b)
    for (size_t t = 0; t < s.T; ++t)
      for (size_t hh = 0; hh < s.H; ++hh)
        std::memcpy(x + (b * s.T + t) * s.D + hh * dh, h + ((b * s.H + hh) * s.T + t) * dh,
                    dh * sizeof(float));
}

void add_inplace(float *a, const float *b, size_t n) {
  for (size_t i = 0; i < n; ++i) a[i] = a[i] + b[i];
}

struct LayerCache {
  Vec x_in, n1, q, k, v, qh, kh, vh, probs, oh, o, x_mid, n2, u, g;
};

constexpr float kRmsEps = 1e-6f; // runtime.cpp:1044

struct Forward {
  std::vector<LayerCache> layers;
  Vec x_final, nf, logits;
};

void forward(const orc_gpt_config &c, const ParamView &P, const uint32_t *tokens, Forward &f) {
  const Shapes s{c.vocab, c.seq, c.dim, c.heads, c.layers, c.batch, c.ffn};
  const size_t R = s.rows(), D = s.D, F = s.F, dh = D / s.H;
  // Embeddings: add(embedding_lookup(tok, input), embedding_lookup(pos, positions))
  Vec x(R * D), pe(R * D);
  std::vector<uint32_t> positions(R);
  for (size_t r = 0; r < R; ++r) positions[r] = uint32_t(r % s.T);
  orc_embedding_lookup(P.p[0], uint32_t(D), tokens, R, x.data());
  orc_embedding_lookup(P.p[1], uint32_t(D), positions.data(), R, pe.data());
  add_inplace(x.data(), pe.data(), R * D);

  f.layers.assign(s.L, {});
  for (uint32_t l = 0; l < s.L; ++l) {
    LayerCache &L = f.layers[l];
    float *const *w = P.p.data() + 2 + 12 * l;
    L.x_in = x;
    L.n1.resize(R * D);
    orc_rms_norm(x.data(), nullptr, L.n1.data(), nullptr, R, uint32_t(D), kRmsEps);
    L.q.resize(R * D); L.k.resize(R * D); L.v.resize(R * D);
    linear(L.n1.data(), w[0], w[1], L.q.data(), R, D, D);
    linear(L.n1.data(), w[2], w[3], L.k.data(), R, D, D);
    linear(L.n1.data(), w[4], w[5], L.v.data(), R, D, D);
    L.qh.resize(R * D); L.kh.resize(R * D); L.vh.resize(R * D);
    to_heads(L.q.data(), L.qh.data(), s);
    to_heads(L.k.data(), L.kh.data(), s);
    to_heads(L.v.data(), L.vh.data(), s);
    L.probs.resize(size_t(s.B) * s.H * s.T * s.T);
    L.oh.resize(R * D);
    orc_attention_forward(L.qh.data(), L.kh.data(), L.vh.data(), L.oh.data(), L.probs.data(),
                          s.B, s.H, s.T, uint32_t(dh), 1);
    L.o.resize(R * D);
    from_heads(L.oh.data(), L.o.data(), s);
    Vec a(R * D);
    linear(L.o.data(), w[6], w[7], a.data(), R, D, D);
    L.x_mid = L.x_in;
    add_inplace(L.x_mid.data(), a.data(), R * D);
    L.n2.resize(R * D);
    orc_rms_norm(L.x_mid.data(), nullptr, L.n2.data(), nullptr, R, uint32_t(D), kRmsEps);
    L.u.resize(R * F);
    linear(L.n2.data(), w[8], w[9], L.u.data(), R, D, F);
    L.g.resize(R * F);
    orc_unary(ORC_GELU, L.u.data(), L.g.data(), R * F);
    Vec ff(R * D);
    linear(L.g.data(), w[10], w[11], ff.data(), R, F, D);
    x = L.x_mid;
    add_inplace(x.data(), ff.data(), R * D);
  }
  f.x_final = x;
  f.nf.resize(R * D);
  orc_rms_norm(x.data(), nullptr, f.nf.data(), nullptr, R, uint32_t(D), kRmsEps);
  const uint32_t last = 2 + 12 * s.L;
  f.logits.resize(R * s.V);
  linear(f.nf.data(), P.p[last], P.p[last + 1], f.logits.data(), R, D, s.V);
}

} // namespace

extern "C" {

uint32_t orc_gpt_param_count(const orc_gpt_config *cfg) { return param_count(*cfg); }

uint64_t orc_gpt_param_size(const orc_gpt_config *cfg, uint32_t index) {
  return param_size(*cfg, index);
}

uint64_t orc_gpt_total_params(const orc_gpt_config *cfg) {
  uint64_t t = 0;
  for (uint32_t i = 0; i < param_count(*cfg); ++i) t += param_size(*cfg, i);
  return t;
}

int orc_gpt_forward(const orc_gpt_config *cfg, const float *params, const uint32_t *tokens,
                    float *logits) {
  if (cfg->dim % cfg->heads) return 1;
  ParamView P = view(*cfg, const_cast<float *>(params));
  Forward f;
  forward(*cfg, P, tokens, f);
  std::memcpy(logits, f.logits.data(), f.logits.size() * sizeof(float));
  return 0;
}

int orc_gpt_train_step(const orc_gpt_config *cfg, float *params, float *m, float *v,
                       uint32_t step, const uint32_t *tokens, const uint32_t *targets,
                       float root_grad, float lr, float beta1, float beta2, float eps,
                       float weight_decay, float max_norm, float *losses, float *grads,
                       float *squared_norm) {
  const orc_gpt_config &c = *cfg;
  if (c.dim % c.heads) return 1;
  const Shapes s{c.vocab, c.seq, c.dim, c.heads, c.layers, c.batch, c.ffn};
  const size_t R = s.rows(), D = s.D, F = s.F, V = s.V, dh = D / s.H;
  ParamView P = view(c, params);
  ParamView G = view(c, grads);
  Forward f;
  forward(c, P, tokens, f);
  orc_cross_entropy_rows(f.logits.data(), targets, losses, R, uint32_t(V));

  // ---- backward ----
  // dlogits = CE'(logits, t) (hadamard) root_grad  (autograd of X_ENTROPY)
  Vec dlogits(R * V);
  orc_cross_entropy_rows_backward(f.logits.data(), targets, dlogits.data(), R, uint32_t(V));
  for (size_t r = 0; r < R; ++r)
    for (size_t j = 0; j < V; ++j) dlogits[r * V + j] = dlogits[r * V + j] * root_grad;
  const uint32_t last = 2 + 12 * s.L;
  weight_grad(f.nf.data(), dlogits.data(), G.p[last], R, D, V);
  bias_grad(dlogits.data(), G.p[last + 1], R, V);
  Vec dnf(R * D);
  input_grad(dlogits.data(), P.p[last], dnf.data(), R, D, V);
  Vec dx(R * D);
  orc_rms_norm_backward(dnf.data(), f.x_final.data(), nullptr, dx.data(), nullptr, R,
                        uint32_t(D), kRmsEps);

  Vec tmpD(R * D), dg(R * F), dn(R * D);
  for (int l = int(s.L) - 1; l >= 0; --l) {
    LayerCache &L = f.layers[l];
    float *const *w = P.p.data() + 2 + 12 * l;
    float *const *gw = G.p.data() + 2 + 12 * l;
    // FFN branch: x = x_mid + W2.GELU(W1.RMSNorm(x_mid))
    weight_grad(L.g.data(), dx.data(), gw[10], R, F, D);
    bias_grad(dx.data(), gw[11], R, D);
    input_grad(dx.data(), w[10], dg.data(), R, F, D);
    for (size_t i = 0; i < R * F; ++i) {
      float gd;
      orc_unary(ORC_GELU_DERIVATIVE, &L.u[i], &gd, 1);
      dg[i] = dg[i] * gd;
    }
    weight_grad(L.n2.data(), dg.data(), gw[8], R, D, F);
    bias_grad(dg.data(), gw[9], R, F);
    input_grad(dg.data(), w[8], dn.data(), R, D, F);
    orc_rms_norm_backward(dn.data(), L.x_mid.data(), nullptr, tmpD.data(), nullptr, R,
                          uint32_t(D), kRmsEps);
    add_inplace(dx.data(), tmpD.data(), R * D); // dx_mid = residual + norm path
    // attention branch: x_mid = x_in + Wo.attn(RMSNorm(x_in))
    weight_grad(L.o.data(), dx.data(), gw[6], R, D, D);
    bias_grad(dx.data(), gw[7], R, D);
    Vec dO(R * D), dOh(R * D), dqh(R * D), dkh(R * D), dvh(R * D);
    input_grad(dx.data(), w[6], dO.data(), R, D, D);
    to_heads(dO.data(), dOh.data(), s);
    orc_attention_backward(L.qh.data(), L.kh.data(), L.vh.data(), L.probs.data(), dOh.data(),
                           dqh.data(), dkh.data(), dvh.data(), s.B, s.H, s.T, uint32_t(dh));
    Vec dq(R * D), dk(R * D), dv(R * D);
    from_heads(dqh.data(), dq.data(), s);
    from_heads(dkh.data(), dk.data(), s);
    from_heads(dvh.data(), dv.data(), s);
    weight_grad(L.n1.data(), dq.data(), gw[0], R, D, D);
    bias_grad(dq.data(), gw[1], R, D);
    weight_grad(L.n1.data(), dk.data(), gw[2], R, D, D);
    bias_grad(dk.data(), gw[3], R, D);
    weight_grad(L.n1.data(), dv.data(), gw[4], R, D, D);
    bias_grad(dv.data(), gw[5], R, D);
    Vec dn1(R * D), part(R * D);
    input_grad(dq.data(), w[0], dn1.data(), R, D, D);
    input_grad(dk.data(), w[2], part.data(), R, D, D);
    add_inplace(dn1.data(), part.data(), R * D);
    input_grad(dv.data(), w[4], part.data(), R, D, D);
    add_inplace(dn1.data(), part.data(), R * D);
    orc_rms_norm_backward(dn1.data(), L.x_in.data(), nullptr, tmpD.data(), nullptr, R,
                          uint32_t(D), kRmsEps);
    add_inplace(dx.data(), tmpD.data(), R * D);
  }
  // embeddings: scatter_index (zero, then scatter_add_rows) for both tables
  std::memset(G.p[0], 0, G.n[0] * sizeof(float));
  std::memset(G.p[1], 0, G.n[1] * sizeof(float));
  std::vector<uint32_t> positions(R);
  for (size_t r = 0; r < R; ++r) positions[r] = uint32_t(r % s.T);
  orc_scatter_add_rows(dx.data(), tokens, R, uint32_t(D), G.p[0]);
  orc_scatter_add_rows(dx.data(), positions.data(), R, uint32_t(D), G.p[1]);

  // ---- step(max_norm): norm over every gradient, clip, AdamW ----
  *squared_norm = 0.0f;
  for (uint32_t i = 0; i < param_count(c); ++i)
    orc_accumulate_gradient_squared_norm(G.p[i], G.n[i], squared_norm);
  if (max_norm <= 0.0f) return 0;
  const float decay = 1.0f - lr * weight_decay; // AdamW.h:28-29
  ParamView M1 = view(c, m), M2 = view(c, v);
  Vec clipped;
  for (uint32_t i = 0; i < param_count(c); ++i) {
    clipped.resize(G.n[i]);
    orc_clip_gradient(G.p[i], squared_norm, max_norm, clipped.data(), G.n[i]);
    orc_adamw(P.p[i], clipped.data(), P.p[i], M1.p[i], M2.p[i], beta1, beta2, decay, lr, eps,
              step, G.n[i]);
  }
  return 0;
}

} // extern "C"
