/*
 * oracle.h -- CPU oracle for the TempLit runtime hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path
 * is compared against; it is imported only by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg. The product
 * (libtemplit_hip.so, libtemplit_gpt.so) never links or calls it.
 *
 * It restates, single-threaded and in fp32 like the reference:
 *   - the reference CPU runtime (src/CPU/cpu.cpp:14-532,
 *     include/CPU/runtime.h:19-124), generalised from rank 2 to rank N;
 *   - the Metal kernels (include/my_metal/math.metal) and the host
 *     composites of src/my_metal/runtime.cpp where the CPU runtime lacks
 *     the op;
 *   - the executor composites of include/passes/execute.h (softmax',
 *     RMSNorm', matmul derivatives) and the AdamW host logic of
 *     include/optimiser/AdamW.h;
 *   - the GPT of include/nn/GPT.h as a training step (forward, backward by
 *     hand-derived gradients, global clip, AdamW).
 * Every function cites the reference lines it follows. How each one is
 * pinned (golden vectors, reference CPU runtime, closed forms) is listed in
 * the oracle's test files under tests/.
 */
#ifndef TEMPLIT_ORACLE_H
#define TEMPLIT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- portable synthetic data (SplitMix64 + Box-Muller in double) ---- */
void orc_fill_normal(float *out, size_t n, uint64_t seed, float mean, float std);
void orc_fill_uniform_u32(uint32_t *out, size_t n, uint64_t seed, uint32_t bound);

/* ---- elementwise ---- */
enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3 };
void orc_binary(int op, const float *a, const float *b, float *out, uint32_t ndim,
                const uint32_t *out_shape, const uint32_t *stride_a,
                const uint32_t *stride_b);
enum { ORC_SQRT = 0, ORC_EXP = 1, ORC_SIGMOID = 2, ORC_GELU = 3,
       ORC_GELU_DERIVATIVE = 4, ORC_COPY = 5 };
void orc_unary(int op, const float *a, float *out, size_t n);
enum { ORC_ADD_SCALAR = 0, ORC_DIVIDE_SCALAR = 1, ORC_POW_SCALAR = 2 };
void orc_scalar(int op, const float *a, float s, float *out, size_t n);
void orc_transpose(const float *a, float *out, uint32_t ndim, const uint32_t *out_shape,
                   const uint32_t *in_strides);

/* ---- matmul ---- */
void orc_matmul(const float *a, const float *b, float *c, uint32_t M, uint32_t K,
                uint32_t N, uint32_t batch_ndim, const uint32_t *batch_shape,
                const uint32_t *batch_stride_a, const uint32_t *batch_stride_b);

/* ---- reductions ---- */
float orc_sum(const float *a, size_t n);
void orc_sum_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                      const uint32_t *out_shape);
void orc_max_to_shape(const float *a, float *out, uint32_t ndim, const uint32_t *a_shape,
                      const uint32_t *out_shape);
uint32_t orc_argmax(const float *a, size_t n);

/* ---- row ops ---- */
void orc_softmax(const float *x, float *out, size_t rows, uint32_t cols);
void orc_softmax_backward(const float *g, const float *y, float *out, size_t rows,
                          uint32_t cols);
void orc_cross_entropy_rows(const float *logits, const uint32_t *targets, float *losses,
                            size_t rows, uint32_t vocab);
void orc_cross_entropy_rows_backward(const float *logits, const uint32_t *targets,
                                     float *grad, size_t rows, uint32_t vocab);
void orc_rms(const float *x, float *rms, size_t rows, uint32_t cols, float eps);
void orc_rms_norm(const float *x, const float *gain, float *y, float *rms_out,
                  size_t rows, uint32_t cols, float eps);
void orc_rms_norm_backward(const float *g, const float *x, const float *gain, float *dx,
                           float *grad_gain, size_t rows, uint32_t cols, float eps);

/* ---- embedding ---- */
void orc_embedding_lookup(const float *w, uint32_t dim, const uint32_t *ids, size_t n_ids,
                          float *out);
void orc_scatter_add_rows(const float *values, const uint32_t *ids, size_t n_ids,
                          uint32_t dim, float *dst);

/* ---- optimiser ---- */
void orc_accumulate_gradient_squared_norm(const float *g, size_t n, float *squared_norm);
void orc_clip_gradient(const float *g, const float *squared_norm, float max_norm,
                       float *out, size_t n);
void orc_adamw(const float *param, const float *grad, float *out, float *m1, float *m2,
               float beta1, float beta2, float decay, float lr, float eps, uint32_t step,
               size_t n);

/* ---- attention (the decomposed chain of include/nn/multi_head.h:33-55) ---- */
void orc_attention_forward(const float *q, const float *k, const float *v, float *o,
                           float *probs, uint32_t B, uint32_t H, uint32_t T, uint32_t D,
                           int causal);
void orc_attention_backward(const float *q, const float *k, const float *v,
                            const float *probs, const float *dout, float *dq, float *dk,
                            float *dv, uint32_t B, uint32_t H, uint32_t T, uint32_t D);

/* ---- top-k sampling (include/inference.h:14-43, 80-84) ----
 * Per row: the top_k (clamped to [1, vocab]) largest logits in descending
 * order (equal logits: lower token first; NaN ranks as -INF), weights
 * w_i = exp((l_i - l_0) / temperature) with the difference and quotient in
 * fp32 and the exponential rounded to fp32 from double, then the
 * discrete_distribution draw: cumulative sums of w_i / S in double
 * (S = the double sum of the w_i in order), the last set to 1, and the first
 * candidate whose cumulative sum is >= u. Draw d of row r uses
 * u = uniforms[r * max_draws + d] when uniforms is given, else the
 * (counter + r * max_draws + d + 1)-th output x of the SplitMix64 stream
 * seeded with `seed`, as (x >> 11) * 2^-53. With resample_eos, a draw that
 * yields eos_token is repeated with the next u, at most max_draws draws in
 * all (the last result stands). tokens[r] = the token, draws[r] = the draws
 * used. */
void orc_sample_top_k(const float *logits, uint32_t rows, uint32_t vocab, uint32_t row_stride,
                      uint32_t top_k, float temperature, uint64_t seed, uint64_t counter,
                      const double *uniforms, uint32_t eos_token, int resample_eos,
                      uint32_t max_draws, uint32_t *tokens, uint32_t *draws);

/* ---- GPT training step (include/nn/GPT.h, src/train.cpp loop body) ---- */
typedef struct orc_gpt_config {
  uint32_t vocab, seq, dim, heads, layers, batch, ffn;
} orc_gpt_config;

/* Parameter tensors in canonical order (count = 2 + 12*layers + 2):
 *   tok [V,D], pos [T,D], per layer: wq [D,D], bq [D], wk, bk, wv, bv,
 *   wo, bo, w1 [D,F], b1 [F], w2 [F,D], b2 [D]; then wp [D,V], bp [V]. */
uint32_t orc_gpt_param_count(const orc_gpt_config *cfg);
uint64_t orc_gpt_param_size(const orc_gpt_config *cfg, uint32_t index);
uint64_t orc_gpt_total_params(const orc_gpt_config *cfg);

/* One training step on `params` (flat, canonical order). Writes per-row
 * losses [B*T], gradients (flat, before clipping), the squared gradient
 * norm, and updates params/m/v in place with clip(max_norm) + AdamW.
 * If max_norm <= 0 no clipping and no AdamW step are done (forward +
 * backward only). Returns 0 on success. */
int orc_gpt_train_step(const orc_gpt_config *cfg, float *params, float *m, float *v,
                       uint32_t step, const uint32_t *tokens, const uint32_t *targets,
                       float root_grad, float lr, float beta1, float beta2, float eps,
                       float weight_decay, float max_norm, float *losses, float *grads,
                       float *squared_norm);

/* Forward only: logits [B*T, V]. */
int orc_gpt_forward(const orc_gpt_config *cfg, const float *params, const uint32_t *tokens,
                    float *logits);

#ifdef __cplusplus
}
#endif

#endif
