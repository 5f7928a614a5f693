/*
 * templit_gpt.h -- C-ABI of libtemplit_gpt.so: the GPT training-step
 * program that drives libtemplit_hip.so.
 *
 * This is the program layer above the runtime surface. In the reference
 * the same work is done by passes::Compiled over nn::GPT
 * (include/passes/compile.h:37-304, include/nn/GPT.h:17-69) and the
 * training loop of src/train.cpp:120-187: forward(), backward(root_grad),
 * step(max_norm) with AdamW. Here the step is a fixed sequence of fused
 * gfx950 kernels on one HIP stream with lifetime-planned device buffers,
 * recordable as one hipGraph and replayed every step.
 *
 * Model (nn::GPT): token + position embedding, `layers` pre-RMSNorm decoder
 * blocks (causal multi-head attention with Q/K/V/O linears, GELU FFN of
 * width `ffn`), final RMSNorm, vocabulary projection; loss = per-row
 * cross-entropy. Parameters are fp32 and live in one device allocation in
 * this canonical order (tlg_param_info gives each tensor's offset):
 *   tok [V,D], pos [T,D], per layer: wq [D,D], bq [D], wk, bk, wv, bv,
 *   wo, bo, w1 [D,F], b1 [F], w2 [F,D], b2 [D]; then wp [D,V], bp [V].
 * Weights are stored [in, out] row-major as nn::Layer does (y = x.W + b).
 *
 * Conventions as in templit_hip.h: int return = hipError_t (0 = success),
 * device pointers unless host_*, asynchronous on the program's stream.
 */
#ifndef TEMPLIT_GPT_H
#define TEMPLIT_GPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tlg_config {
  uint32_t vocab, seq, dim, heads, layers, batch, ffn;
} tlg_config;

/* Allocates parameters, gradients, AdamW state and every activation /
 * scratch buffer of one step (nothing is allocated per step). head dim must
 * be 64. `stream` = hipStream_t used for all work. */
int tlg_create(const tlg_config *cfg, void *stream, void **program);
int tlg_destroy(void *program);

/* Parameter table: count, and per tensor its element count and device
 * pointer (params / grads / AdamW moments share one layout). */
int tlg_param_count(void *program, uint32_t *count);
int tlg_param_info(void *program, uint32_t index, uint64_t *size, float **param,
                   float **grad, float **m1, float **m2);
/* Total elements of the flat canonical (unpadded) parameter vector. */
int tlg_total_params(void *program, uint64_t *total);

/* Host <-> device copies of the flat canonical parameter vector. Synchronous. */
int tlg_set_params(void *program, const float *host_params);
int tlg_get_params(void *program, float *host_params);
int tlg_get_grads(void *program, float *host_grads);
int tlg_get_moments(void *program, float *host_m1, float *host_m2);
/* AdamW per-tensor step counters (AdamW::step_, AdamW.h:42,78) and the
 * optimiser scalars {beta1, beta2, decay, lr} as the device holds them. */
int tlg_get_steps(void *program, uint32_t *host_steps);
int tlg_get_scalars(void *program, float *host_scalars4);
/* Device-side init: weights ~ N(0, std) (SplitMix64 + Box-Muller per
 * element), biases 0, moments 0, step counters 0. */
int tlg_init_params(void *program, uint64_t seed, float std);

/* AdamW hyper-parameters (Optimiser::AdamW::Shared, AdamW.h:15-39): lr and
 * decay = 1 - lr*weight_decay live in device scalars, so changing them does
 * not invalidate a captured step. */
int tlg_set_optimizer(void *program, float lr, float beta1, float beta2, float eps,
                      float weight_decay);
int tlg_set_lr(void *program, float lr);

/* Streams of the training step: 1 runs the weight gradients on a second
 * stream beside the chain of input gradients (fork/join events order
 * them), 0 runs the whole step on the program's stream, -1 (the default at
 * tlg_create) picks 1 while the [batch*seq, dim] products have fewer than
 * 4 tiles of 64x64 per compute unit and 0 above. Results are bitwise the
 * same either way (every kernel is deterministic). Applies to steps issued
 * or captured after the call. tlg_get_concurrency reports the choice. */
int tlg_set_concurrency(void *program, int mode);
int tlg_get_concurrency(void *program, int *two_streams);

/* Weight layout of the forward products (no counterpart in the reference):
 * 1 runs them on K-contiguous copies of the weight matrices, rebuilt from
 * the weights by one transpose launch at the start of every forward (so
 * writes through tlg_param_info pointers are seen), 0 on the [in, out]
 * weights themselves, -1 (the default at tlg_create) picks 1 while the
 * [batch*seq, dim] products have fewer than 4 tiles of 64x64 per compute
 * unit and 0 above. Results are bitwise the same either way.
 * Applies to forwards issued or captured after the call. */
int tlg_set_forward_copies(void *program, int mode);
int tlg_get_forward_copies(void *program, int *copies);

/* Device buffers the step reads its batch from (uint32 [B*T] each) and
 * writes per-row losses to (float [B*T]); stable for the program's life. */
int tlg_io(void *program, uint32_t **tokens, uint32_t **targets, float **losses,
           float **logits);

/* One training step on the batch in the io buffers: forward, per-row loss,
 * backward with uniform root gradient `root_grad` (src/train.cpp:109-113),
 * global squared gradient norm, clip to max_norm (if > 0) and AdamW.
 * update = 0 runs forward + backward only (gradients left in grad buffers). */
int tlg_train_step(void *program, float root_grad, float max_norm, int update);
/* Forward only: logits [B*T, V] into the io logits buffer. */
int tlg_forward(void *program);
/* Greedy autoregressive generation (inference::autoregression,
 * include/inference.h:45-99, with top_k = 1): the program must have
 * batch 1; its window of `seq` tokens starts as the prompt followed by
 * eos_token padding. Each of n_new steps runs the forward, takes the
 * lowest-index argmax of the logits at the last valid position, appends it
 * (sliding the window once full) and stores it in host_out[step]; EOS does
 * not end generation. prefix_only = 0 recomputes the whole padded window
 * as the reference does; 1 computes only the valid prefix, which gives the
 * same logits because attention is causal; 2 keeps the window's keys and
 * values (KV cache): after one window forward each new position runs alone
 * through the blocks (tlh_attention_decode over the cached keys) until the
 * window is full, then it recomputes as 0 does. Modes 1 and 2 compute the
 * same quantities as 0 in a different order, so their logits agree with
 * mode 0's to rounding. Synchronous. */
int tlg_generate_greedy(void *program, const uint32_t *host_prompt, uint32_t prompt_len,
                        uint32_t n_new, uint32_t eos_token, int prefix_only,
                        uint32_t *host_out);

/* Sampled autoregressive generation, inference::autoregression
 * (include/inference.h:45-99) with inference::sample_top_k (14-43) on the
 * device (tlh_sample_top_k): the window and the three prefix_only modes are
 * tlg_generate_greedy's; each step samples the next token from the top_k
 * logits at temperature `temperature`, drawing again while it is eos_token
 * and fewer than min(minimum_length, seq) tokens were generated, and
 * generation ends after an emitted eos_token or n_new tokens. Uniforms come
 * from the SplitMix64 stream seeded with `seed`, each draw taking the next
 * output (the reference's std::mt19937 is a host-side choice). The tokens
 * go to host_out, their number to *host_count. Synchronous. */
int tlg_generate_sample(void *program, const uint32_t *host_prompt, uint32_t prompt_len,
                        uint32_t n_new, uint32_t eos_token, uint32_t top_k, float temperature,
                        uint32_t minimum_length, uint64_t seed, int prefix_only,
                        uint32_t *host_out, uint32_t *host_count);

/* Squared gradient norm of the last step (host read, synchronous). */
int tlg_last_squared_norm(void *program, float *host_value);

/* One eager training step, every launch on the program's stream, with HIP
 * events around every GEMM launch and every attention launch: returns the
 * summed GEMM time (ms), the GEMMs' algorithmic flops (2*M*N*K each) and
 * algorithmic HBM bytes (every operand read once, every result written
 * once: A, B, C, bias, residual, beta*C, the GELU pre-activation, the bias
 * gradient), the number of GEMM launches, the summed attention time and the
 * whole step's time. */
int tlg_profile_step(void *program, float root_grad, float max_norm, float *host_gemm_ms,
                     double *host_gemm_flops, double *host_gemm_bytes,
                     uint32_t *host_gemm_launches, float *host_attention_ms,
                     float *host_step_ms);

/* Kernel time of the GEMMs of the last tlg_profile_step: each of its GEMM
 * launches is repeated `iters` times back to back between two HIP events on
 * the program's stream; *host_ms = sum over the step's launches of the
 * per-launch time (ms). Rewrites the step's scratch and gradient buffers. */
int tlg_time_gemms(void *program, uint32_t iters, float *host_ms);

/* Checkpoints in the reference's archive format (include/model_utils/
 * archive.h, src/model_utils/archive.cpp:9-92), holding what
 * passes::Compiled::save and save_optimisers write
 * (include/passes/compile.h:259-299): for each parameter i in the
 * reference's gradient-path order
 *   parameters/<i>/size  u32 shape ([in, out] weights, [1, n] biases,
 *                        [V, D] token and [T, D] position tables)
 *   parameters/<i>/data  fp32 values
 * and, with `optimiser` != 0, AdamW's state (include/optimiser/
 * AdamW.h:84-106)
 *   optimisers/<i>/momentum1/size|data, optimisers/<i>/momentum2/size|data,
 *   optimisers/<i>/step  u32.
 * The order runs over the blocks from the last to the first, each as
 * w1, b1, w2, b2, wq, bq, wk, bk, wv, bv, wo, bo, then the token and
 * position tables, then the vocabulary projection wp, bp.
 * Save and load are synchronous; load checks every shape and size and
 * leaves the program unchanged on a mismatch (hipErrorInvalidValue). */
int tlg_save_archive(void *program, const char *path, int optimiser);
int tlg_load_archive(void *program, const char *path, int optimiser);
/* Host-only: the canonical parameter index (tlg_param_info order) and the
 * 2-d shape of archive entry `index` for `cfg`. */
int tlg_archive_entry(const tlg_config *cfg, uint32_t index, uint32_t *canonical,
                      uint32_t *shape2);

/* Host batch -> the program's token and target buffers (batch*seq uint32
 * ids each, row-major). Synchronous. */
int tlg_set_batch(void *program, const uint32_t *host_tokens, const uint32_t *host_targets);

/* Token-file loader (src/train.cpp:75-77, 142): Dataset::load_tokens of a
 * raw uint32 file with the reference's split at `training_fraction`
 * (src/model_utils/dataset.cpp:16-102) and a Loader over its training
 * (validation = 0) or validation split seeded with `seed`
 * (src/model_utils/loader.cpp:5-43); the same batches as the reference's
 * for one seed. tlg_loader_batch draws the next batch to the host;
 * tlg_loader_next draws it for a program's (batch, seq) and uploads it
 * (tlg_set_batch). hipErrorInvalidValue for unreadable files, bad
 * fractions or sizes. */
int tlg_loader_open(const char *tokens_path, double training_fraction, int validation,
                    uint32_t seed, void **loader);
int tlg_loader_batch(void *loader, uint32_t batch, uint32_t seq, uint32_t *host_inputs,
                     uint32_t *host_targets);
int tlg_loader_next(void *loader, void *program);
int tlg_loader_close(void *loader);

/* Records tlg_train_step(root_grad, max_norm, 1) as a hipGraph; replays it. */
int tlg_capture_train_step(void *program, float root_grad, float max_norm);
int tlg_replay(void *program);

#ifdef __cplusplus
}
#endif

#endif
