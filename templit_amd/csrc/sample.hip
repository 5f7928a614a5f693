// Top-k sampling with temperature on the device: replaces the host loop of
// inference::sample_top_k (include/inference.h:14-43) and the EOS re-draw of
// inference::autoregression (inference.h:80-84), so that a generation step
// reads back one token instead of the vocabulary's logits.
//
// One 256-thread block per row. The row's (logit, token) pairs are sorted in
// LDS by a bitonic network -- logit descending, equal logits lower token
// first, NaN as -INF -- into the top-k candidates. Weights, normalisation
// and the draw follow the reference's fp32 weights and libstdc++'s
// std::discrete_distribution: w_i = exp((l_i - l_0) / T) (fp32 difference
// and quotient; the exponential in double, rounded to fp32), S = the double
// sum of the w_i in candidate order, cumulative sums of w_i / S in double
// with the last set to 1, and the first candidate whose cumulative sum is
// >= u. The uniforms u come from the caller (one per draw) or from the
// SplitMix64 stream seeded with `seed`: draw d of row r takes its output
// number counter + r * max_draws + d + 1, as (x >> 11) * 2^-53.
#include "common.h"

namespace tlh {
namespace {

constexpr uint32_t kMaxSampleVocab = 4096; // sort size; keys + ids + terms fill 64 KiB

__device__ inline double splitmix_uniform(uint64_t seed, uint64_t n) {
  uint64_t z = seed + (n + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return double(z >> 11) * (1.0 / 9007199254740992.0);
}

// `a` comes before `b`: larger logit, or equal logit and lower token.
__device__ inline bool before(float ka, uint32_t ia, float kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

template <uint32_t P>
__global__ __launch_bounds__(256) void sample_top_k_kernel(
    const float *logits, uint32_t vocab, uint32_t row_stride, uint32_t k, float temperature,
    uint64_t seed, uint64_t counter, const double *uniforms, uint32_t eos_token,
    int resample_eos, uint32_t max_draws, uint32_t *tokens, uint32_t *draws) {
  __shared__ float key[P];
  __shared__ uint32_t id[P];
  __shared__ double term[P]; // w_i / S of the candidates (term[0] first carries S)
  const uint32_t tid = threadIdx.x, row = blockIdx.x;
  const float *x = logits + size_t(row) * row_stride;
  for (uint32_t i = tid; i < P; i += 256) {
    float v = -INFINITY;
    uint32_t t = 0xffffffffu; // padding sorts after every token
    if (i < vocab) {
      v = x[i];
      if (v != v) v = -INFINITY;
      t = i;
    }
    key[i] = v;
    id[i] = t;
  }
  __syncthreads();
  // bitonic sort of P entries into the `before` order
  for (uint32_t size = 2; size <= P; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (uint32_t i = tid; i < P / 2; i += 256) {
        const uint32_t lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
        const bool up = (lo & size) == 0;
        const float kl = key[lo], kh = key[hi];
        const uint32_t il = id[lo], ih = id[hi];
        if (before(kh, ih, kl, il) == up) {
          key[lo] = kh;
          key[hi] = kl;
          id[lo] = ih;
          id[hi] = il;
        }
      }
      __syncthreads();
    }
  }
  const float maximum = key[0];
  __syncthreads();
  for (uint32_t i = tid; i < k; i += 256)
    key[i] = float(exp(double((key[i] - maximum) / temperature)));
  __syncthreads();
  if (tid == 0) {
    double s = 0.0;
    for (uint32_t i = 0; i < k; ++i) s += double(key[i]);
    term[0] = s;
  }
  __syncthreads();
  const double total = term[0];
  __syncthreads();
  for (uint32_t i = tid; i < k; i += 256) term[i] = double(key[i]) / total;
  __syncthreads();
  if (tid != 0) return;
  uint32_t token = 0, d = 0;
  for (; d < max_draws; ++d) {
    const uint64_t n = counter + uint64_t(row) * max_draws + d;
    const double u = uniforms ? uniforms[size_t(row) * max_draws + d] : splitmix_uniform(seed, n);
    uint32_t pick = k - 1;
    double c = 0.0;
    for (uint32_t i = 0; i + 1 < k; ++i) {
      c += term[i];
      if (c >= u) {
        pick = i;
        break;
      }
    }
    token = id[pick];
    if (!(resample_eos && token == eos_token)) {
      ++d;
      break;
    }
  }
  tokens[row] = token;
  if (draws) draws[row] = d < max_draws ? d : max_draws;
}

template <uint32_t P>
void launch_sample(uint32_t rows, hipStream_t s, const float *logits, uint32_t vocab,
                   uint32_t row_stride, uint32_t k, float temperature, uint64_t seed,
                   uint64_t counter, const double *uniforms, uint32_t eos_token, int resample_eos,
                   uint32_t max_draws, uint32_t *tokens, uint32_t *draws) {
  sample_top_k_kernel<P><<<rows, 256, 0, s>>>(logits, vocab, row_stride, k, temperature, seed,
                                               counter, uniforms, eos_token, resample_eos,
                                               max_draws, tokens, draws);
}

} // namespace
} // namespace tlh

#include "../../include/templit_hip.h"

TLH_API int tlh_sample_top_k(const float *logits, uint32_t rows, uint32_t vocab,
                             uint32_t row_stride, uint32_t top_k, float temperature,
                             uint64_t seed, uint64_t counter, const double *uniforms,
                             uint32_t eos_token, int resample_eos, uint32_t max_draws,
                             uint32_t *tokens, uint32_t *draws, void *stream) {
  using namespace tlh;
  if (!logits || !tokens || rows == 0 || rows > 65535 || vocab == 0 ||
      vocab > kMaxSampleVocab || (rows > 1 && row_stride < vocab) || max_draws == 0 ||
      !(temperature > 0.0f) || !(temperature < INFINITY))
    return int(hipErrorInvalidValue);
  const uint32_t k = top_k < 1 ? 1 : (top_k > vocab ? vocab : top_k);
  hipStream_t s = as_stream(stream);
#define TLH_SAMPLE(P)                                                                         \
  launch_sample<P>(rows, s, logits, vocab, row_stride, k, temperature, seed, counter,         \
                   uniforms, eos_token, resample_eos, max_draws, tokens, draws)
  if (vocab <= 256) TLH_SAMPLE(256);
  else if (vocab <= 512) TLH_SAMPLE(512);
  else if (vocab <= 1024) TLH_SAMPLE(1024);
  else if (vocab <= 2048) TLH_SAMPLE(2048);
  else TLH_SAMPLE(4096);
#undef TLH_SAMPLE
  return launch_status();
}
