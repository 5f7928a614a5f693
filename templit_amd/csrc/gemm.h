// Host-side descriptor of the fp32 MFMA GEMM (shared by the C-ABI entry
// points and the GPT step program).
#pragma once

#include <cstddef>
#include <cstdint>

namespace tlh {

enum GemmEpilogue : int {
  kEpiStore = 0,   // C = acc (+bias) (+beta*C) (+residual)
  kEpiGelu = 1,    // aux = acc + bias ; C = GELU(aux)
  kEpiGeluBwd = 2, // C = acc * GELU'(aux)
};

struct GemmDesc {
  const float *A = nullptr; // op(A) is [M,K]; stored [M,K] (lda) or [K,M] when trans_a
  const float *B = nullptr; // op(B) is [K,N]; stored [K,N] (ldb) or [N,K] when trans_b
  float *C = nullptr;       // [M,N] with row stride ldc (or head layout, see remap_*)
  const float *bias = nullptr;     // [N] row vector, optional
  const float *residual = nullptr; // [M,N] added after bias, same indexing as C
  float *aux = nullptr;            // GELU pre-activation (written or read), same indexing as C
  // Bias gradient of a weight gradient: bias_grad[n] = beta*bias_grad[n] +
  // sum_k op(B)[k][n] (the column sums of dY when C = X^T.dY).
  float *bias_grad = nullptr;
  int M = 0, N = 0, K = 0;
  int lda = 0, ldb = 0, ldc = 0;
  int trans_a = 0, trans_b = 0;
  float beta = 0.0f; // C = acc + beta * C_old
  int epilogue = kEpiStore;
  // Output row m = b*remap_t + t, column n = h*remap_d + d is stored at
  // ((b*remap_h + h)*remap_t + t)*remap_d + d  (the [B,H,T,dh] head layout).
  int remap_t = 0, remap_h = 0, remap_d = 0;
  // Batched product: gridDim.z = batch; per-batch element offsets are
  // decoded from up to 4 batch dimensions (0 stride = broadcast operand).
  int batch = 1;
  int batch_ndim = 0;
  uint32_t batch_shape[4] = {1, 1, 1, 1};
  uint32_t batch_stride_a[4] = {0, 0, 0, 0};
  uint32_t batch_stride_b[4] = {0, 0, 0, 0};
  uint32_t batch_stride_c[4] = {0, 0, 0, 0};
  // Bias (and bias-gradient) elements between consecutive batch entries
  // (0: one shared bias).
  uint32_t bias_batch_stride = 0;
  // The batch entries (1-D batch) are K-partials of one product: each entry
  // multiplies its own A and B and the results are summed into C (with the
  // epilogue applied once). Needs a workspace; no bias gradient.
  int sum_batches = 0;
  // Split-K (batch == 1 only, chosen by gemm_launch when a workspace is
  // given): partial products go to `workspace` ([splits, M, N] then
  // [splits, N] bias-gradient partials) and a reduction kernel applies the
  // epilogue in a fixed order.
  float *workspace = nullptr;
  // Elements available at `workspace` (0: sized by gemm_workspace_elems for
  // this descriptor). A tail split that needs more is not used.
  size_t workspace_elems = 0;
};

// Launches the GEMM described by `d` on `stream`. Returns hipError_t.
int gemm_launch(const GemmDesc &d, void *stream);

// Number of fp32 elements of split-K workspace gemm_launch wants for `d`
// under its own tile/split choice (0 = no split).
size_t gemm_workspace_elems(const GemmDesc &d);

// Chooses the split count gemm_launch would use for `d` (1 = none).
int gemm_choose_splits(const GemmDesc &d);

// Compute units of the current device (256 when the query fails), cached
// per device.
int cu_count();

// Device address of the current GPU's copy of the allocation-free entry
// point's scratch array (TLH_NOALLOC_SCRATCH_FLOATS floats), resolved with
// hipGetSymbolAddress on the first call per device. Returns hipError_t.
int noalloc_scratch(float **out);

} // namespace tlh
