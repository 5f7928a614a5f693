// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x2f32).
//
// Replaces the Metal matmul kernels K1-K3 (include/my_metal/math.metal:13-400,
// launched from src/my_metal/runtime.cpp:375-505). Differences by design:
//  * one kernel family covers contiguous, transposed-operand (A^T.B, A.B^T)
//    and masked edge tiles, so the executor's materialised transposes can be
//    skipped by callers that know the layout;
//  * fused epilogues (bias, residual, GELU, GELU', head-layout store);
//  * split-K with a deterministic reduction for the tall-K weight gradients.
//
// Tile: BM x BN per 256-thread block (4 waves in a 2x2 grid), BK = 16,
// LDS double-buffered with a register prefetch of the next K tile.
// MFMA operand mapping (32x32x2, 64 lanes): lane l supplies A[m=l%32][k=l/32]
// and B[k=l/32][n=l%32]; accumulator v of lane l holds
// D[8*(v/4) + 4*(l/32) + v%4][l%32]. Within a K tile the two MFMA k-slots
// are assigned actual k = slot*(BK/2) + s, so a lane reads BK/2 consecutive
// k of one row of a K-contiguous LDS tile with ds_read_b128.
#include "common.h"
#include "gemm.h"

#include <algorithm>
#include <mutex>
#include <numeric>

namespace tlh {
namespace {

constexpr int kBK = 32; // largest K tile; split-K chunks are multiples of it
constexpr int kPad = 4;
// Row padding of the 16x16 kernels' K-contiguous LDS tiles (see gemm_mfma16_kernel).
constexpr int kPad16 = 8;

struct GemmParams {
  const float *A;
  const float *B;
  float *C;
  const float *bias;
  const float *residual;
  float *aux;
  float *workspace;
  float *bias_grad;
  int M, N, K;
  int lda, ldb, ldc;
  float beta;
  int epilogue;
  int remap_t, remap_h, remap_d;
  int batch_ndim;
  uint32_t batch_shape[4];
  uint32_t bsa[4], bsb[4], bsc[4];
  int splits;
  int k_chunk;
  int tiles_n;
  int xcd_remap;
  // XCD rectangles (0 = off): XCD j takes the rect_m x rect_n tile block at
  // ((j / py) * rect_m, (j % py) * rect_n), py = tiles_n / rect_n; 8 blocks
  // tile the grid exactly. Set only without a tail split.
  int rect_m, rect_n;
  // Split-major XCD order (0 = off, else the grid's z extent): work item
  // w = z * gx + x, XCD j takes items [j * G/8, (j+1) * G/8) of the G = gx *
  // gz blocks, so each XCD holds whole K splits (or batch entries) and its
  // L2 fetches their operand panels once. Set when G is a multiple of 8.
  int zmajor;
  uint32_t bias_bstride; // bias (and bias-gradient) elements between batch entries
  int batch;             // output entries (blockIdx.z = entry * splits + split)
  // K-segmented operands (summed batch entries): K index k lies in segment
  // k / seg_k, whose A and B start seg_a / seg_b elements further on.
  int seg_k;
  uint32_t seg_a, seg_b;
  // Tail split (batch 1, no split-K): tiles [0, dp_tiles) are whole-K blocks
  // (a multiple of the CU count); each remaining tile is split into
  // tail_splits K chunks of tail_k_chunk whose partial tiles go to the
  // workspace ([tail tile][split][BM*BN]) for gemm_tail_reduce. 0 = off.
  int dp_tiles, tail_tiles, tail_splits, tail_k_chunk;
  // Output rows (C, residual, aux, or the raw partial planes) take float4
  // access at multiples of 4 columns: 16-byte aligned bases and row
  // strides, and 4 | remap_d for the head layout (set by the host).
  int out_vec;
};

__device__ inline size_t out_index(const GemmParams &p, int m, int n) {
  if (p.remap_h > 0) {
    const int b = m / p.remap_t, t = m - b * p.remap_t;
    const int h = n / p.remap_d, d = n - h * p.remap_d;
    return ((size_t(b) * p.remap_h + h) * p.remap_t + t) * p.remap_d + d;
  }
  return size_t(m) * p.ldc + n;
}

// Applies the epilogue to one output element. `C` already carries the batch
// offset; bias/residual/aux are only used for batch == 1 (host-checked).
__device__ inline void epilogue_store(const GemmParams &p, const float *bias, float *C, int m,
                                      int n, float v) {
  const size_t idx = out_index(p, m, n);
  if (bias) v += bias[n];
  if (p.beta != 0.0f) v += p.beta * C[idx];
  if (p.residual) v += p.residual[idx];
  if (p.epilogue == kEpiGelu) {
    p.aux[idx] = v;
    v = gelu_fwd(v);
  } else if (p.epilogue == kEpiGeluBwd) {
    v *= gelu_grad(p.aux[idx]);
  }
  C[idx] = v;
}

// One block's output tile, K range and operand bases.
struct BlockCtx {
  bool partial; // a tail-split block: raw partial tile into the workspace
  int tm, m0, n0;
  int k_begin, k_end;
  const float *A, *B;
  float *C;
  const float *bias;
  float *bias_grad;
  int bz; // the block's z coordinate: output entry * splits + split
};

// (bx, gx, bz): the block's x coordinate, the grid's x extent and its z
// coordinate (blockIdx.x, gridDim.x, blockIdx.z of the launch).
template <int BM, int BN>
__device__ inline BlockCtx block_ctx(const GemmParams &p, int bx, int gx, int bz) {
  BlockCtx b;
  // Blocks are dispatched round-robin over the 8 XCDs (block x runs on XCD
  // x % 8), each with its own L2. Give XCD j a block of tiles that share
  // operand panels in its L2: a rectangle of the tile grid (rows share A
  // rows, columns share B columns) when the host found one that needs fewer
  // panels, else the contiguous tile range [j*G/8, (j+1)*G/8).
  if (p.zmajor > 0) {
    // the hardware puts linear block L = x + gx * z on XCD L % 8
    const int lin = bx + gx * bz, per = (gx * p.zmajor) >> 3;
    const int w = (lin & 7) * per + (lin >> 3);
    bz = w / gx;
    bx = w - bz * gx;
  }
  b.bz = bz;
  b.partial = p.tail_splits > 0 && bx >= p.dp_tiles;
  const int nblk = p.tail_splits > 0 ? p.dp_tiles : gx;
  int tile;
  if (p.rect_m > 0) {
    const int xcd = bx & 7, i = bx >> 3, py = p.tiles_n / p.rect_n;
    const int tm = (xcd / py) * p.rect_m + i / p.rect_n;
    const int tn = (xcd % py) * p.rect_n + i % p.rect_n;
    tile = tm * p.tiles_n + tn;
  } else {
    tile = (p.xcd_remap && (nblk & 7) == 0) ? (bx & 7) * (nblk >> 3) + (bx >> 3) : bx;
  }
  int tail = 0, tail_split = 0;
  if (b.partial) {
    tail = (bx - p.dp_tiles) / p.tail_splits;
    tail_split = bx - p.dp_tiles - tail * p.tail_splits;
    tile = p.dp_tiles + tail;
  }
  b.tm = tile / p.tiles_n;
  b.m0 = b.tm * BM;
  b.n0 = (tile - b.tm * p.tiles_n) * BN;
  // (p stays unmodified: writing a kernel-argument struct that is also
  // passed by reference moves it to scratch memory)
  b.A = p.A;
  b.B = p.B;
  b.C = p.C;
  b.bias = p.bias;
  b.bias_grad = p.bias_grad;
  // bz = output entry * splits + split (a split is a K range).
  const int zs = p.splits > 1 ? bz % p.splits : 0;
  const int zb = p.splits > 1 ? bz / p.splits : bz;
  b.k_begin = 0;
  b.k_end = p.K;
  if (p.batch_ndim > 0) {
    uint32_t rem = uint32_t(zb);
    size_t oa = 0, ob = 0, oc = 0;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
      const uint32_t c = rem % p.batch_shape[d];
      rem /= p.batch_shape[d];
      oa += size_t(c) * p.bsa[d];
      ob += size_t(c) * p.bsb[d];
      oc += size_t(c) * p.bsc[d];
    }
    b.A += oa;
    b.B += ob;
    b.C += oc;
    if (b.bias) b.bias += size_t(zb) * p.bias_bstride;
    if (b.bias_grad) b.bias_grad += size_t(zb) * p.bias_bstride;
  }
  if (p.splits > 1) {
    b.k_begin = zs * p.k_chunk;
    b.k_end = min(p.K, b.k_begin + p.k_chunk);
    b.C = p.workspace + (size_t(zb) * p.splits + zs) * p.M * p.N;
  }
  if (b.partial) {
    b.k_begin = tail_split * p.tail_k_chunk;
    b.k_end = min(p.K, b.k_begin + p.tail_k_chunk);
    b.C = p.workspace + (size_t(tail) * p.tail_splits + tail_split) * size_t(BM * BN);
  }
  return b;
}

// Bias gradient of the blocks of the first tile row: each thread's partial
// column sum goes through LDS (free again: every thread is past the main
// loop's last barrier), then to the output or the split-K partials.
template <int BN>
__device__ inline void bias_grad_store(const GemmParams &p, const BlockCtx &b, float *smem,
                                       float bsum, bool full) {
  constexpr int BGROUPS = 256 / BN;
  const int tid = threadIdx.x;
  smem[tid] = bsum;
  __syncthreads();
  const int n = b.n0 + tid;
  if (tid < BN && (full || n < p.N)) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < BGROUPS; ++g) t += smem[g * BN + tid];
    if (p.splits > 1) {
      p.workspace[size_t(p.batch) * p.splits * p.M * p.N + size_t(b.bz) * p.N + n] = t;
    } else {
      b.bias_grad[n] = p.beta != 0.0f ? t + p.beta * b.bias_grad[n] : t;
    }
  }
}

// Writes the accumulators of one wave (TM x TN 32x32 tiles) through the
// epilogue, or raw: into the split-K plane, or into the block's partial
// tile of a tail split (row-major BM x BN).
template <int BN, int TM, int TN, int WM, int WN, bool FULL>
__device__ inline void store_acc(const GemmParams &p, const BlockCtx &b, const f16x (&acc)[TM][TN],
                                 int wm, int wn, int r, int hk) {
  const bool raw = b.partial || p.splits > 1;
  const int rs = b.partial ? BN : p.N;
  float *rbase = b.partial ? b.C - (size_t(b.m0) * BN + b.n0) : b.C;
  // (the gathered path is kept to waves with at most two accumulator tiles:
  // with four, the unrolled epilogue no longer fits and spills)
  const bool reads = TM * TN <= 2 &&
                     (p.beta != 0.0f || p.residual != nullptr || p.epilogue == kEpiGeluBwd);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = b.n0 + wn * WN + j * 32 + r;
      if (!FULL && n >= p.N) continue;
      const int mb = b.m0 + wm * WM + i * 32 + 4 * hk;
      if (raw || !reads) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = mb + 8 * (v >> 2) + (v & 3);
          if (!FULL && m >= p.M) continue;
          if (raw) {
            rbase[size_t(m) * rs + n] = acc[i][j][v];
          } else {
            epilogue_store(p, b.bias, b.C, m, n, acc[i][j][v]);
          }
        }
      } else if constexpr (TM * TN <= 2) {
        // The epilogue reads C, the residual or the GELU pre-activation. Each
        // group of rows loads its operands before its first store:
        // interleaved, every load would wait behind the previous element's
        // store (which might alias it), one memory latency per element. Same
        // arithmetic, same order as epilogue_store. GS rows per group: all 16
        // with one accumulator tile per wave, 4 with two.
        constexpr int GS = TM * TN == 1 ? 16 : 4;
#pragma unroll
        for (int g = 0; g < 16 / GS; ++g) {
          float cold[GS], res[GS], ax[GS];
#pragma unroll
          for (int e = 0; e < GS; ++e) {
            const int v = g * GS + e, m = mb + 8 * (v >> 2) + (v & 3);
            cold[e] = res[e] = ax[e] = 0.f;
            if (!FULL && m >= p.M) continue;
            const size_t idx = out_index(p, m, n);
            if (p.beta != 0.0f) cold[e] = b.C[idx];
            if (p.residual) res[e] = p.residual[idx];
            if (p.epilogue == kEpiGeluBwd) ax[e] = p.aux[idx];
          }
#pragma unroll
          for (int e = 0; e < GS; ++e) {
            const int v = g * GS + e, m = mb + 8 * (v >> 2) + (v & 3);
            if (!FULL && m >= p.M) continue;
            const size_t idx = out_index(p, m, n);
            float x = acc[i][j][v];
            if (b.bias) x += b.bias[n];
            if (p.beta != 0.0f) x += p.beta * cold[e];
            if (p.residual) x += res[e];
            if (p.epilogue == kEpiGelu) {
              p.aux[idx] = x;
              x = gelu_fwd(x);
            } else if (p.epilogue == kEpiGeluBwd) {
              x *= gelu_grad(ax[e]);
            }
            b.C[idx] = x;
          }
        }
      }
    }
  }
}


// Global -> register fetch of one K tile of both operands (A_CHUNKS and
// B_CHUNKS float4 per thread), zero-filled outside the matrix unless FULL.
// Summed batch entries (seg_k > 0): a K tile never straddles a segment.
template <int BM, int BN, int BK, bool TA, bool TB, bool VEC, bool FULL, int NT = 256>
__device__ inline void fetch_operands(const GemmParams &p, const float *A, const float *B, int m0,
                                      int n0, int k0, int k_end, f4 (&ra)[BM * BK / (4 * NT)],
                                      f4 (&rb)[BN * BK / (4 * NT)]) {
  constexpr int A_CHUNKS = BM * BK / (4 * NT), B_CHUNKS = BN * BK / (4 * NT);
  const int tid = threadIdx.x;
  const float *As = A, *Bs = B;
  int kofs = 0; // global k minus the segment-local k
  if (p.seg_k > 0) {
    const int sg = k0 / p.seg_k;
    kofs = sg * p.seg_k;
    As += size_t(sg) * p.seg_a;
    Bs += size_t(sg) * p.seg_b;
  }
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = tid + i * NT;
    int row, col; // in stored layout
    if (!TA) { row = c / (BK / 4); col = (c % (BK / 4)) * 4; }
    else     { row = c / (BM / 4); col = (c % (BM / 4)) * 4; }
    const int grow = TA ? (k0 + row) : (m0 + row);
    const int gcol = TA ? (m0 + col) : (k0 + col);
    const int row_lim = TA ? k_end : p.M;
    const int col_lim = TA ? p.M : k_end;
    const float *src = As + size_t(TA ? grow - kofs : grow) * p.lda + (TA ? gcol : gcol - kofs);
    if constexpr (FULL) {
      ra[i] = *reinterpret_cast<const f4 *>(src);
    } else {
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (grow < row_lim) {
        if (VEC && gcol + 3 < col_lim) {
          v = *reinterpret_cast<const f4 *>(src);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (gcol + j < col_lim) v[j] = src[j];
        }
      }
      ra[i] = v;
    }
  }
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = tid + i * NT;
    int row, col;
    if (TB) { row = c / (BK / 4); col = (c % (BK / 4)) * 4; }
    else    { row = c / (BN / 4); col = (c % (BN / 4)) * 4; }
    const int grow = TB ? (n0 + row) : (k0 + row);
    const int gcol = TB ? (k0 + col) : (n0 + col);
    const int row_lim = TB ? p.N : k_end;
    const int col_lim = TB ? k_end : p.N;
    const float *src = Bs + size_t(TB ? grow : grow - kofs) * p.ldb + (TB ? gcol - kofs : gcol);
    if constexpr (FULL) {
      rb[i] = *reinterpret_cast<const f4 *>(src);
    } else {
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (grow < row_lim) {
        if (VEC && gcol + 3 < col_lim) {
          v = *reinterpret_cast<const f4 *>(src);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (gcol + j < col_lim) v[j] = src[j];
        }
      }
      rb[i] = v;
    }
  }
}

// Register -> LDS store of the fetched K tile: K-contiguous tiles as [rows]
// [BK + pad], row-contiguous tiles as [BK][rows + pad].
template <int BM, int BN, int BK, int A_LD, int B_LD, bool TA, bool TB, int NT = 256>
__device__ inline void stage_operands(float *as, float *bs, const f4 (&ra)[BM * BK / (4 * NT)],
                                      const f4 (&rb)[BN * BK / (4 * NT)]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < BM * BK / (4 * NT); ++i) {
    const int c = tid + i * NT;
    int row, col;
    if (!TA) { row = c / (BK / 4); col = (c % (BK / 4)) * 4; }
    else     { row = c / (BM / 4); col = (c % (BM / 4)) * 4; }
    *reinterpret_cast<f4 *>(as + row * A_LD + col) = ra[i];
  }
#pragma unroll
  for (int i = 0; i < BN * BK / (4 * NT); ++i) {
    const int c = tid + i * NT;
    int row, col;
    if (TB) { row = c / (BK / 4); col = (c % (BK / 4)) * 4; }
    else    { row = c / (BN / 4); col = (c % (BN / 4)) * 4; }
    *reinterpret_cast<f4 *>(bs + row * B_LD + col) = rb[i];
  }
}

// FULL: M, N are multiples of the tile, the K range of every block is a
// multiple of BK and the operands are float4-aligned: no bounds checks.
// LDS floats of gemm_tile32: two stages of both operand tiles.
template <int BM, int BN, int BK, bool TA, bool TB>
constexpr int tile32_smem() {
  constexpr int A_LD = TA ? (BM + kPad) : (BK + kPad);
  constexpr int B_LD = TB ? (BK + kPad) : (BN + kPad);
  return 2 * ((TA ? BK * A_LD : BM * A_LD) + (TB ? BN * B_LD : BK * B_LD));
}

template <int BM, int BN, int WM, int WN, int BK, bool TA, bool TB, bool VEC, bool FULL>
__device__ inline void gemm_tile32(const GemmParams &p, float *smem, int bx, int gx, int bz) {
  static_assert(BK % 8 == 0 && BK <= kBK, "K tile must be a multiple of 8 and divide the split chunk");
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  constexpr int WAVES_N = BN / WN;
  static_assert((BM / WM) * (BN / WN) == 4, "4 waves per block");
  // LDS tile geometry (floats). K-contiguous tiles: [rows][BK+pad];
  // row-contiguous tiles: [BK][rows+pad].
  constexpr int A_LD = TA ? (BM + kPad) : (BK + kPad);
  constexpr int B_LD = TB ? (BK + kPad) : (BN + kPad);
  constexpr int A_TILE = TA ? BK * A_LD : BM * A_LD;
  constexpr int B_TILE = TB ? BN * B_LD : BK * B_LD;
  constexpr int A_CHUNKS = BM * BK / 4 / 256;
  constexpr int B_CHUNKS = BN * BK / 4 / 256;
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for 256 threads");
  static_assert(2 * (A_TILE + B_TILE) == tile32_smem<BM, BN, BK, TA, TB>(), "LDS geometry");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int r = lane & 31;
  const int hk = lane >> 5;

  const BlockCtx ctx = block_ctx<BM, BN>(p, bx, gx, bz);
  const int tm = ctx.tm, m0 = ctx.m0, n0 = ctx.n0;
  const int k_begin = ctx.k_begin, k_end = ctx.k_end;
  const float *A = ctx.A;
  const float *B = ctx.B;

  // ---- global -> register prefetch ----------------------------------------
  f4 ra[A_CHUNKS], rb[B_CHUNKS];
  auto load_tile = [&](int k0) {
    fetch_operands<BM, BN, BK, TA, TB, VEC, FULL>(p, A, B, m0, n0, k0, k_end, ra, rb);
  };
  auto store_tile = [&](int buf) {
    float *as = smem + buf * (A_TILE + B_TILE);
    stage_operands<BM, BN, BK, A_LD, B_LD, TA, TB>(as, as + A_TILE, ra, rb);
  };

  f16x acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int a_row0 = wm * WM + r; // + i*32
  const int b_col0 = wn * WN + r; // + j*32

  // All of a lane's fragments of one K tile are read from LDS first, then
  // the MFMAs run back to back: the LDS latency is paid once per tile.
  auto compute_tile = [&](int buf) {
    const float *as = smem + buf * (A_TILE + B_TILE);
    const float *bs = as + A_TILE;
    constexpr int Q = BK / 8; // float4 groups per lane per K tile
    f4 af[TM][Q], bf[TN][Q];
#pragma unroll
    for (int s4 = 0; s4 < Q; ++s4) {
      const int kb = hk * (BK / 2) + s4 * 4; // first of 4 consecutive k
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = a_row0 + i * 32;
        if (!TA) {
          af[i][s4] = *reinterpret_cast<const f4 *>(as + m * A_LD + kb);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) af[i][s4][q] = as[(kb + q) * A_LD + m];
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = b_col0 + j * 32;
        if (TB) {
          bf[j][s4] = *reinterpret_cast<const f4 *>(bs + n * B_LD + kb);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) bf[j][s4][q] = bs[(kb + q) * B_LD + n];
        }
      }
    }
#pragma unroll
    for (int s4 = 0; s4 < Q; ++s4)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s4][q], bf[j][s4][q],
                                                             acc[i][j], 0, 0, 0);
    // Scheduling hint: interleave this tile's LDS reads with the MFMAs so
    // that each fragment is read one MFMA group ahead of its use (measured
    // on MI355X: transposed-B and 128x128 products 3-7% faster; products
    // with a transposed A -- the weight gradients -- are not, so they keep
    // the default schedule).
    if constexpr (!TA) __builtin_amdgcn_iglp_opt(1);
  };

  // Bias gradient: the blocks of the first tile row also sum the op(B)
  // tiles they stage (threads = BN columns x 256/BN k groups).
  const bool do_bias = p.bias_grad != nullptr && tm == 0;
  constexpr int BGROUPS = 256 / BN;
  const int bcol = tid % BN, bgrp = tid / BN;
  float bsum = 0.f;

  const int nk = (k_end > k_begin) ? (k_end - k_begin + BK - 1) / BK : 0;
  if (nk > 0) {
    load_tile(k_begin);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tile(k_begin + (kt + 1) * BK);
      compute_tile(cur);
      if (do_bias) {
        const float *bs = smem + cur * (A_TILE + B_TILE) + A_TILE;
#pragma unroll
        for (int kk = bgrp; kk < BK; kk += BGROUPS)
          bsum += TB ? bs[bcol * B_LD + kk] : bs[kk * B_LD + bcol];
      }
      if (kt + 1 < nk) store_tile(cur ^ 1);
      __syncthreads();
    }
  }
  if (do_bias) bias_grad_store<BN>(p, ctx, smem, bsum, FULL);
  store_acc<BN, TM, TN, WM, WN, FULL>(p, ctx, acc, wm, wn, r, hk);
}

template <int BM, int BN, int WM, int WN, int BK, bool TA, bool TB, bool VEC, bool FULL>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) float smem[tile32_smem<BM, BN, BK, TA, TB>()];
  gemm_tile32<BM, BN, WM, WN, BK, TA, TB, VEC, FULL>(p, smem, int(blockIdx.x), int(gridDim.x),
                                                     int(blockIdx.z));
}

// ---- 16x16x4 MFMA tiles --------------------------------------------------------
// v_mfma_f32_16x16x4f32 (64 lanes): lane l supplies A[m = l%16][k = l/16] and
// B[k = l/16][n = l%16]; accumulator v of lane l holds D[4*(l/16) + v][l%16].
// Its 16-row granularity allows tiles of 96 = 3 x 32 rows and columns: a
// [6144, 384] output is exactly 256 tiles of 96x96 (one per CU) where 64x64
// tiles give 576 (2.25 per CU, and the CUs holding a third tile set the
// time), and [6144, 1536] is 1024 (4 per CU) at 1.5x the operand reuse of a
// 64x64 tile.

// Epilogue of a block tile staged in LDS (ct: BM x BN, row stride BN + 4):
// all 256 threads walk the tile row-major, float4 by float4, so each row of
// the output is written by consecutive lanes (the 16x16 accumulator layout
// would store 64-byte pieces of 4 rows). Raw into the split-K plane or a
// tail split's partial tile, else through the epilogue with the arithmetic
// and order of epilogue_store. With float4 access every group of 3 float4s
// loads its epilogue operands (C, residual, GELU pre-activation) before its
// stores, which might alias them.
template <int BM, int BN, bool FULL, int NT = 256, int PARTS = 1>
__device__ inline void tile_epilogue(const GemmParams &p, const BlockCtx &b, const float *ct) {
  constexpr int C_LD = BN + 4, ROW4 = BN / 4, GROUPS = BM * ROW4, PER = (GROUPS + NT - 1) / NT;
  constexpr int PART = BM * C_LD; // floats between the partial tiles (PARTS = 2)
  static_assert(PARTS == 1 || PARTS == 2, "one tile or two partial tiles");
  const int tid = threadIdx.x;
  const bool raw = b.partial || p.splits > 1;
  const int rs = b.partial ? BN : p.N;
  float *rbase = b.partial ? b.C - (size_t(b.m0) * BN + b.n0) : b.C;
  if (FULL && p.out_vec) {
    constexpr int U = 3;
#pragma unroll
    for (int it0 = 0; it0 < PER; it0 += U) {
      f4 v[U], cold[U], res[U], ax[U];
      size_t oi[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = tid + (it0 + u) * NT;
        cold[u] = res[u] = ax[u] = f4{0.f, 0.f, 0.f, 0.f};
        oi[u] = 0;
        if (it0 + u >= PER || e >= GROUPS) continue;
        const int r = e / ROW4, c = (e - r * ROW4) * 4;
        v[u] = *reinterpret_cast<const f4 *>(ct + r * C_LD + c);
        if constexpr (PARTS == 2) v[u] += *reinterpret_cast<const f4 *>(ct + PART + r * C_LD + c);
        const int m = b.m0 + r, n = b.n0 + c;
        if (raw) {
          oi[u] = size_t(m) * rs + n;
        } else {
          oi[u] = out_index(p, m, n);
          if (p.beta != 0.0f) cold[u] = *reinterpret_cast<const f4 *>(b.C + oi[u]);
          if (p.residual) res[u] = *reinterpret_cast<const f4 *>(p.residual + oi[u]);
          if (p.epilogue == kEpiGeluBwd) ax[u] = *reinterpret_cast<const f4 *>(p.aux + oi[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = tid + (it0 + u) * NT;
        if (it0 + u >= PER || e >= GROUPS) continue;
        if (raw) {
          *reinterpret_cast<f4 *>(rbase + oi[u]) = v[u];
          continue;
        }
        const int r = e / ROW4, n = b.n0 + (e - r * ROW4) * 4;
        f4 x = v[u];
        if (b.bias) x += f4{b.bias[n], b.bias[n + 1], b.bias[n + 2], b.bias[n + 3]};
        if (p.beta != 0.0f) x += p.beta * cold[u];
        if (p.residual) x += res[u];
        if (p.epilogue == kEpiGelu) {
          *reinterpret_cast<f4 *>(p.aux + oi[u]) = x;
#pragma unroll
          for (int q = 0; q < 4; ++q) x[q] = gelu_fwd(x[q]);
        } else if (p.epilogue == kEpiGeluBwd) {
#pragma unroll
          for (int q = 0; q < 4; ++q) x[q] *= gelu_grad(ax[u][q]);
        }
        *reinterpret_cast<f4 *>(b.C + oi[u]) = x;
      }
    }
  } else {
    for (int e = tid; e < BM * BN; e += NT) {
      const int r = e / BN, c = e - r * BN;
      const int m = b.m0 + r, n = b.n0 + c;
      if (!FULL && (m >= p.M || n >= p.N)) continue;
      float v = ct[r * C_LD + c];
      if constexpr (PARTS == 2) v += ct[PART + r * C_LD + c];
      if (raw) rbase[size_t(m) * rs + n] = v;
      else epilogue_store(p, b.bias, b.C, m, n, v);
    }
  }
}

// 4 waves in a 2x2 grid, each (BM/2) x (BN/2) as TM x TN subtiles of 16x16.
// Within a K tile, lane group g = l/16 reads k = 4*(g + 4*s) + q for MFMA
// step 4*s + q with one ds_read_b128 per s from a K-contiguous LDS row. With
// a row stride of BK + 8 floats (an even, not a multiple of 4, number of
// 16-byte groups) the 32 lanes of each read pass -- rows 0..15 of groups g
// and g+1, one 16-byte group apart -- hit distinct banks of gfx950's LDS
// (measured: no bank conflicts; with a stride of BK + 4, or consecutive k
// blocks per lane group, 13% of the read cycles conflict).
// Row-contiguous operand tiles (A transposed, B not: [BK][rows + pad]) are
// read with the subtiles interleaved when a wave has 2 or 4 of them in that
// dimension: row slot r16 of subtile i is row TM*r16 + i of the wave's WM
// rows (columns alike), so a lane's TM values of one k sit side by side in
// LDS and come in one ds_read_b64 / b128 instead of TM ds_read_b32; the
// accumulators are put back in order when they are staged for the
// epilogue. Same staging, K loop and epilogues as gemm_mfma_kernel,
// including the bias gradient of the first tile row.
// LDS floats of gemm_tile16: two stages of both operand tiles.
template <int BM, int BN, int BK, bool TA, bool TB>
constexpr int tile16_smem() {
  constexpr int A_LD = TA ? (BM + kPad) : (BK + kPad16);
  constexpr int B_LD = TB ? (BK + kPad16) : (BN + kPad);
  return 2 * ((TA ? BK * A_LD : BM * A_LD) + (TB ? BN * B_LD : BK * B_LD));
}

template <int BM, int BN, int BK, bool TA, bool TB, bool VEC, bool FULL>
__device__ inline void gemm_tile16(const GemmParams &p, float *smem, int bx, int gx, int bz) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  static_assert(WM % 16 == 0 && WN % 16 == 0 && BK % 16 == 0 && BK <= kBK, "tile geometry");
  constexpr int A_LD = TA ? (BM + kPad) : (BK + kPad16);
  constexpr int B_LD = TB ? (BK + kPad16) : (BN + kPad);
  constexpr int A_TILE = TA ? BK * A_LD : BM * A_LD;
  constexpr int B_TILE = TB ? BN * B_LD : BK * B_LD;
  constexpr int A_CHUNKS = BM * BK / 1024, B_CHUNKS = BN * BK / 1024;
  static_assert(A_CHUNKS * 1024 == BM * BK && B_CHUNKS * 1024 == BN * BK,
                "every thread stages whole float4s of both operands");
  static_assert(2 * (A_TILE + B_TILE) == tile16_smem<BM, BN, BK, TA, TB>(), "LDS geometry");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;

  const BlockCtx ctx = block_ctx<BM, BN>(p, bx, gx, bz);
  const int m0 = ctx.m0, n0 = ctx.n0;
  const int k_begin = ctx.k_begin, k_end = ctx.k_end;
  const float *A = ctx.A;
  const float *B = ctx.B;

  f4 ra[A_CHUNKS], rb[B_CHUNKS];
  auto load_tile = [&](int k0) {
    fetch_operands<BM, BN, BK, TA, TB, VEC, FULL>(p, A, B, m0, n0, k0, k_end, ra, rb);
  };
  auto store_tile = [&](int buf) {
    float *as = smem + buf * (A_TILE + B_TILE);
    stage_operands<BM, BN, BK, A_LD, B_LD, TA, TB>(as, as + A_TILE, ra, rb);
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  // interleaved subtiles of the row-contiguous operand tiles
  constexpr bool IA = TA && (TM == 2 || TM == 4);
  constexpr bool IB = !TB && (TN == 2 || TN == 4);
  const int a_row0 = wm * WM + (IA ? TM * r16 : r16); // + i (interleaved) or i*16
  const int b_col0 = wn * WN + (IB ? TN * r16 : r16); // + j or j*16

  auto compute_tile = [&](int buf) {
    const float *as = smem + buf * (A_TILE + B_TILE);
    const float *bs = as + A_TILE;
    constexpr int Q = BK / 16; // float4 groups per lane per K tile
    f4 af[TM][Q], bf[TN][Q];
#pragma unroll
    for (int s4 = 0; s4 < Q; ++s4) {
      const int kb = 4 * (g + 4 * s4); // first of 4 consecutive k
      if constexpr (IA) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float *src = as + (kb + q) * A_LD + a_row0;
          if constexpr (TM == 4) {
            const f4 v = *reinterpret_cast<const f4 *>(src);
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i][s4][q] = v[i];
          } else {
            const float2 v = *reinterpret_cast<const float2 *>(src);
            af[0][s4][q] = v.x;
            af[1][s4][q] = v.y;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = a_row0 + i * 16;
          if (!TA) {
            af[i][s4] = *reinterpret_cast<const f4 *>(as + m * A_LD + kb);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) af[i][s4][q] = as[(kb + q) * A_LD + m];
          }
        }
      }
      if constexpr (IB) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float *src = bs + (kb + q) * B_LD + b_col0;
          if constexpr (TN == 4) {
            const f4 v = *reinterpret_cast<const f4 *>(src);
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j][s4][q] = v[j];
          } else {
            const float2 v = *reinterpret_cast<const float2 *>(src);
            bf[0][s4][q] = v.x;
            bf[1][s4][q] = v.y;
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = b_col0 + j * 16;
          if (TB) {
            bf[j][s4] = *reinterpret_cast<const f4 *>(bs + n * B_LD + kb);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) bf[j][s4][q] = bs[(kb + q) * B_LD + n];
          }
        }
      }
    }
#pragma unroll
    for (int s4 = 0; s4 < Q; ++s4)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s4][q], bf[j][s4][q],
                                                             acc[i][j], 0, 0, 0);
    if constexpr (!TA) __builtin_amdgcn_iglp_opt(1);
  };

  // Bias gradient: the blocks of the first tile row also sum the op(B)
  // tiles they stage (threads = BN columns x 256/BN k groups).
  // (tiles of 64 and 128 columns; the planner keeps bias gradients off 96)
  constexpr bool BIAS = 256 % BN == 0;
  const bool do_bias = BIAS && p.bias_grad != nullptr && ctx.tm == 0;
  constexpr int BGROUPS = 256 / BN;
  const int bcol = tid % BN, bgrp = tid / BN;
  float bsum = 0.f;

  const int nk = (k_end > k_begin) ? (k_end - k_begin + BK - 1) / BK : 0;
  if (nk > 0) {
    load_tile(k_begin);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tile(k_begin + (kt + 1) * BK);
      compute_tile(cur);
      if constexpr (BIAS) {
        if (do_bias) {
          const float *bs = smem + cur * (A_TILE + B_TILE) + A_TILE;
#pragma unroll
          for (int kk = bgrp; kk < BK; kk += BGROUPS)
            bsum += TB ? bs[bcol * B_LD + kk] : bs[kk * B_LD + bcol];
        }
      }
      if (kt + 1 < nk) store_tile(cur ^ 1);
      __syncthreads();
    }
  }
  if constexpr (BIAS) {
    if (do_bias) {
      bias_grad_store<BN>(p, ctx, smem, bsum, FULL);
      __syncthreads(); // smem is the output tile next
    }
  }
  // Accumulators -> LDS (free again: the K loop ended with a barrier), then
  // the row-major epilogue. Lane l holds row slots 4*(l/16) + v, column slot
  // l%16 of each 16x16 subtile (interleaved subtiles: slot s of subtile i is
  // row TM*s + i).
  constexpr int C_LD = BN + 4;
  static_assert(BM * C_LD <= 2 * (A_TILE + B_TILE), "output tile fits the operand buffers");
  float *ct = smem;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = wm * WM + (IA ? TM * (4 * g + v) + i : i * 16 + 4 * g + v);
        const int col = wn * WN + (IB ? TN * r16 + j : j * 16 + r16);
        ct[row * C_LD + col] = acc[i][j][v];
      }
  __syncthreads();
  tile_epilogue<BM, BN, FULL>(p, ctx, ct);
}

template <int BM, int BN, int BK, bool TA, bool TB, bool VEC, bool FULL>
__global__ __launch_bounds__(256) void gemm_mfma16_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) float smem[tile16_smem<BM, BN, BK, TA, TB>()];
  gemm_tile16<BM, BN, BK, TA, TB, VEC, FULL>(p, smem, int(blockIdx.x), int(gridDim.x),
                                             int(blockIdx.z));
}

// 8 waves, 2 per SIMD, in two groups of 4. Each stage holds a K tile of 64
// of both operands (staged by all 512 threads); group h multiplies k in
// [32h, 32h + 32) of it into its own accumulators, as gemm_mfma16_kernel's
// 2x2 waves do. A stage carries twice the MFMA work per barrier of the
// 4-wave kernel, and a wave's LDS and barrier stalls overlap the other
// group's MFMAs on its SIMD. The epilogue adds the two partial tiles (group
// 0 + group 1). K tiles of 64: summed batch entries need 64 | seg_k, and
// there is no split-K, tail split or bias gradient.
template <int BM, int BN, bool TA, bool TB, bool VEC, bool FULL>
__global__ __launch_bounds__(512) void gemm_mfma16x8_kernel(GemmParams p) {
  constexpr int BK = 64, KH = 32, NT = 512;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "tile geometry");
  constexpr int A_LD = TA ? (BM + kPad) : (BK + kPad16);
  constexpr int B_LD = TB ? (BK + kPad16) : (BN + kPad);
  constexpr int A_TILE = TA ? BK * A_LD : BM * A_LD;
  constexpr int B_TILE = TB ? BN * B_LD : BK * B_LD;
  constexpr int A_CHUNKS = BM * BK / (4 * NT), B_CHUNKS = BN * BK / (4 * NT);
  static_assert(A_CHUNKS * 4 * NT == BM * BK && B_CHUNKS * 4 * NT == BN * BK,
                "every thread stages whole float4s of both operands");
  constexpr int C_LD = BN + 4;
  static_assert(2 * BM * C_LD <= 2 * (A_TILE + B_TILE), "both partial tiles fit the operand buffers");

  __shared__ __attribute__((aligned(16))) float smem[2 * (A_TILE + B_TILE)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave >> 2, wq = wave & 3;
  const int wm = wq >> 1, wn = wq & 1;
  const int r16 = lane & 15, g = lane >> 4;

  const BlockCtx ctx = block_ctx<BM, BN>(p, int(blockIdx.x), int(gridDim.x), int(blockIdx.z));
  const int m0 = ctx.m0, n0 = ctx.n0;
  const int k_begin = ctx.k_begin, k_end = ctx.k_end;
  const float *A = ctx.A;
  const float *B = ctx.B;

  f4 ra[A_CHUNKS], rb[B_CHUNKS];
  auto load_tile = [&](int k0) {
    fetch_operands<BM, BN, BK, TA, TB, VEC, FULL, NT>(p, A, B, m0, n0, k0, k_end, ra, rb);
  };
  auto store_tile = [&](int buf) {
    float *as = smem + buf * (A_TILE + B_TILE);
    stage_operands<BM, BN, BK, A_LD, B_LD, TA, TB, NT>(as, as + A_TILE, ra, rb);
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int a_row0 = wm * WM + r16; // + i*16
  const int b_col0 = wn * WN + r16; // + j*16
  const int kg = grp * KH;          // the group's half of the stage

  auto compute_tile = [&](int buf) {
    const float *as = smem + buf * (A_TILE + B_TILE);
    const float *bs = as + A_TILE;
    constexpr int Q = KH / 16; // float4 groups per lane per half stage
    f4 af[TM][Q], bf[TN][Q];
#pragma unroll
    for (int s4 = 0; s4 < Q; ++s4) {
      const int kb = kg + 4 * (g + 4 * s4); // first of 4 consecutive k
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = a_row0 + i * 16;
        if (!TA) {
          af[i][s4] = *reinterpret_cast<const f4 *>(as + m * A_LD + kb);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) af[i][s4][q] = as[(kb + q) * A_LD + m];
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = b_col0 + j * 16;
        if (TB) {
          bf[j][s4] = *reinterpret_cast<const f4 *>(bs + n * B_LD + kb);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) bf[j][s4][q] = bs[(kb + q) * B_LD + n];
        }
      }
    }
#pragma unroll
    for (int s4 = 0; s4 < Q; ++s4)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s4][q], bf[j][s4][q],
                                                             acc[i][j], 0, 0, 0);
    if constexpr (!TA) __builtin_amdgcn_iglp_opt(1);
  };

  const int nk = (k_end > k_begin) ? (k_end - k_begin + BK - 1) / BK : 0;
  if (nk > 0) {
    load_tile(k_begin);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tile(k_begin + (kt + 1) * BK);
      compute_tile(cur);
      if (kt + 1 < nk) store_tile(cur ^ 1);
      __syncthreads();
    }
  }
  // Each group's partial tile -> LDS (group h at h * BM * C_LD), then the
  // row-major epilogue over their sum.
  float *ct = smem + grp * (BM * C_LD);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        ct[(wm * WM + i * 16 + 4 * g + v) * C_LD + wn * WN + j * 16 + r16] = acc[i][j][v];
  __syncthreads();
  tile_epilogue<BM, BN, FULL, NT, 2>(p, ctx, smem);
}


// ---- one-row products (M = 1): GEMV ------------------------------------------
// y = x . B with x [1, K] and B [K, N] row-major: memory-bound on B, and a
// 64-row MFMA tile would compute 63 rows of padding. Pass 1: block (256
// output columns x, K chunk y, entry z) -- the 64 lanes across the columns
// in float4, the 4 waves over the chunk's rows, 4 loads in flight per lane --
// writes its column sums to partials[entry][chunk][N]. Pass 2 adds the
// chunks in a fixed order and applies the epilogue (deterministic).
__global__ __launch_bounds__(256) void gemv_partial_kernel(GemmParams p, int chunk_k,
                                                           int chunks) {
  __shared__ f4 part[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c4 = int(blockIdx.x) * 64 + lane; // float4 column
  const int entry = int(blockIdx.z);
  const float *A = p.A + (p.batch_ndim > 0 ? size_t(entry) * p.bsa[0] : 0);
  const f4 *B4 = reinterpret_cast<const f4 *>(p.B + (p.batch_ndim > 0 ? size_t(entry) * p.bsb[0] : 0));
  const size_t ldb4 = size_t(p.ldb) / 4;
  const int k0 = int(blockIdx.y) * chunk_k;
  const int k1 = min(p.K, k0 + chunk_k);
  f4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
  if (c4 * 4 < p.N) {
    int k = k0 + w;
    for (; k + 12 < k1; k += 16) {
      a0 += A[k] * B4[size_t(k) * ldb4 + c4];
      a1 += A[k + 4] * B4[size_t(k + 4) * ldb4 + c4];
      a2 += A[k + 8] * B4[size_t(k + 8) * ldb4 + c4];
      a3 += A[k + 12] * B4[size_t(k + 12) * ldb4 + c4];
    }
    for (; k < k1; k += 4) a0 += A[k] * B4[size_t(k) * ldb4 + c4];
  }
  part[w][lane] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (w == 0 && c4 * 4 < p.N) {
    const f4 t = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    reinterpret_cast<f4 *>(p.workspace)[(size_t(entry) * chunks + blockIdx.y) * (p.N / 4) + c4] = t;
  }
}

// Pass 2: block (64 columns x, entry y); wave w adds chunks w, w + 4, ...
// (8 loads in flight, coalesced across the lanes' columns); the 4 wave sums
// are added in wave order.
__global__ __launch_bounds__(256) void gemv_reduce_kernel(GemmParams p, int chunks) {
  __shared__ float wsum[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int n = int(blockIdx.x) * 64 + lane, entry = int(blockIdx.y);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (n < p.N) {
    const float *part = p.workspace + size_t(entry) * chunks * p.N + n;
    for (int c0 = w; c0 < chunks; c0 += 32) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c0 + 4 * j < chunks) acc[j] += part[size_t(c0 + 4 * j) * p.N];
    }
  }
  float v = acc[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) v += acc[j];
  wsum[w][lane] = v;
  __syncthreads();
  if (w == 0 && n < p.N) {
    const float t = ((wsum[0][lane] + wsum[1][lane]) + wsum[2][lane]) + wsum[3][lane];
    float *C = p.C + (p.batch_ndim > 0 ? size_t(entry) * p.bsc[0] : 0);
    const float *bias = p.bias ? p.bias + size_t(entry) * p.bias_bstride : nullptr;
    epilogue_store(p, bias, C, 0, n, t);
  }
}

// Sums the split-K partials of every output entry in split order --
// deterministic -- and applies the epilogue.
// VEC4: the plane is read as float4 (N % 4 == 0, so the 4 elements of a
// float4 share a row) with the split loop unrolled for loads in flight.
template <bool VEC4>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(GemmParams p) {
  const size_t plane = size_t(p.M) * p.N;
  const size_t step = size_t(gridDim.x) * blockDim.x;
  const size_t tid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int entries = p.batch;
  for (int b = 0; b < entries; ++b) {
    float *C = p.C;
    const float *bias = p.bias;
    if (p.batch_ndim > 0) {
      C += size_t(b) * p.bsc[0];
      if (bias) bias += size_t(b) * p.bias_bstride;
    }
    const float *ws = p.workspace + size_t(b) * p.splits * plane;
    if constexpr (VEC4) {
      const f4 *w = reinterpret_cast<const f4 *>(ws);
      const size_t plane4 = plane / 4;
      for (size_t i = tid; i < plane4; i += step) {
        f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
        int z = 0;
        for (; z + 1 < p.splits; z += 2) {
          const f4 a = w[size_t(z) * plane4 + i], c = w[size_t(z + 1) * plane4 + i];
          s0 += a;
          s1 += c;
        }
        if (z < p.splits) s0 += w[size_t(z) * plane4 + i];
        const f4 sum = s0 + s1;
        const int m = int((i * 4) / p.N);
        const int n = int(i * 4 - size_t(m) * p.N);
#pragma unroll
        for (int e = 0; e < 4; ++e) epilogue_store(p, bias, C, m, n + e, sum[e]);
      }
    } else {
      for (size_t i = tid; i < plane; i += step) {
        float s = 0.f;
        for (int z = 0; z < p.splits; ++z) s += ws[z * plane + i];
        const int m = int(i / p.N);
        const int n = int(i - size_t(m) * p.N);
        epilogue_store(p, bias, C, m, n, s);
      }
    }
    if (p.bias_grad) {
      float *bg = p.bias_grad + (p.batch_ndim > 0 ? size_t(b) * p.bias_bstride : 0);
      const float *wb = p.workspace + size_t(entries) * p.splits * plane + size_t(b) * p.splits * p.N;
      for (size_t n = tid; n < size_t(p.N); n += step) {
        float s = 0.f;
        for (int z = 0; z < p.splits; ++z) s += wb[z * size_t(p.N) + n];
        bg[n] = p.beta != 0.0f ? s + p.beta * bg[n] : s;
      }
    }
  }
}

// The float4 form of gemm_splitk_reduce<true> (N % 4 == 0, 16-byte aligned
// planes, at most kMaxSplits splits): grid (float4 groups of one plane / 256,
// entries); a thread issues the loads of all of its group's partials before
// the adds, which keep gemm_splitk_reduce's order (even splits, odd splits,
// then the two sums), so both kernels give the same bits. Thread i < N of
// each entry also sums bias-gradient column i's partials.
constexpr int kMaxSplits = 16;
__global__ __launch_bounds__(256) void gemm_splitk_reduce4(GemmParams p) {
  const size_t plane = size_t(p.M) * p.N;
  const size_t plane4 = plane / 4;
  const int b = blockIdx.y;
  const int splits = p.splits;
  float *C = p.C;
  const float *bias = p.bias;
  if (p.batch_ndim > 0) {
    C += size_t(b) * p.bsc[0];
    if (bias) bias += size_t(b) * p.bias_bstride;
  }
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < plane4) {
    const f4 *w = reinterpret_cast<const f4 *>(p.workspace + size_t(b) * splits * plane) + i;
    f4 v[kMaxSplits];
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z)
      if (z < splits) v[z] = w[size_t(z) * plane4];
    f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int z = 0; z + 1 < kMaxSplits; z += 2) {
      if (z + 1 < splits) {
        s0 += v[z];
        s1 += v[z + 1];
      } else if (z < splits) {
        s0 += v[z];
      }
    }
    const f4 sum = s0 + s1;
    const int m = int((i * 4) / p.N);
    const int n = int(i * 4 - size_t(m) * p.N);
#pragma unroll
    for (int e = 0; e < 4; ++e) epilogue_store(p, bias, C, m, n + e, sum[e]);
  }
  if (p.bias_grad && i < size_t(p.N)) {
    float *bg = p.bias_grad + (p.batch_ndim > 0 ? size_t(b) * p.bias_bstride : 0);
    const float *wb = p.workspace + size_t(p.batch) * splits * plane + size_t(b) * splits * p.N + i;
    float v[kMaxSplits];
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z)
      if (z < splits) v[z] = wb[z * size_t(p.N)];
    float s = 0.f;
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z)
      if (z < splits) s += v[z];
    bg[i] = p.beta != 0.0f ? s + p.beta * bg[i] : s;
  }
}

// Sums the tail tiles' K-chunk partials in chunk order -- deterministic --
// and applies the epilogue. Float4 groups of a BM x BN tile (BN % 4 == 0).
template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_tail_reduce(GemmParams p) {
  constexpr int TILE = BM * BN;
  const int tails = p.tail_tiles;
  const size_t groups = size_t(tails) * (TILE / 4);
  const size_t step = size_t(gridDim.x) * blockDim.x;
  for (size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x; g < groups; g += step) {
    const int t = int(g / (TILE / 4));
    const int e = int(g - size_t(t) * (TILE / 4)) * 4;
    const f4 *w = reinterpret_cast<const f4 *>(p.workspace + size_t(t) * p.tail_splits * TILE + e);
    // every chunk's load is issued before the adds (at most 16 chunks)
    f4 v[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s)
      if (s < p.tail_splits) v[s] = w[size_t(s) * (TILE / 4)];
    f4 sum = v[0];
#pragma unroll
    for (int s = 1; s < kMaxSplits; ++s)
      if (s < p.tail_splits) sum += v[s];
    const int tile = p.dp_tiles + t;
    const int tm = tile / p.tiles_n;
    const int m = tm * BM + e / BN;
    const int n = (tile - tm * p.tiles_n) * BN + e % BN;
#pragma unroll
    for (int q = 0; q < 4; ++q) epilogue_store(p, p.bias, p.C, m, n + q, sum[q]);
  }
}

struct Plan {
  int bm, bn, splits, bk = 16;
  bool m16 = false; // the 16x16x4 MFMA kernel (gemm_tile16) at bm x bn
};

template <int BM, int BN, int WM, int WN, int BK>
void launch_cfg(const GemmParams &p, bool ta, bool tb, bool vec, bool full, dim3 grid,
                hipStream_t s) {
#define TLH_GEMM_CASE(TA_, TB_, V_, F_)                                          \
  if (ta == TA_ && tb == TB_ && vec == V_ && full == F_) {                       \
    gemm_mfma_kernel<BM, BN, WM, WN, BK, TA_, TB_, V_, F_><<<grid, 256, 0, s>>>(p); \
    return;                                                                      \
  }
  TLH_GEMM_CASE(false, false, true, true)
  TLH_GEMM_CASE(false, true, true, true)
  TLH_GEMM_CASE(true, false, true, true)
  TLH_GEMM_CASE(true, true, true, true)
  TLH_GEMM_CASE(false, false, true, false)
  TLH_GEMM_CASE(false, true, true, false)
  TLH_GEMM_CASE(true, false, true, false)
  TLH_GEMM_CASE(true, true, true, false)
  TLH_GEMM_CASE(false, false, false, false)
  TLH_GEMM_CASE(false, true, false, false)
  TLH_GEMM_CASE(true, false, false, false)
  TLH_GEMM_CASE(true, true, false, false)
#undef TLH_GEMM_CASE
}

template <int BM, int BN>
void launch16x8(const GemmParams &p, bool ta, bool tb, bool vec, bool full, dim3 grid,
                hipStream_t s) {
#define TLH_GEMM_CASE(TA_, TB_, V_, F_)                                             \
  if (ta == TA_ && tb == TB_ && vec == V_ && full == F_) {                          \
    gemm_mfma16x8_kernel<BM, BN, TA_, TB_, V_, F_><<<grid, 512, 0, s>>>(p);         \
    return;                                                                         \
  }
  TLH_GEMM_CASE(false, false, true, true)
  TLH_GEMM_CASE(false, true, true, true)
  TLH_GEMM_CASE(true, false, true, true)
  TLH_GEMM_CASE(true, true, true, true)
  TLH_GEMM_CASE(false, false, true, false)
  TLH_GEMM_CASE(false, true, true, false)
  TLH_GEMM_CASE(true, false, true, false)
  TLH_GEMM_CASE(true, true, true, false)
  TLH_GEMM_CASE(false, false, false, false)
  TLH_GEMM_CASE(false, true, false, false)
  TLH_GEMM_CASE(true, false, false, false)
  TLH_GEMM_CASE(true, true, false, false)
#undef TLH_GEMM_CASE
}

template <int BM, int BN, int BK>
void launch16(const GemmParams &p, bool ta, bool tb, bool vec, bool full, dim3 grid,
              hipStream_t s) {
#define TLH_GEMM_CASE(TA_, TB_, V_, F_)                                             \
  if (ta == TA_ && tb == TB_ && vec == V_ && full == F_) {                          \
    gemm_mfma16_kernel<BM, BN, BK, TA_, TB_, V_, F_><<<grid, 256, 0, s>>>(p);       \
    return;                                                                         \
  }
  TLH_GEMM_CASE(false, false, true, true)
  TLH_GEMM_CASE(false, true, true, true)
  TLH_GEMM_CASE(true, false, true, true)
  TLH_GEMM_CASE(true, true, true, true)
  TLH_GEMM_CASE(false, false, true, false)
  TLH_GEMM_CASE(false, true, true, false)
  TLH_GEMM_CASE(true, false, true, false)
  TLH_GEMM_CASE(true, true, true, false)
  TLH_GEMM_CASE(false, false, false, false)
  TLH_GEMM_CASE(false, true, false, false)
  TLH_GEMM_CASE(true, false, false, false)
  TLH_GEMM_CASE(true, true, false, false)
#undef TLH_GEMM_CASE
}

inline size_t tiles_for(const GemmDesc &d, int bm, int bn) {
  return size_t((d.M + bm - 1) / bm) * size_t((d.N + bn - 1) / bn);
}

constexpr int kTargetBlocks = 256; // one block per CU at least
constexpr int kMinTailSplitK = 1024; // shortest K the tail split (below) is used for

// Process-wide plan override for tuning sweeps (tlh_gemm_set_plan); 0 = the
// planner decides.
int g_force_bm = 0, g_force_bn = 0, g_force_splits = 0, g_force_bk = 16;
int g_tile16_wgrad = 1; // split weight gradients on the 16x16x4 kernel
int g_tile16_rowb = 1;  // products with B row-contiguous on the 16x16x4 kernel
int g_xcd_remap = 1;
int g_xcd_rects = 1;
int g_gemv = 1;
// float4 split-K reduce over a (plane, entry) grid (see gemm_splitk_reduce4)
int g_reduce4 = 1;


// The 8-way partition of a tiles_m x tiles_n grid into equal rectangles
// (1x8, 2x4, 4x2 or 8x1 of them) whose rectangle needs the fewest operand
// panels (rect_m A row panels + rect_n B column panels), used when it needs
// fewer than the contiguous range of the same size, which spans
// ceil(G/8 / tiles_n) tile rows (one more when it starts mid-row) and up to
// tiles_n columns. {0, 0}: none.
struct XcdRect {
  int rect_m = 0, rect_n = 0;
};
XcdRect xcd_rect(int tiles_m, int tiles_n) {
  XcdRect best;
  const long tiles = long(tiles_m) * tiles_n;
  if (tiles_m <= 0 || tiles_n <= 0 || tiles % 8 != 0) return best;
  const long per = tiles / 8;
  const long rows = (per + tiles_n - 1) / tiles_n + (per % tiles_n ? 1 : 0);
  long best_cost = std::min<long>(rows, tiles_m) + std::min<long>(per, tiles_n);
  for (int px = 1; px <= 8; px *= 2) {
    const int py = 8 / px;
    if (tiles_m % px || tiles_n % py) continue;
    const long cost = tiles_m / px + tiles_n / py;
    if (cost < best_cost) {
      best_cost = cost;
      best.rect_m = tiles_m / px;
      best.rect_n = tiles_n / py;
    }
  }
  return best;
}
int g_tail_split = 1;
int g_tile96 = 1; // 96x96 tiles for tile-aligned products (see make_plan)
int g_xcd_zmajor = 1; // split-major XCD order of split-K / batched grids
constexpr int kMinSplitK = 256;    // K elements per split-K chunk, at least

bool vec_ok(const GemmDesc &d) {
  auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int a_contig = d.trans_a ? d.M : d.K;
  const int b_contig = d.trans_b ? d.K : d.N;
  if (!al(d.A) || !al(d.B)) return false;
  if (a_contig % 4 || b_contig % 4 || d.lda % 4 || d.ldb % 4) return false;
  if (d.batch_ndim > 0) {
    for (int i = 0; i < d.batch_ndim; ++i)
      if (d.batch_stride_a[i] % 4 || d.batch_stride_b[i] % 4) return false;
  }
  return true;
}

// Tile plan, from measurements on MI355X of the GPT step's shapes
// (M, N, K in {384, 1536, 2048, 6144}) and the d=1024 shapes:
//  - 128x128 tiles (K tile 16) only when they give every CU three or more
//    blocks and pad the output little more than 64x64 tiles do (192x192
//    attention scores: 4 tiles of 128 cover 1.8x the area, 9 of 64 exactly,
//    and run 2x faster) and K >= 384 (with K = 192 the tile's fill and
//    epilogue outweigh its reuse: the reference executor's per-sequence
//    weight gradients [32 x 384x192 . 192x1536] take 118 us on 128x128 tiles,
//    90 us on 64x64); their 4 accumulators per wave win when the grid is
//    deep;
//  - otherwise 64x64 tiles with a K tile of 32 (16 when K <= 256: the
//    executor's K = 64 attention scores 19 us instead of 23): 2-4
//    co-resident blocks per CU hide the global/LDS latency a single block
//    per CU cannot;
//  - K >= 1024 with at least 3 tiles of 64x128 per CU: 64x128 tiles (K tile
//    16), also in place of 128x128 when B is transposed (the d = 1024 / T =
//    1024 shapes: 4-7% faster than 64x64, and than 128x128 for dG);
//  - tall-K products (weight gradients, K = B*T) with too few output tiles
//    split K so that about 768 blocks (3 per CU) run, each with K chunks of
//    >= 256 ([384,2048] with K = 6144: 4 splits, 10% faster than 8).
Plan make_plan(const GemmDesc &d, bool allow_split) {
  // Summed batch entries are one product over the folded K (see gemm_launch).
  const size_t outputs = d.sum_batches ? 1 : size_t(std::max(1, d.batch));
  const int K = d.sum_batches ? d.K * d.batch : d.K;
  const bool one_dim = d.sum_batches || d.batch_ndim <= 1;
  if (g_force_bm > 0) {
    const bool can_split = allow_split && one_dim;
    if (g_force_bm == 16) // 16x16 MFMA, square tiles of g_force_bn, K tile 32
      return {g_force_bn, g_force_bn, can_split ? std::max(1, g_force_splits) : 1, 32, true};
    if (g_force_bm == 96 && g_force_bn == 64) { // 96x64 tiles
      // 8 waves over K tiles of 64 (as 96x96 below), else 4 waves
      if (g_force_bk == 64 && !d.bias_grad && (!d.sum_batches || d.K % 64 == 0))
        return {96, 64, 1, 64};
      return {96, 64, can_split ? std::max(1, g_force_splits) : 1, 32};
    }
    if (g_force_bm == 96) { // 16x16 MFMA tiles, no bias gradient
      if (d.bias_grad) return {64, 64, 1, 32};
      // 8 waves over K tiles of 64: no split-K, summed entries of 64 | K
      if (g_force_bk == 64 && (!d.sum_batches || d.K % 64 == 0)) return {96, 96, 1, 64};
      return {96, 96, can_split ? std::max(1, g_force_splits) : 1, 32};
    }
    return {g_force_bm, g_force_bn, can_split ? std::max(1, g_force_splits) : 1, g_force_bk};
  }
  // 96x96 tiles on the 16x16x4 MFMA for tile-aligned outputs of 3/4 to 4
  // tiles per CU: [6144, 384] is exactly one tile per CU where 64x64 tiles
  // leave 64 CUs a third block (75% balance), [6144, 1536] four. At one
  // tile per CU or fewer, 8 waves over K tiles of 64 (two wave groups per
  // block: 25.0 -> 22.9 us at K = 384); above, 4 waves with two blocks
  // co-resident per CU (N = 1536: 76.4 -> 69.2 us against 64x64).
  // Measured on MI355X at M = 6144, N = 384 / 1536, K = 96 .. 3072, and the
  // batched (3 x 256 tiles: 67.0 -> 64.4 us) and summed-batch Q/K/V forms.
  if (g_tile96 && !d.bias_grad && !d.trans_a && vec_ok(d) && d.M % 96 == 0 && d.N % 96 == 0 &&
      K % 32 == 0 && K >= 128) {
    const size_t t96 = tiles_for(d, 96, 96) * outputs;
    const size_t cus = size_t(cu_count());
    const bool k64 = K % 64 == 0 && (!d.sum_batches || d.K % 64 == 0);
    // (fewer tiles than about one per CU leave the product to split-K)
    if (4 * t96 >= 3 * cus && t96 <= cus && k64) return {96, 96, 1, 64};
    if (4 * t96 >= 3 * cus && t96 <= 4 * cus) return {96, 96, 1, 32};
  }
  // 96x64 tiles where they cover the output in 3/4 to 1 tile per CU and
  // 64x64 tiles would give some CUs a second one: [768,384].[384,1536]
  // (matmul + bias at batch 4 x 192) is 192 tiles instead of 288. With K
  // tiles of 64 the block has 8 waves in two K groups (two waves per SIMD):
  // 19.8 us on 64x64 tiles, 17.9 on 4-wave and 15.9 on 8-wave 96x64 tiles.
  if (g_tile96 && !d.trans_a && !d.bias_grad && vec_ok(d) && d.M % 96 == 0 && d.N % 64 == 0 &&
      K % 32 == 0 && K >= 128) {
    const size_t cus = size_t(cu_count());
    const size_t t = tiles_for(d, 96, 64) * outputs;
    const bool k64 = K % 64 == 0 && (!d.sum_batches || d.K % 64 == 0);
    if (4 * t >= 3 * cus && t <= cus && tiles_for(d, 64, 64) * outputs > cus)
      return {96, 64, 1, k64 ? 64 : 32};
  }
  // output area over the area of the tiles that cover it
  auto coverage = [&](int bm, int bn) {
    return double(d.M) * double(d.N) /
           (double((d.M + bm - 1) / bm * bm) * double((d.N + bn - 1) / bn * bn));
  };
  // B row-contiguous in LDS (not transposed, A not transposed either): the
  // 16x16x4 kernel's interleaved B reads win at 128x128 where those tiles
  // are taken ([8192,1024].[1024,4096] 559 -> 541 us, [8192,1024].[1024,1024]
  // 152 -> 137 us, [6144,384].[384,2048] 96 -> 91 us) and at 64x64 for K >=
  // 384 and below the tail split's K ([768,384].[384,1536] 21.5 -> 19.0
  // us).
  const bool row_b = g_tile16_rowb && !d.trans_a && !d.trans_b && K % 32 == 0;
  if (K >= 384 && tiles_for(d, 128, 128) * outputs >= 3 * size_t(kTargetBlocks) &&
      coverage(128, 128) >= 0.9 * coverage(64, 64)) {
    if (row_b) return {128, 128, 1, 32, true};
    return (K >= 1024 && d.trans_b) ? Plan{64, 128, 1, 16} : Plan{128, 128, 1, 16};
  }
  if (K >= 1024 && tiles_for(d, 64, 128) * outputs >= 3 * size_t(kTargetBlocks) &&
      coverage(64, 128) >= 0.9 * coverage(64, 64))
    return row_b ? Plan{128, 128, 1, 32, true} : Plan{64, 128, 1, 16};
  const size_t tiles = tiles_for(d, 64, 64) * outputs;
  // weight gradients (transposed A, K = tokens) split K below 3 tiles per CU:
  // one long whole-K block per CU runs [1024,1024] x K 8192 at 72 TFLOP/s, 8
  // splits at 105. With both operand tiles row-contiguous (A transposed, B
  // not) the 16x16x4 kernel reads them with interleaved subtiles: [384,384]
  // 38.7 -> 35.9 us, [1536,384] 99.7 -> 84.7, [384,1536] 100.7 -> 86.5,
  // [384,2048] 104.8 -> 98.1 (K = 6144).
  const size_t split_below = (d.trans_a ? 3 : 1) * size_t(kTargetBlocks);
  if (allow_split && one_dim && tiles < split_below && K >= 2 * kMinSplitK) {
    int splits = 1;
    while (splits < 16 && tiles * size_t(splits) < 3 * size_t(kTargetBlocks) &&
           K / (splits * 2) >= kMinSplitK)
      splits *= 2;
    if (splits >= 2) return {64, 64, splits, 32, g_tile16_wgrad && d.trans_a && !d.trans_b};
  }
  // (from K = 1024 the tail split on the 32x32 kernel is taken instead)
  if (row_b && K >= 384 && K < kMinTailSplitK) return {64, 64, 1, 32, true};
  return {64, 64, 1, K <= 256 ? 16 : 32};
}


// One-row products that take the GEMV path: x [1, K], B [K, N] row-major
// and float4-aligned, one batch dimension at most, no bias gradient.
bool gemv_ok(const GemmDesc &d) {
  if (d.M != 1 || d.trans_a || d.trans_b || d.bias_grad || d.sum_batches || d.K < 64) return false;
  if (d.batch_ndim > 1 || (d.batch_ndim == 0 && d.batch > 1)) return false;
  if (d.N % 4 || d.ldb % 4 || (reinterpret_cast<uintptr_t>(d.B) & 15)) return false;
  return d.batch_ndim == 0 || d.batch_stride_b[0] % 4 == 0;
}

// K chunks of the GEMV: about 256 blocks, chunks of >= 64 rows (multiples
// of 16: 4 waves x 4 loads in flight).
struct GemvPlan {
  int chunks = 1, chunk_k = 0;
};
GemvPlan gemv_plan(const GemmDesc &d) {
  GemvPlan g;
  const long col_blocks = (d.N + 255) / 256, entries = std::max(1, d.batch);
  long chunks = std::max<long>(1, 256 / (col_blocks * entries));
  chunks = std::min<long>(chunks, std::max(1, d.K / 64));
  long ck = (d.K + chunks - 1) / chunks;
  ck = (ck + 15) / 16 * 16;
  g.chunk_k = int(ck);
  g.chunks = int((d.K + ck - 1) / ck);
  return g;
}

} // namespace

int gemm_choose_splits(const GemmDesc &d) { return make_plan(d, true).splits; }

int cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Tail split of a tile-aligned single product (no split-K, no bias
// gradient). Its blocks run co-resident, so a CU holding ceil(tiles/CUs)
// blocks sets the time: 576 tiles on 256 CUs leave 64 CUs with a third
// block (75% balance). The first floor(tiles/CUs)*CUs tiles stay whole-K
// blocks; each remaining tile is cut into `splits` K chunks (multiples of
// kBK, so no K tile straddles a chunk or a K segment) that spread over the
// CUs, and gemm_tail_reduce sums them.

struct TailSplit {
  int dp_tiles = 0, tails = 0, splits = 0, k_chunk = 0;
  size_t elems(const Plan &plan) const { return size_t(tails) * splits * plan.bm * plan.bn; }
};

TailSplit tail_split(const GemmDesc &d, const Plan &plan, int K) {
  TailSplit t;
  if (!g_tail_split || plan.splits > 1 || plan.bm == 96 || plan.m16 || d.bias_grad ||
      (d.batch > 1 && !d.sum_batches))
    return t;
  // the reduction launch costs a few microseconds: only long K ranges gain
  if (d.M % plan.bm || d.N % plan.bn || K % plan.bk || K < kMinTailSplitK) return t;
  const int tiles = (d.M / plan.bm) * (d.N / plan.bn);
  const int cus = cu_count();
  const int per = tiles / cus, tail = tiles - per * cus;
  if (per < 1 || tail == 0 || double(tiles) / cus / (per + 1) >= 0.9) return t;
  int splits = std::min(16, cus / std::gcd(tail, cus));
  const int chunk = ((K + splits - 1) / splits + kBK - 1) / kBK * kBK;
  splits = (K + chunk - 1) / chunk;
  if (splits < 2) return t;
  t.dp_tiles = per * cus;
  t.tails = tail;
  t.splits = splits;
  t.k_chunk = chunk;
  return t;
}

int folded_k(const GemmDesc &d) { return d.sum_batches ? d.K * d.batch : d.K; }

size_t gemm_workspace_elems(const GemmDesc &d) {
  if (gemv_ok(d)) return size_t(std::max(1, d.batch)) * gemv_plan(d).chunks * size_t(d.N);
  const Plan plan = make_plan(d, true);
  const int s = plan.splits;
  const size_t outputs = d.sum_batches ? 1 : size_t(std::max(1, d.batch));
  // C partials [outputs, s, M, N] followed by bias-gradient partials
  // [outputs, s, N]
  if (s > 1) return outputs * size_t(s) * (size_t(d.M) * d.N + d.N);
  return tail_split(d, plan, folded_k(d)).elems(plan); // [tails, splits, bm*bn]
}

// A product planned for launch: its kernel parameters, tile plan, grid and
// the finishing pass it needs (gemm_prepare / gemm_main / gemm_finish).
struct Prepared {
  bool none = false; // nothing to launch (empty output or empty batch)
  bool gemv = false;
  GemvPlan gv;
  GemmParams p{};
  Plan plan;
  TailSplit ts;
  dim3 grid;
  bool ta = false, tb = false, vec = false, full = false;
  bool k_empty = false; // K == 0: the reducer writes the epilogue of 0
  size_t reduce_elems = 0;
  bool v4 = false; // float4 split-K reduction
};

int gemm_prepare(const GemmDesc &d, Prepared &L) {
  L = Prepared{};
  if (d.M <= 0 || d.N <= 0) {
    L.none = true;
    return 0;
  }
  if (d.bias_grad && (d.batch_ndim > 1 || d.remap_h > 0 || d.sum_batches))
    return int(hipErrorInvalidValue);
  // Summed batch entries: K segments of kBK-multiple length (a K tile never
  // straddles two entries' operands).
  if (d.sum_batches && (d.batch < 2 || d.batch_ndim != 1 || d.K % kBK))
    return int(hipErrorInvalidValue);
  GemmParams &p = L.p;
  p.A = d.A; p.B = d.B; p.C = d.C;
  p.bias = d.bias; p.residual = d.residual; p.aux = d.aux;
  p.workspace = d.workspace;
  p.bias_grad = d.bias_grad;
  p.M = d.M; p.N = d.N; p.K = d.K;
  p.lda = d.lda; p.ldb = d.ldb; p.ldc = d.ldc;
  p.beta = d.beta;
  p.epilogue = d.epilogue;
  p.remap_t = d.remap_t; p.remap_h = d.remap_h; p.remap_d = d.remap_d;
  p.batch_ndim = d.batch_ndim;
  p.bias_bstride = d.bias_batch_stride;
  {
    auto al16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    bool ov = al16(d.C) && (!d.residual || al16(d.residual)) && (!d.aux || al16(d.aux)) &&
              (!d.workspace || al16(d.workspace)) && d.N % 4 == 0 &&
              (d.remap_h > 0 ? d.remap_d % 4 == 0 : d.ldc % 4 == 0);
    for (int i = 0; i < d.batch_ndim && i < 4; ++i) ov = ov && d.batch_stride_c[i] % 4 == 0;
    p.out_vec = ov;
  }
  p.batch = std::max(1, d.batch);
  int K = d.K;
  if (d.sum_batches) { // fold the batch into K: one product over batch*K
    K = d.K * d.batch;
    p.K = K;
    p.seg_k = d.K;
    p.seg_a = d.batch_stride_a[0];
    p.seg_b = d.batch_stride_b[0];
    p.batch = 1;
    p.batch_ndim = 0;
  }
  for (int i = 0; i < 4; ++i) {
    p.batch_shape[i] = d.batch_shape[i];
    p.bsa[i] = d.batch_stride_a[i];
    p.bsb[i] = d.batch_stride_b[i];
    p.bsc[i] = d.batch_stride_c[i];
  }
  if (gemv_ok(d) && d.workspace && g_gemv &&
      (!d.workspace_elems || gemm_workspace_elems(d) <= d.workspace_elems)) {
    L.gemv = true;
    L.gv = gemv_plan(d);
    return 0;
  }
  Plan plan = make_plan(d, d.workspace != nullptr);
  if (plan.splits > 1 && d.workspace_elems && gemm_workspace_elems(d) > d.workspace_elems)
    plan = make_plan(d, false); // the given workspace is too small to split K
  L.plan = plan;
  p.tiles_n = (d.N + plan.bn - 1) / plan.bn;
  p.xcd_remap = g_xcd_remap;
  const int tiles_m = (d.M + plan.bm - 1) / plan.bm;
  p.splits = plan.splits;
  p.k_chunk = p.splits > 1 ? ((K + p.splits - 1) / p.splits + kBK - 1) / kBK * kBK : K;
  if (p.splits > 1) p.splits = (K + p.k_chunk - 1) / p.k_chunk; // <= plan.splits
  L.reduce_elems = size_t(d.M) * d.N;
  L.vec = vec_ok(d);
  TailSplit ts;
  if (p.splits <= 1 && d.workspace && L.vec) {
    ts = tail_split(d, plan, K);
    if (ts.splits && d.workspace_elems && d.workspace_elems < ts.elems(plan)) ts = TailSplit{};
  }
  L.ts = ts;
  p.dp_tiles = ts.dp_tiles;
  p.tail_tiles = ts.tails;
  p.tail_splits = ts.splits;
  p.tail_k_chunk = ts.k_chunk;
  p.rect_m = p.rect_n = 0;
  p.zmajor = 0;
  const int zext = p.splits > 1 ? p.batch * p.splits : p.batch;
  if (p.xcd_remap && g_xcd_zmajor && zext > 1 && !ts.splits &&
      (size_t(tiles_m) * p.tiles_n * zext) % 8 == 0) {
    // whole K splits / batch entries per XCD; the tiles of one go in row-
    // major order to consecutive blocks of that XCD
    p.zmajor = zext;
    p.xcd_remap = 0;
  } else if (p.xcd_remap && g_xcd_rects && !ts.splits) {
    const XcdRect r = xcd_rect(tiles_m, p.tiles_n);
    p.rect_m = r.rect_m;
    p.rect_n = r.rect_n;
  }
  if (K <= 0) { // nothing to accumulate: the reducer applies the epilogue to 0
    p.splits = 0;
    L.k_empty = true;
    return 0;
  }
  const int z = p.splits > 1 ? p.batch * p.splits : p.batch;
  const int blocks = ts.splits ? ts.dp_tiles + ts.tails * ts.splits : tiles_m * p.tiles_n;
  L.grid = dim3(unsigned(blocks), 1, unsigned(z));
  L.ta = d.trans_a != 0;
  L.tb = d.trans_b != 0;
  // Every block's K range is a multiple of the K tile when K is and the
  // split chunk (a multiple of kBK) is.
  L.full = L.vec && d.M % plan.bm == 0 && d.N % plan.bn == 0 && K % plan.bk == 0 &&
           (p.splits <= 1 || p.k_chunk % plan.bk == 0);
  // The workspace planes start 16-byte aligned when M*N is a multiple of 4.
  L.v4 = d.N % 4 == 0 && (reinterpret_cast<uintptr_t>(d.workspace) & 15) == 0;
  return 0;
}

// The product's tile (or GEMV partial) kernel.
int gemm_main(const Prepared &L, hipStream_t s) {
  if (L.none) return 0;
  const GemmParams &p = L.p;
  if (L.gemv) {
    dim3 grid(unsigned((p.N + 255) / 256), unsigned(L.gv.chunks), unsigned(p.batch));
    gemv_partial_kernel<<<grid, 256, 0, s>>>(p, L.gv.chunk_k, L.gv.chunks);
    return launch_status();
  }
  if (L.k_empty) return 0;
  const Plan &plan = L.plan;
  const bool ta = L.ta, tb = L.tb, vec = L.vec, full = L.full;
  const dim3 grid = L.grid;
  if (plan.m16 && plan.bm == 64) {
    launch16<64, 64, 32>(p, ta, tb, vec, full, grid, s);
  } else if (plan.m16 && plan.bm == 128) {
    launch16<128, 128, 32>(p, ta, tb, vec, full, grid, s);
  } else if (plan.bm == 96 && plan.bn == 64 && plan.bk == 64) {
    launch16x8<96, 64>(p, ta, tb, vec, full, grid, s);
  } else if (plan.bm == 96 && plan.bn == 64) {
    launch16<96, 64, 32>(p, ta, tb, vec, full, grid, s);
  } else if (plan.bm == 96 && plan.bk == 64) {
    launch16x8<96, 96>(p, ta, tb, vec, full, grid, s);
  } else if (plan.bm == 96) {
    launch16<96, 96, 32>(p, ta, tb, vec, full, grid, s);
  } else if (plan.bk == 32) {
    if (plan.bm == 128 && plan.bn == 128) launch_cfg<128, 128, 64, 64, 32>(p, ta, tb, vec, full, grid, s);
    else if (plan.bm == 128 && plan.bn == 64) launch_cfg<128, 64, 64, 32, 32>(p, ta, tb, vec, full, grid, s);
    else if (plan.bm == 64 && plan.bn == 128) launch_cfg<64, 128, 32, 64, 32>(p, ta, tb, vec, full, grid, s);
    else launch_cfg<64, 64, 32, 32, 32>(p, ta, tb, vec, full, grid, s);
  } else {
    if (plan.bm == 128 && plan.bn == 128) launch_cfg<128, 128, 64, 64, 16>(p, ta, tb, vec, full, grid, s);
    else if (plan.bm == 128 && plan.bn == 64) launch_cfg<128, 64, 64, 32, 16>(p, ta, tb, vec, full, grid, s);
    else if (plan.bm == 64 && plan.bn == 128) launch_cfg<64, 128, 32, 64, 16>(p, ta, tb, vec, full, grid, s);
    else launch_cfg<64, 64, 32, 32, 16>(p, ta, tb, vec, full, grid, s);
  }
  return launch_status();
}

// The product's finishing pass: GEMV chunk sums, tail-tile or split-K
// reduction (with the epilogue), or the epilogue of an empty K range.
int gemm_finish(const Prepared &L, hipStream_t s) {
  if (L.none) return 0;
  const GemmParams &p = L.p;
  if (L.gemv) {
    gemv_reduce_kernel<<<dim3(unsigned((p.N + 63) / 64), unsigned(p.batch)), 256, 0, s>>>(
        p, L.gv.chunks);
    return launch_status();
  }
  if (L.k_empty) {
    gemm_splitk_reduce<false><<<stride_grid(L.reduce_elems, 256), 256, 0, s>>>(p);
    return launch_status();
  }
  const Plan &plan = L.plan;
  if (L.ts.splits) {
    const size_t groups = size_t(L.ts.tails) * plan.bm * plan.bn / 4;
    const unsigned g = stride_grid(groups, 256);
    if (plan.bm == 128 && plan.bn == 128) gemm_tail_reduce<128, 128><<<g, 256, 0, s>>>(p);
    else if (plan.bm == 128) gemm_tail_reduce<128, 64><<<g, 256, 0, s>>>(p);
    else if (plan.bn == 128) gemm_tail_reduce<64, 128><<<g, 256, 0, s>>>(p);
    else gemm_tail_reduce<64, 64><<<g, 256, 0, s>>>(p);
    return launch_status();
  }
  if (p.splits > 1) {
    const size_t reduce_elems = L.reduce_elems;
    if (L.v4 && p.splits <= kMaxSplits && p.batch <= 65535 && g_reduce4)
      gemm_splitk_reduce4<<<dim3(unsigned((std::max(reduce_elems / 4, size_t(p.N)) + 255) / 256),
                                 unsigned(p.batch)),
                            256, 0, s>>>(p);
    else if (L.v4)
      gemm_splitk_reduce<true><<<stride_grid(reduce_elems / 4 + 1, 256), 256, 0, s>>>(p);
    else
      gemm_splitk_reduce<false><<<stride_grid(reduce_elems, 256), 256, 0, s>>>(p);
    return launch_status();
  }
  return 0;
}

int gemm_launch(const GemmDesc &d, void *stream) {
  Prepared L;
  int st = gemm_prepare(d, L);
  if (st) return st;
  hipStream_t s = as_stream(stream);
  if ((st = gemm_main(L, s))) return st;
  return gemm_finish(L, s);
}

} // namespace tlh

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
#include "../../include/templit_hip.h"

namespace {
tlh::GemmDesc from_c(const tlh_gemm_desc &c) {
  tlh::GemmDesc d;
  d.A = c.a; d.B = c.b; d.C = c.c;
  d.bias = c.bias; d.residual = c.residual; d.aux = c.aux;
  d.workspace = c.workspace;
  d.workspace_elems = c.workspace_elems;
  d.M = c.m; d.N = c.n; d.K = c.k;
  d.lda = c.lda; d.ldb = c.ldb; d.ldc = c.ldc;
  d.trans_a = c.trans_a; d.trans_b = c.trans_b;
  d.beta = c.beta;
  d.epilogue = c.epilogue;
  d.remap_t = c.remap_t; d.remap_h = c.remap_h; d.remap_d = c.remap_d;
  d.bias_grad = c.bias_grad;
  if (c.batch > 1) {
    d.batch = c.batch;
    d.batch_ndim = 1;
    d.batch_shape[0] = uint32_t(c.batch);
    d.batch_stride_a[0] = c.batch_stride_a;
    d.batch_stride_b[0] = c.batch_stride_b;
    d.batch_stride_c[0] = c.batch_stride_c;
    d.bias_batch_stride = c.bias_batch_stride;
    d.sum_batches = c.sum_batches != 0;
  }
  return d;
}
} // namespace

TLH_API int tlh_gemm_set_plan(int bm, int bn, int splits, int bk) {
  // bk < 0 toggles instead: the XCD-aware block order off (-1) or on (-2),
  // the tail split off (-3) or on (-4), the XCD rectangles off (-5) or on
  // (-6), the one-row GEMV off (-7) or on (-8), the float4 split-K reduction
  // off (-9) or on (-10), the planner's 96x96 tiles off (-11) or on (-12),
  // the split-major XCD order off (-13) or on (-14), split weight gradients
  // on the 16x16x4 kernel off (-15) or on (-16), products with B not
  // transposed on the 16x16x4 kernel off (-17) or on (-18). bm = 16 forces the 16x16x4
  // kernel with square tiles of bn (64 or 128) and a K tile of 32.
  if (bk == -1 || bk == -2) {
    tlh::g_xcd_remap = bk == -2;
    return 0;
  }
  if (bk == -3 || bk == -4) {
    tlh::g_tail_split = bk == -4;
    return 0;
  }
  if (bk == -5 || bk == -6) {
    tlh::g_xcd_rects = bk == -6;
    return 0;
  }
  if (bk == -7 || bk == -8) {
    tlh::g_gemv = bk == -8;
    return 0;
  }
  if (bk == -9 || bk == -10) {
    tlh::g_reduce4 = bk == -10;
    return 0;
  }
  if (bk == -11 || bk == -12) {
    tlh::g_tile96 = bk == -12;
    return 0;
  }
  if (bk == -13 || bk == -14) {
    tlh::g_xcd_zmajor = bk == -14;
    return 0;
  }
  if (bk == -15 || bk == -16) {
    tlh::g_tile16_wgrad = bk == -16;
    return 0;
  }
  if (bk == -17 || bk == -18) {
    tlh::g_tile16_rowb = bk == -18;
    return 0;
  }
  const bool ok = (bm == 0 && bn == 0) || (bm == 96 && bn == 96 && (bk == 32 || bk == 64)) ||
                  (bm == 96 && bn == 64 && (bk == 32 || bk == 64)) ||
                  (bm == 16 && (bn == 64 || bn == 128) && bk == 32) ||
                  ((bm == 64 || bm == 128) && (bn == 64 || bn == 128));
  if (!ok || splits < 0 || splits > 64 || (bk != 16 && bk != 32 && (bk != 64 || bm != 96)))
    return int(hipErrorInvalidValue);
  tlh::g_force_bm = bm;
  tlh::g_force_bn = bn;
  tlh::g_force_splits = splits;
  tlh::g_force_bk = bk;
  return 0;
}

namespace {
// The descriptor checks of tlh_gemm (0 or hipErrorInvalidValue).
int check_desc(const tlh_gemm_desc &c, const tlh::GemmDesc &d) {
  if (d.M < 0 || d.N < 0 || d.K < 0) return int(hipErrorInvalidValue);
  if ((d.epilogue == tlh::kEpiGelu || d.epilogue == tlh::kEpiGeluBwd) && !d.aux)
    return int(hipErrorInvalidValue);
  if (d.remap_h > 0 && (d.remap_t <= 0 || d.remap_d <= 0 ||
                        (d.M % d.remap_t && d.M > d.remap_t) || d.N != d.remap_h * d.remap_d))
    return int(hipErrorInvalidValue);
  if (c.batch > 1 && (d.aux || d.epilogue != tlh::kEpiStore || (d.residual && !d.sum_batches)))
    return int(hipErrorInvalidValue);
  return 0;
}
} // namespace

TLH_API int tlh_gemm(const tlh_gemm_desc *desc, void *stream) {
  if (!desc) return int(hipErrorInvalidValue);
  tlh::GemmDesc d = from_c(*desc);
  const int st = check_desc(*desc, d);
  if (st) return st;
  return tlh::gemm_launch(d, stream);
}

TLH_API int tlh_gemm_workspace_size(const tlh_gemm_desc *desc, size_t *elems) {
  if (!desc || !elems) return int(hipErrorInvalidValue);
  *elems = tlh::gemm_workspace_elems(from_c(*desc));
  return 0;
}

namespace {
// tlh_matmul's strided operands -> a GemmDesc (`skip`: nothing to compute).
int matmul_desc(const float *a, const float *b, float *c, uint32_t M, uint32_t K, uint32_t N,
                uint32_t a_rs, uint32_t a_cs, uint32_t b_rs, uint32_t b_cs, uint32_t c_rs,
                uint32_t c_cs, uint32_t batch_ndim, const uint32_t *batch_shape,
                const uint32_t *batch_stride_a, const uint32_t *batch_stride_b,
                const uint32_t *batch_stride_c, tlh::GemmDesc &d, bool &skip) {

  skip = false;
  if (batch_ndim > 4 || c_cs != 1) return int(hipErrorInvalidValue);
  if (M == 0 || N == 0) { skip = true; return 0; }
  d.A = a; d.B = b; d.C = c;
  d.M = int(M); d.N = int(N); d.K = int(K);
  // A: row-major (column stride 1) or column-major (row stride 1).
  if (a_cs == 1 || K == 1) { d.trans_a = 0; d.lda = int(a_cs == 1 ? a_rs : 1); }
  else if (a_rs == 1 || M == 1) { d.trans_a = 1; d.lda = int(a_cs); }
  else return int(hipErrorInvalidValue);
  if (b_cs == 1 || N == 1) { d.trans_b = 0; d.ldb = int(b_cs == 1 ? b_rs : 1); }
  else if (b_rs == 1 || K == 1) { d.trans_b = 1; d.ldb = int(b_cs); }
  else return int(hipErrorInvalidValue);
  if (d.trans_a == 0 && K == 1) d.lda = int(a_rs);
  d.ldc = int(c_rs);
  size_t batch = 1;
  d.batch_ndim = int(batch_ndim);
  for (uint32_t i = 0; i < batch_ndim; ++i) {
    d.batch_shape[i] = batch_shape[i];
    d.batch_stride_a[i] = batch_stride_a[i];
    d.batch_stride_b[i] = batch_stride_b[i];
    d.batch_stride_c[i] = batch_stride_c[i];
    batch *= batch_shape[i];
  }
  if (batch == 0) { skip = true; return 0; }
  if (batch > 65535) return int(hipErrorInvalidValue);
  d.batch = int(batch);
  // Collapse a batch whose right operand is shared (stride 0 on every batch
  // dim) and whose left operand and output are packed row-major into one
  // tall GEMM with batch*M rows (the weight-broadcast case of nn::Layer).
  bool b_shared = true, packed = (d.trans_a == 0);
  size_t expect = size_t(M);
  for (int i = int(batch_ndim) - 1; i >= 0; --i) {
    if (batch_shape[i] == 1) continue;
    if (batch_stride_b[i] != 0) b_shared = false;
    if (size_t(batch_stride_a[i]) != expect * size_t(d.lda) ||
        size_t(batch_stride_c[i]) != expect * d.ldc)
      packed = false;
    expect *= batch_shape[i];
  }
  if (batch > 1 && b_shared && packed && size_t(d.lda) == K && size_t(d.ldc) == N &&
      batch * M <= 0x7fffffffu) {
    d.M = int(batch * M);
    d.batch = 1;
    d.batch_ndim = 0;
  }
  if (d.batch == 1) d.batch_ndim = 0;
  return 0;
}
} // namespace

#define TLH_MATMUL_ARGS                                                                   \
  a, b, c, M, K, N, a_rs, a_cs, b_rs, b_cs, c_rs, c_cs, batch_ndim, batch_shape,           \
      batch_stride_a, batch_stride_b, batch_stride_c

TLH_API int tlh_matmul(const float *a, const float *b, float *c, uint32_t M,
                       uint32_t K, uint32_t N, uint32_t a_rs, uint32_t a_cs,
                       uint32_t b_rs, uint32_t b_cs, uint32_t c_rs, uint32_t c_cs,
                       uint32_t batch_ndim, const uint32_t *batch_shape,
                       const uint32_t *batch_stride_a, const uint32_t *batch_stride_b,
                       const uint32_t *batch_stride_c, void *stream) {
  tlh::GemmDesc d;
  bool skip = false;
  const int st = matmul_desc(TLH_MATMUL_ARGS, d, skip);
  if (st || skip) return st;
  return tlh::gemm_launch(d, stream);
}

TLH_API int tlh_matmul_workspace_size(uint32_t M, uint32_t K, uint32_t N, uint32_t a_rs,
                                      uint32_t a_cs, uint32_t b_rs, uint32_t b_cs,
                                      uint32_t c_rs, uint32_t c_cs, uint32_t batch_ndim,
                                      const uint32_t *batch_shape,
                                      const uint32_t *batch_stride_a,
                                      const uint32_t *batch_stride_b,
                                      const uint32_t *batch_stride_c, size_t *elems) {
  if (!elems) return int(hipErrorInvalidValue);
  *elems = 0;
  const float *a = nullptr, *b = nullptr;
  float *c = nullptr;
  tlh::GemmDesc d;
  bool skip = false;
  const int st = matmul_desc(TLH_MATMUL_ARGS, d, skip);
  if (st || skip) return st;
  *elems = tlh::gemm_workspace_elems(d);
  return 0;
}

TLH_API int tlh_matmul_ws(const float *a, const float *b, float *c, uint32_t M, uint32_t K,
                          uint32_t N, uint32_t a_rs, uint32_t a_cs, uint32_t b_rs,
                          uint32_t b_cs, uint32_t c_rs, uint32_t c_cs, uint32_t batch_ndim,
                          const uint32_t *batch_shape, const uint32_t *batch_stride_a,
                          const uint32_t *batch_stride_b, const uint32_t *batch_stride_c,
                          float *workspace, size_t workspace_elems, void *stream) {
  tlh::GemmDesc d;
  bool skip = false;
  const int st = matmul_desc(TLH_MATMUL_ARGS, d, skip);
  if (st || skip) return st;
  if (workspace && workspace_elems) {
    d.workspace = workspace;
    d.workspace_elems = workspace_elems;
  }
  return tlh::gemm_launch(d, stream);
}
TLH_API int tlh_matmul_bias_ws(const float *a, const float *b, float *c, const float *bias,
                               float *gelu_pre, uint32_t M, uint32_t K, uint32_t N,
                               uint32_t a_rs, uint32_t a_cs,
                               uint32_t b_rs, uint32_t b_cs, uint32_t c_rs, uint32_t c_cs,
                               uint32_t batch_ndim, const uint32_t *batch_shape,
                               const uint32_t *batch_stride_a, const uint32_t *batch_stride_b,
                               const uint32_t *batch_stride_c, float *workspace,
                               size_t workspace_elems, void *stream) {
  if (!bias) return int(hipErrorInvalidValue);
  tlh::GemmDesc d;
  bool skip = false;
  const int st = matmul_desc(TLH_MATMUL_ARGS, d, skip);
  if (st || skip) return st; // (skip: no output elements)
  d.bias = bias;
  d.bias_batch_stride = 0;
  if (gelu_pre) { // c = GELU(x), gelu_pre = x: one product, no batch entries
    if (d.batch > 1) return int(hipErrorInvalidValue);
    d.epilogue = tlh::kEpiGelu;
    d.aux = gelu_pre;
  }
  if (workspace && workspace_elems) {
    d.workspace = workspace;
    d.workspace_elems = workspace_elems;
  }
  return tlh::gemm_launch(d, stream);
}
TLH_API int tlh_matmul_noalloc(const float *a, const float *b, float *c, uint32_t M,
                               uint32_t K, uint32_t N, uint32_t a_rs, uint32_t a_cs,
                               uint32_t b_rs, uint32_t b_cs, uint32_t c_rs, uint32_t c_cs,
                               uint32_t batch_ndim, const uint32_t *batch_shape,
                               const uint32_t *batch_stride_a, const uint32_t *batch_stride_b,
                               const uint32_t *batch_stride_c, void *stream) {
  tlh::GemmDesc d;
  bool skip = false;
  int st = matmul_desc(TLH_MATMUL_ARGS, d, skip);
  if (st || skip) return st;
  const size_t need = tlh::gemm_workspace_elems(d);
  if (need > TLH_NOALLOC_SCRATCH_FLOATS) return int(hipErrorInvalidValue);
  if (need) {
    float *ws = nullptr;
    if ((st = tlh::noalloc_scratch(&ws))) return st;
    d.workspace = ws;
    d.workspace_elems = need;
  }
  return tlh::gemm_launch(d, stream);
}
#undef TLH_MATMUL_ARGS

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point
// ---------------------------------------------------------------------------
// K-chunk partials of tlh_matmul_noalloc. Each GPU the library runs on holds
// its own copy from module load until the process ends. In host code the
// name `scratch` is a host-side stand-in, not a device address: kernels get
// the address hipGetSymbolAddress returns for the current device, resolved
// once per device and kept in g_scratch_ptr. Every partial plane is written
// before it is read, so the array needs no clearing between calls.
static __device__ __align__(256) float scratch[TLH_NOALLOC_SCRATCH_FLOATS];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxScratchDevices] = {};
} // namespace

namespace tlh {
int noalloc_scratch(float **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return int(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return int(e);
    if (!p) return int(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = static_cast<float *>(p);
  }
  if (out) *out = g_scratch_ptr[dev];
  return 0;
}
} // namespace tlh
