// Fused causal multi-head attention, forward and backward, on fp32 MFMA.
//
// No reference kernel: the reference builds attention from ~14 runtime calls
// per block (include/nn/multi_head.h:37-52): split_last_dim + transpose for
// Q/K/V, a transpose of K, a batched matmul, divide by sqrt(64), add the
// causal mask (include/nn/attention.h:9-22), softmax, matmul with V,
// transpose + merge_last_dims -- materialising [B,H,T,T] scores twice.
// Here each wave keeps 32 query (or key) rows in registers and streams
// 64-row K/V (or Q/dO) tiles through LDS; scores never reach HBM.
// A block owns 64 rows (two 32-row tiles) and has 4 waves: wave w works on
// row tile w%2 and on half w/2 of every streamed 64-row tile, so each
// 64-row tile feeds four waves and a short sequence still gives every SIMD
// two or more waves. The two halves' partial results (softmax state and O,
// or dK/dV, or dQ) are combined through LDS at the end.
// Grid: x = batch*head, y = 64-row block, ordered so that the blocks with
// the most causal work are dispatched first (the short ones fill the tail).
//
// MFMA v_mfma_f32_32x32x2f32, 64 lanes, r = lane%32, h = lane/32:
//   A operand: A[m=r][k-slot h];  B operand: B[k-slot h][n=r];
//   accumulator reg v: D[m = 8*(v/4) + 4*h + v%4][n = r].
// The forward computes S^T = K.Q^T (m = key, n = query). Its accumulator
// holds, per lane, keys key(v,h) = 8*(v/4)+4h+v%4 of query r -- exactly the
// B-operand layout P^T needs for O^T = V^T.P^T when step s uses k-slot key
// key(s,h). So P never leaves the registers. The backward uses the same
// identity in both directions.
#include "common.h"

#include "../../include/templit_hip.h"

using namespace tlh;

namespace {

constexpr int HD = 64;       // head dim
constexpr int LDP = HD + 4;  // padded LDS row (floats)
constexpr int KB = 64;       // rows per streamed LDS tile
constexpr int WQ = 32;       // rows per wave
constexpr int BQ = 2 * WQ;   // rows per block (two row tiles x two halves of the stream)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 2^x on the hardware unit (v_exp_f32): 2^-inf = 0, results below the
// normal range flush to 0. Softmax and its backward evaluate
// exp(s*scale - m) as 2^(s*scale*log2(e) - m*log2(e)).
__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

struct Dims {
  uint32_t B, H, T;
};

// element offset of (b, h, t, 0) in head layout [B,H,T,D] or merged [B,T,H*D]
__device__ inline size_t row_off(const Dims &d, uint32_t b, uint32_t h, uint32_t t, int merged) {
  return merged ? ((size_t(b) * d.T + t) * d.H + h) * HD : ((size_t(b) * d.H + h) * d.T + t) * HD;
}

__device__ inline int key_of(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

__device__ inline f16x mfma(float a, float b, const f16x &c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Rows [r0, r0+64) of a [T, 64] head matrix held by the block's 256 threads
// (4 float4 each; rows >= T are zero): fetched from global memory into
// registers while the previous tile is being used, then put into LDS.
struct TileRegs {
  f4 v[4];
};

__device__ inline void fetch_tile(TileRegs &t, const float *src_base, const Dims &d, uint32_t b,
                                  uint32_t h, int r0, int merged) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = threadIdx.x + i * 256;
    const int row = idx >> 4, c4 = idx & 15;
    const int tt = r0 + row;
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (tt < int(d.T)) v = *reinterpret_cast<const f4 *>(src_base + row_off(d, b, h, tt, merged) + c4 * 4);
    t.v[i] = v;
  }
}

__device__ inline void put_tile(float *tile, const TileRegs &t) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = threadIdx.x + i * 256;
    const int row = idx >> 4, c4 = idx & 15;
    *reinterpret_cast<f4 *>(tile + row * LDP + c4 * 4) = t.v[i];
  }
}

// Loads 32 consecutive head-dim values (dims 32*hh .. +31) of row t into regs.
__device__ inline void load_row_half(float (&reg)[32], const float *src, bool valid) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (valid) v = *reinterpret_cast<const f4 *>(src + i * 4);
    reg[4 * i] = v.x; reg[4 * i + 1] = v.y; reg[4 * i + 2] = v.z; reg[4 * i + 3] = v.w;
  }
}

// Stores a wave's 32x64 result, held transposed in MFMA accumulators
// (acc[dt][v] = X[row r][dim 32dt + key_of(v,h)]), scaled by `mul`: lane
// (r, h) holds 4 consecutive dims of row r for each (dt, v/4), so it writes
// them as one float4 (8 per lane; the two lane halves write adjacent 16-byte
// pieces of a row). Rows >= T are not stored.
__device__ inline void store_rows(const f16x (&acc)[2], float mul, float *dst_base,
                                  const Dims &d, uint32_t b, uint32_t h, int row, int merged,
                                  int hh) {
  if (row >= int(d.T)) return;
  float *dst = dst_base + row_off(d, b, h, uint32_t(row), merged) + 4 * hh;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f4 v = {acc[dt][4 * j] * mul, acc[dt][4 * j + 1] * mul, acc[dt][4 * j + 2] * mul,
                    acc[dt][4 * j + 3] * mul};
      *reinterpret_cast<f4 *>(dst + 32 * dt + 8 * j) = v;
    }
}

// Adds the accumulators of the half-1 wave of each row tile into the half-0
// wave's (waves rt and rt+2). Called by every wave (barriers); smem must be
// free and hold NACC * 16 * 64 floats per row tile.
template <int NACC>
__device__ inline void sum_halves(float *smem, f16x (&acc)[NACC], int lane, int rt, int half) {
  float *buf = smem + rt * NACC * 16 * 64;
  __syncthreads();
  if (half == 1) {
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
      for (int i = 0; i < 16; ++i) buf[(a * 16 + i) * 64 + lane] = acc[a][i];
  }
  __syncthreads();
  if (half == 0) {
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][i] += buf[(a * 16 + i) * 64 + lane];
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 3) void attn_fwd_kernel(const float *__restrict__ q,
                                                       const float *__restrict__ k,
                                                       const float *__restrict__ v,
                                                       float *__restrict__ o,
                                                       float *__restrict__ lse, Dims d,
                                                       float scale, int causal, int o_merged) {
  __shared__ __attribute__((aligned(16))) float smem[2 * KB * LDP];
  float *Ks = smem;
  float *Vs = smem + KB * LDP;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, hh = lane >> 5;
  const int rt = wave & 1, half = wave >> 1; // row tile; half of each key tile
  const uint32_t bh = blockIdx.x;
  const uint32_t b = bh / d.H, h = bh % d.H;
  const int q_block = int(gridDim.y - 1 - blockIdx.y) * BQ; // latest queries first
  const int q0 = q_block + rt * WQ;
  const int my_q = q0 + r;
  const bool active = q0 < int(d.T);

  float qreg[32];
  load_row_half(qreg, q + row_off(d, b, h, my_q < int(d.T) ? my_q : 0, 0) + 32 * hh,
                my_q < int(d.T));

  f16x oacc[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
  // the running max m_run is kept in base-2 units (scores times
  // scale*log2(e)), so every exponential is one hardware 2^x
  float m_run = -INFINITY, l_run = 0.f;
  const float scale2 = scale * kLog2e;

  const int q_end = min(int(d.T), q_block + BQ);
  const int k_end = causal ? q_end : int(d.T);
  const int nkb = (k_end + KB - 1) / KB;
  // K/V tile kb+1 is fetched into registers while tile kb is in use.
  TileRegs kpre, vpre;
  fetch_tile(kpre, k, d, b, h, 0, 0);
  fetch_tile(vpre, v, d, b, h, 0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * KB + half * WQ; // this wave's 32 keys of the tile
    __syncthreads(); // every wave is done with the previous tile
    put_tile(Ks, kpre);
    put_tile(Vs, vpre);
    __syncthreads();
    if (kb + 1 < nkb) {
      fetch_tile(kpre, k, d, b, h, (kb + 1) * KB, 0);
      fetch_tile(vpre, v, d, b, h, (kb + 1) * KB, 0);
    }
    if (!active || k0 >= int(d.T) || (causal && k0 > q0 + WQ - 1)) continue;
    const float *Kh = Ks + half * WQ * LDP, *Vh = Vs + half * WQ * LDP;
    f16x st;
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] = 0.f;
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      const f4 ka = *reinterpret_cast<const f4 *>(Kh + r * LDP + 32 * hh + 4 * s4);
#pragma unroll
      for (int j = 0; j < 4; ++j) st = mfma(ka[j], qreg[4 * s4 + j], st);
    }
    // scale, mask, online softmax (per query = r; keys spread over v and h);
    // only tiles on the causal diagonal or past the sequence end need the mask
    const bool masked = k0 + WQ > int(d.T) || (causal && k0 + WQ - 1 > q0);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = k0 + key_of(i, hh);
      float sv = st[i] * scale2;
      if (masked && (key >= int(d.T) || (causal && key > my_q))) sv = -INFINITY;
      st[i] = sv;
      mx = fmaxf(mx, sv);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = exp2_fast(st[i] - m_use);
      st[i] = p;
      ps += p;
    }
    ps += __shfl_xor(ps, 32, 64);
    const float alpha = exp2_fast(m_run - m_use);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
    // O^T += V^T . P^T ; step i -> key key_of(i, hh) of this wave's 32
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = key_of(i, hh);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) oacc[dt] = mfma(Vh[key * LDP + 32 * dt + r], st[i], oacc[dt]);
    }
  }
  // combine the two key halves of each query: half 1 hands (m, l, O) to half 0
  {
    float *buf = smem + rt * (2 * 16 * 64 + 2 * WQ);
    __syncthreads(); // every wave is done with Ks/Vs
    if (half == 1) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) buf[(dt * 16 + i) * 64 + lane] = oacc[dt][i];
      if (hh == 0) {
        buf[2 * 16 * 64 + r] = m_run;
        buf[2 * 16 * 64 + WQ + r] = l_run;
      }
    }
    __syncthreads();
    if (half == 0) {
      const float m1 = buf[2 * 16 * 64 + r], l1 = buf[2 * 16 * 64 + WQ + r];
      const float m = fmaxf(m_run, m1);
      const float mu = (m == -INFINITY) ? 0.f : m;
      const float a0 = exp2_fast(m_run - mu), a1 = exp2_fast(m1 - mu);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          oacc[dt][i] = oacc[dt][i] * a0 + buf[(dt * 16 + i) * 64 + lane] * a1;
      l_run = l_run * a0 + l1 * a1;
      m_run = m;
    }
  }
  // epilogue: O = O / l ; lse = m + log(l)
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  if (active && half == 0 && hh == 0 && my_q < int(d.T))
    lse[(size_t(b) * d.H + h) * d.T + my_q] = m_run * kLn2 + logf(l_run);
  if (active && half == 0) store_rows(oacc, inv_l, o, d, b, h, my_q, o_merged, hh);
}

// ---------------------------------------------------------------------------
// backward, part 1: dK, dV. Each wave owns 32 keys; query tiles stream
// through LDS. S = Q.K^T is computed with m = query, n = key, so a lane holds
// queries q(v,h) of key r: the A-operand layout of P^T / dS^T for
// dV = P^T.dO and dK = dS^T.Q.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void attn_bwd_kv_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dk, float *__restrict__ dv, Dims d,
    float scale, int causal, int o_merged, int dqkv_merged) {
  __shared__ __attribute__((aligned(16))) float smem[2 * KB * LDP + 2 * KB];
  float *Qs = smem;
  float *dOs = smem + KB * LDP;
  float *lse_s = smem + 2 * KB * LDP;
  float *delta_s = lse_s + KB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, hh = lane >> 5;
  const int rt = wave & 1, half = wave >> 1; // key tile; half of each query tile
  const uint32_t bh = blockIdx.x;
  const uint32_t b = bh / d.H, h = bh % d.H;
  const int k_block = int(blockIdx.y) * BQ; // earliest keys (most queries) first
  const int key0 = k_block + rt * WQ;
  const int my_key = key0 + r;
  const bool active = key0 < int(d.T);

  float kreg[32], vreg[32];
  const bool kvalid = my_key < int(d.T);
  const size_t koff = row_off(d, b, h, kvalid ? my_key : 0, 0) + 32 * hh;
  load_row_half(kreg, k + koff, kvalid);
  load_row_half(vreg, v + koff, kvalid);

  f16x acc[4]; // dk (dt 0, 1), dv (dt 0, 1)
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[a][i] = 0.f;

  const size_t lse_base = (size_t(b) * d.H + h) * d.T;
  const int q_start = causal ? (k_block / KB) * KB : 0;
  const float scale2 = scale * kLog2e;
  // Q/dO tile (and its lse, delta) qt0+KB is fetched while qt0 is in use.
  TileRegs qpre, dopre;
  float lse_pre = 0.f, delta_pre = 0.f;
  auto fetch_q = [&](int qt0) {
    fetch_tile(qpre, q, d, b, h, qt0, 0);
    fetch_tile(dopre, dout, d, b, h, qt0, o_merged);
    const int t = qt0 + int(threadIdx.x);
    if (threadIdx.x < KB && t < int(d.T)) {
      lse_pre = lse[lse_base + t];
      delta_pre = delta[lse_base + t];
    } else {
      lse_pre = delta_pre = 0.f;
    }
  };
  if (q_start < int(d.T)) fetch_q(q_start);
  for (int qt0 = q_start; qt0 < int(d.T); qt0 += KB) {
    __syncthreads(); // every wave is done with the previous tile
    put_tile(Qs, qpre);
    put_tile(dOs, dopre);
    if (threadIdx.x < KB) {
      lse_s[threadIdx.x] = lse_pre * kLog2e; // base-2 units
      delta_s[threadIdx.x] = delta_pre;
    }
    __syncthreads();
    if (qt0 + KB < int(d.T)) fetch_q(qt0 + KB);
    const int qh0 = qt0 + half * WQ; // this wave's 32 queries of the tile
    if (!active || qh0 >= int(d.T) || (causal && qh0 + WQ - 1 < key0)) continue;
    const float *Qh = Qs + half * WQ * LDP, *dOh = dOs + half * WQ * LDP;
    const float *lse_h = lse_s + half * WQ, *delta_h = delta_s + half * WQ;
    // S[q][key] for 32 queries x 32 keys
    f16x sp, dp;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sp[i] = 0.f;
      dp[i] = 0.f;
    }
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      const f4 qa = *reinterpret_cast<const f4 *>(Qh + r * LDP + 32 * hh + 4 * s4);
      const f4 da = *reinterpret_cast<const f4 *>(dOh + r * LDP + 32 * hh + 4 * s4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sp = mfma(qa[j], kreg[4 * s4 + j], sp);
        dp = mfma(da[j], vreg[4 * s4 + j], dp);
      }
    }
    // P = exp(S*scale - lse[q]) masked; dS = P * (dP - delta[q]); only
    // tiles on the causal diagonal or past the sequence end need the mask
    const bool masked = qh0 + WQ > int(d.T) || key0 + WQ > int(d.T) ||
                        (causal && key0 + WQ - 1 > qh0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ql = key_of(i, hh);
      const int qq = qh0 + ql;
      float p = exp2_fast(sp[i] * scale2 - lse_h[ql]);
      if (masked && (qq >= int(d.T) || my_key >= int(d.T) || (causal && my_key > qq))) p = 0.f;
      sp[i] = p;
      dp[i] = p * (dp[i] - delta_h[ql]);
    }
    // dV[key][dim] += P^T . dO ; dK[key][dim] += dS^T . Q
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ql = key_of(i, hh);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        acc[2 + dt] = mfma(sp[i], dOh[ql * LDP + 32 * dt + r], acc[2 + dt]);
        acc[dt] = mfma(dp[i], Qh[ql * LDP + 32 * dt + r], acc[dt]);
      }
    }
  }
  sum_halves<4>(smem, acc, lane, rt, half);
  if (!active || half != 0) return;
  // accumulators: D[m = key key_of(v,h)][n = dim r + 32dt] -> row-contiguous stores
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = key0 + key_of(i, hh);
      if (key < int(d.T)) {
        const size_t off = row_off(d, b, h, key, dqkv_merged) + 32 * dt + r;
        dk[off] = acc[dt][i] * scale;
        dv[off] = acc[2 + dt][i];
      }
    }
}

// ---------------------------------------------------------------------------
// backward, part 2: dQ. Each wave owns 32 queries; K/V tiles stream through
// LDS (as in the forward). dQ^T = K^T.dS^T uses dS^T straight from the
// S^T-layout registers as the B operand.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void attn_bwd_q_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ o, const float *__restrict__ dout, const float *__restrict__ lse,
    float *__restrict__ delta, float *__restrict__ dq, Dims d, float scale, int causal,
    int o_merged, int dqkv_merged) {
  __shared__ __attribute__((aligned(16))) float smem[2 * KB * LDP];
  float *Ks = smem;
  float *Vs = smem + KB * LDP;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, hh = lane >> 5;
  const int rt = wave & 1, half = wave >> 1; // query tile; half of each key tile
  const uint32_t bh = blockIdx.x;
  const uint32_t b = bh / d.H, h = bh % d.H;
  const int q_block = int(gridDim.y - 1 - blockIdx.y) * BQ; // latest queries first
  const int q0 = q_block + rt * WQ;
  const int my_q = q0 + r;
  const bool active = q0 < int(d.T);
  const bool qvalid = my_q < int(d.T);

  float qreg[32], doreg[32];
  load_row_half(qreg, q + row_off(d, b, h, qvalid ? my_q : 0, 0) + 32 * hh, qvalid);
  const size_t do_off = row_off(d, b, h, qvalid ? my_q : 0, o_merged) + 32 * hh;
  load_row_half(doreg, dout + do_off, qvalid);
  const size_t lse_base = (size_t(b) * d.H + h) * d.T;
  const float my_lse2 = qvalid ? lse[lse_base + my_q] * kLog2e : 0.f; // base-2 units
  const float scale2 = scale * kLog2e;
  // delta = dO . O for this query (the two lane halves hold 32 dims each);
  // stored for the dK/dV kernel, which runs next
  float my_delta = 0.f;
  {
    float oreg[32];
    load_row_half(oreg, o + do_off, qvalid);
#pragma unroll
    for (int i = 0; i < 32; ++i) my_delta += oreg[i] * doreg[i];
    my_delta += __shfl_xor(my_delta, 32, 64);
    if (qvalid && half == 0 && hh == 0) delta[lse_base + my_q] = my_delta;
  }

  f16x dq_acc[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) dq_acc[dt][i] = 0.f;

  const int q_end = min(int(d.T), q_block + BQ);
  const int k_end = causal ? q_end : int(d.T);
  const int nkb = (k_end + KB - 1) / KB;
  TileRegs kpre, vpre;
  fetch_tile(kpre, k, d, b, h, 0, 0);
  fetch_tile(vpre, v, d, b, h, 0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * KB + half * WQ; // this wave's 32 keys of the tile
    __syncthreads(); // every wave is done with the previous tile
    put_tile(Ks, kpre);
    put_tile(Vs, vpre);
    __syncthreads();
    if (kb + 1 < nkb) {
      fetch_tile(kpre, k, d, b, h, (kb + 1) * KB, 0);
      fetch_tile(vpre, v, d, b, h, (kb + 1) * KB, 0);
    }
    if (!active || k0 >= int(d.T) || (causal && k0 > q0 + WQ - 1)) continue;
    const float *Kh = Ks + half * WQ * LDP, *Vh = Vs + half * WQ * LDP;
    f16x st, dpt;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      st[i] = 0.f;
      dpt[i] = 0.f;
    }
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      const f4 ka = *reinterpret_cast<const f4 *>(Kh + r * LDP + 32 * hh + 4 * s4);
      const f4 va = *reinterpret_cast<const f4 *>(Vh + r * LDP + 32 * hh + 4 * s4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        st = mfma(ka[j], qreg[4 * s4 + j], st);
        dpt = mfma(va[j], doreg[4 * s4 + j], dpt);
      }
    }
    const bool masked = k0 + WQ > int(d.T) || (causal && k0 + WQ - 1 > q0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = k0 + key_of(i, hh);
      float p = exp2_fast(st[i] * scale2 - my_lse2);
      if (!qvalid || (masked && (key >= int(d.T) || (causal && key > my_q)))) p = 0.f;
      dpt[i] = p * (dpt[i] - my_delta);
    }
    // dQ^T[dim][q] += K^T[dim][key] . dS^T[key][q]
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = key_of(i, hh);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
        dq_acc[dt] = mfma(Kh[key * LDP + 32 * dt + r], dpt[i], dq_acc[dt]);
    }
  }
  sum_halves<2>(smem, dq_acc, lane, rt, half);
  if (active && half == 0) store_rows(dq_acc, scale, dq, d, b, h, my_q, dqkv_merged, hh);
}

// ---- single-query decode ----------------------------------------------------
// The query of position t attends to keys 0..t of the K/V planes
// ([heads][t_stride][64], the forward's head layout at batch 1): o[h*64 + d].
// Block per head, 256 threads: one key per thread for the scores (kept in
// LDS), block max and sum, then o = sum_j p_j v_j / l with the threads as 16
// key groups x 16 float4 columns (coalesced rows of V, 8 loads in flight per
// thread), the groups added in a fixed order.
constexpr uint32_t kDecodeMaxT = 8192;

__global__ __launch_bounds__(256) void attn_decode_kernel(const float *__restrict__ q,
                                                          const float *__restrict__ k,
                                                          const float *__restrict__ v,
                                                          float *__restrict__ o,
                                                          uint32_t t_stride, uint32_t t,
                                                          float scale) {
  extern __shared__ float sm[];
  float *score = sm;                           // t + 1 scores
  f4 *part = reinterpret_cast<f4 *>(sm + ((t + 1 + 3) & ~3u)); // [16][16] partial sums
  float *red = reinterpret_cast<float *>(part + 16 * 16);        // reduction scratch
  const size_t plane = size_t(blockIdx.x) * t_stride * HD;
  const f4 *qh = reinterpret_cast<const f4 *>(q + plane + size_t(t) * HD);
  const float *kh = k + plane, *vh = v + plane;
  f4 qr[HD / 4];
#pragma unroll
  for (int i = 0; i < HD / 4; ++i) qr[i] = qh[i];
  float mx = -INFINITY;
  for (uint32_t j = threadIdx.x; j <= t; j += blockDim.x) {
    const f4 *kj = reinterpret_cast<const f4 *>(kh + size_t(j) * HD);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
      const f4 kv = kj[i];
      acc += qr[i].x * kv.x + qr[i].y * kv.y + qr[i].z * kv.z + qr[i].w * kv.w;
    }
    const float sc = acc * scale;
    score[j] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = block_max(mx, red);
  float sum = 0.f;
  for (uint32_t j = threadIdx.x; j <= t; j += blockDim.x) {
    const float pj = expf(score[j] - mx);
    score[j] = pj;
    sum += pj;
  }
  const float l = block_sum(sum, red);
  __syncthreads(); // every p_j is in LDS
  const int qd = int(threadIdx.x) & 15, grp = int(threadIdx.x) >> 4;
  const f4 *v4 = reinterpret_cast<const f4 *>(vh) + qd;
  f4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};
  for (uint32_t j0 = uint32_t(grp); j0 <= t; j0 += 128) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t j = j0 + 16u * u;
      if (j <= t) acc[u] += score[j] * v4[size_t(j) * (HD / 4)];
    }
  }
  f4 sum4 = acc[0];
#pragma unroll
  for (int u = 1; u < 8; ++u) sum4 += acc[u];
  part[grp * 16 + qd] = sum4;
  __syncthreads();
  if (grp == 0) {
    f4 r = part[qd];
    for (int g2 = 1; g2 < 16; ++g2) r += part[g2 * 16 + qd];
    reinterpret_cast<f4 *>(o + size_t(blockIdx.x) * HD)[qd] = r / l;
  }
}

} // namespace

TLH_API int tlh_attention_decode(const float *q, const float *k, const float *v, float *o,
                                 uint32_t heads, uint32_t t_stride, uint32_t t,
                                 uint32_t head_dim, float scale, void *stream) {
  if (head_dim != HD || t >= t_stride || t_stride > kDecodeMaxT) return int(hipErrorInvalidValue);
  if (heads == 0) return 0;
  const size_t lds = (((t + 1 + 3) & ~3u) + 16 * 16 * 4 + 4) * sizeof(float);
  attn_decode_kernel<<<heads, 256, lds, as_stream(stream)>>>(q, k, v, o, t_stride, t, scale);
  return launch_status();
}

TLH_API int tlh_attention_forward(const float *q, const float *k, const float *v, float *o,
                                  float *lse, uint32_t batch, uint32_t heads, uint32_t seq,
                                  uint32_t head_dim, float scale, int causal, int o_merged,
                                  void *stream) {
  if (head_dim != HD) return int(hipErrorInvalidValue);
  if (size_t(batch) * heads * seq == 0) return 0;
  if (ceil_div(seq, BQ) > 65535 || size_t(batch) * heads > 0x7fffffffu)
    return int(hipErrorInvalidValue);
  const Dims d{batch, heads, seq};
  dim3 grid(batch * heads, ceil_div(seq, BQ));
  attn_fwd_kernel<<<grid, 256, 0, as_stream(stream)>>>(q, k, v, o, lse, d, scale, causal,
                                                       o_merged);
  return launch_status();
}

TLH_API int tlh_attention_backward(const float *q, const float *k, const float *v,
                                   const float *o, const float *do_, const float *lse,
                                   float *delta, float *dq, float *dk, float *dv,
                                   uint32_t batch, uint32_t heads, uint32_t seq,
                                   uint32_t head_dim, float scale, int causal, int o_merged,
                                   int dqkv_merged, void *stream) {
  if (head_dim != HD) return int(hipErrorInvalidValue);
  if (size_t(batch) * heads * seq == 0) return 0;
  if (ceil_div(seq, BQ) > 65535 || size_t(batch) * heads > 0x7fffffffu)
    return int(hipErrorInvalidValue);
  hipStream_t s = as_stream(stream);
  const Dims d{batch, heads, seq};
  // dQ first: it also computes delta = rowsum(dO * O), which dK/dV need
  dim3 grid(batch * heads, ceil_div(seq, BQ));
  attn_bwd_q_kernel<<<grid, 256, 0, s>>>(q, k, v, o, do_, lse, delta, dq, d, scale, causal,
                                         o_merged, dqkv_merged);
  int st = launch_status();
  if (st) return st;
  attn_bwd_kv_kernel<<<grid, 256, 0, s>>>(q, k, v, do_, lse, delta, dk, dv, d, scale, causal,
                                          o_merged, dqkv_merged);
  return launch_status();
}
