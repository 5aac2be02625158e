// Chunkwise mLSTM forward, two-pass algorithm (float32 arithmetic).
//
// Pass 1 (chunk_states_kernel) runs the inter-chunk recurrence
// (kernel_development/xlstm/mlstm_block/mlstm_chunkwise/vendored/torch/
// native/fw.py:98-143) and writes the state entering every chunk to the
// workspace; pass 2 (chunk_output_kernel) computes each chunk's outputs from
// that state (fw.py:193-245).  It supports every dtype and L in
// {16, 32, 64, 128}; it is the exact (float32) path used for float32 inputs,
// and the fallback for shapes the fused bf16-MFMA kernel does not cover.
//
// Workspace (float32): C_in [BNH][NC][DQK][DV], n_in [BNH][NC][DQK],
// m_in [BNH][NC] — the reference's C_states/n_states/m_states without the
// final entry (fw.py:337-339), which goes to c_last/n_last/m_last.
#include "chunkwise.h"
#include "mfma_bf16.h"

#include <type_traits>

namespace xl {

constexpr int CW_THREADS = 256;
constexpr int CW_TILE = 64;  // d and v tile of the states pass, v tile of the output pass
constexpr int CW_DTILE = 32; // contraction tile of the output pass

// ------------------------------------------------------------ states pass
template <typename TQ, typename TG, int L>
__global__ __launch_bounds__(CW_THREADS) void chunk_states_kernel(
    const TQ* __restrict__ k, const TQ* __restrict__ v, const TG* __restrict__ ig, const TG* __restrict__ fg,
    const float* __restrict__ c0, const float* __restrict__ n0, const float* __restrict__ m0,
    float* __restrict__ Cst, float* __restrict__ nst, float* __restrict__ mst, float* __restrict__ c_last,
    float* __restrict__ n_last, float* __restrict__ m_last, int NC, int DQK, int DV, int ndt, int nvt) {
  __shared__ float sK[L][CW_TILE + 1];
  __shared__ float sV[L][CW_TILE + 1];
  __shared__ float sb[L], si[L], salpha[L];
  __shared__ float s_amax;

  const int tid = threadIdx.x;
  const int ty = tid >> 4, tx = tid & 15;
  const int per_bh = ndt * nvt;
  const int bh = blockIdx.x / per_bh;
  const int rem = blockIdx.x - bh * per_bh;
  const int d0 = (rem / nvt) * CW_TILE, v0 = (rem % nvt) * CW_TILE;
  const bool owns_n = (v0 == 0), owns_m = (v0 == 0 && d0 == 0);
  const int S = NC * L;

  float C[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int d = d0 + 4 * ty + a, vv = v0 + 4 * tx + b;
      C[a][b] = (c0 && d < DQK && vv < DV) ? c0[((size_t)bh * DQK + d) * DV + vv] : 0.f;
    }
  float nn = 0.f;
  if (owns_n && tid < CW_TILE && d0 + tid < DQK && n0) nn = n0[(size_t)bh * DQK + d0 + tid];
  float m = m0 ? m0[bh] : 0.f;

  for (int kc = 0; kc < NC; ++kc) {
    // state entering chunk kc
    const size_t sidx = (size_t)bh * NC + kc;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int d = d0 + 4 * ty + a, vv = v0 + 4 * tx + b;
        if (d < DQK && vv < DV) Cst[(sidx * DQK + d) * DV + vv] = C[a][b];
      }
    if (owns_n && tid < CW_TILE && d0 + tid < DQK) nst[sidx * DQK + d0 + tid] = nn;
    if (owns_m && tid == 0) mst[sidx] = m;

    const size_t g0 = (size_t)bh * S + (size_t)kc * L;
    chunk_gate_prefix<TG, L>(ig, fg, g0, sb, si);
    const float g = sb[L - 1];
    if (tid < 64) {  // max_t a_t, a_t = b_L - b_t + i_t (fw.py:98,100)
      float am = -INFINITY;
      for (int t = tid; t < L; t += 64) am = fmaxf(am, g - sb[t] + si[t]);
      am = wave_max(am);
      if (tid == 0) s_amax = am;
    }
    // K, V tiles of this chunk
    for (int e = tid; e < L * CW_TILE; e += CW_THREADS) {
      const int t = e / CW_TILE, c = e - t * CW_TILE;
      const size_t row = (size_t)bh * S + (size_t)kc * L + t;
      sK[t][c] = (d0 + c < DQK) ? to_f32(k[row * DQK + d0 + c]) : 0.f;
      sV[t][c] = (v0 + c < DV) ? to_f32(v[row * DV + v0 + c]) : 0.f;
    }
    __syncthreads();
    const float m_next = fmaxf(g + m, s_amax);           // fw.py:115
    if (tid < L) salpha[tid] = expf(g - sb[tid] + si[tid] - m_next);  // fw.py:121
    const float gbar = expf(g + m - m_next);             // fw.py:125
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) C[a][b] *= gbar;
    for (int t = 0; t < L; ++t) {  // C += Kbar^T V (fw.py:128-130)
      const float al = salpha[t];
      float kd[4], vv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) kd[a] = sK[t][4 * ty + a] * al;
#pragma unroll
      for (int b = 0; b < 4; ++b) vv[b] = sV[t][4 * tx + b];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) C[a][b] += kd[a] * vv[b];
    }
    if (owns_n && tid < CW_TILE) {  // n += sum_t Kbar (fw.py:133)
      float s = 0.f;
      for (int t = 0; t < L; ++t) s += sK[t][tid] * salpha[t];
      nn = gbar * nn + s;
    }
    m = m_next;
    __syncthreads();  // LDS reused by the next chunk
  }
  if (c_last) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int d = d0 + 4 * ty + a, vv = v0 + 4 * tx + b;
        if (d < DQK && vv < DV) c_last[((size_t)bh * DQK + d) * DV + vv] = C[a][b];
      }
    if (owns_n && tid < CW_TILE && d0 + tid < DQK) n_last[(size_t)bh * DQK + d0 + tid] = nn;
    if (owns_m && tid == 0) m_last[bh] = m;
  }
}

// ------------------------------------------------------------ output pass
template <int L>
struct OutSmem {
  // region A (contraction tiles) is reused for V after the contraction
  static constexpr int QT = 0;                          // [32][L]  Q^T tile
  static constexpr int KT = QT + CW_DTILE * L;          // [32][L]  K^T tile
  static constexpr int CT = KT + CW_DTILE * L;          // [32][64] C tile
  static constexpr int NT = CT + CW_DTILE * CW_TILE;    // [32]     n tile
  static constexpr int A_END = NT + CW_DTILE;
  static constexpr int V = 0;                           // [L][64]  V chunk (after contraction)
  static constexpr int A_SIZE = (A_END > L * CW_TILE) ? A_END : L * CW_TILE;
  static constexpr int MT = A_SIZE;                     // [L][L]   M^T (M^T[j][i])
  static constexpr int GB = MT + L * L;                 // b
  static constexpr int GI = GB + L;                     // i
  static constexpr int GM = GI + L;                     // m_comb
  static constexpr int GQ = GM + L;                     // qbar (includes qk_scale)
  static constexpr int GD = GQ + L;                     // max(|den|, exp(-m)) + eps
  static constexpr int TOTAL = GD + L;
  static constexpr size_t BYTES = (size_t)TOTAL * sizeof(float);
};

template <typename TQ, typename TG, int L>
__global__ __launch_bounds__(CW_THREADS) void chunk_output_kernel(
    const TQ* __restrict__ q, const TQ* __restrict__ k, const TQ* __restrict__ v, const TG* __restrict__ ig,
    const TG* __restrict__ fg, const float* __restrict__ Cst, const float* __restrict__ nst,
    const float* __restrict__ mst, TQ* __restrict__ h, int NC, int DQK, int DV, int nvt, float qk_scale,
    float eps) {
  constexpr int RS = L / 16;  // S rows/cols and H rows per thread
  using SM = OutSmem<L>;
  extern __shared__ float smem[];
  float* sQt = smem + SM::QT;
  float* sKt = smem + SM::KT;
  float* sC = smem + SM::CT;
  float* sn = smem + SM::NT;
  float* sV = smem + SM::V;
  float* sMt = smem + SM::MT;
  float* sb = smem + SM::GB;
  float* si = smem + SM::GI;
  float* smc = smem + SM::GM;
  float* sqb = smem + SM::GQ;
  float* sden = smem + SM::GD;

  const int tid = threadIdx.x;
  const int ty = tid >> 4, tx = tid & 15;
  const int per_bh = NC * nvt;
  const int bh = blockIdx.x / per_bh;
  const int rem = blockIdx.x - bh * per_bh;
  const int kc = rem / nvt;
  const int v0 = (rem - kc * nvt) * CW_TILE;
  const int S = NC * L;
  const size_t row0 = (size_t)bh * S + (size_t)kc * L;  // first token of the chunk
  const size_t sidx = (size_t)bh * NC + kc;

  chunk_gate_prefix<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {  // fw.py:204-217, 230
    const int i = tid;
    const float mprev = mst[sidx];
    float mi = -INFINITY;
    for (int j = 0; j <= i; ++j) mi = fmaxf(mi, sb[i] - sb[j] + si[j]);
    const float mb = sb[i] + mprev;
    const float mc = fmaxf(mb, mi);
    smc[i] = mc;
    sqb[i] = expf(mb - mc) * qk_scale;
  }

  float accS[RS][RS], accH[RS][4];
#pragma unroll
  for (int a = 0; a < RS; ++a) {
#pragma unroll
    for (int b = 0; b < RS; ++b) accS[a][b] = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) accH[a][c] = 0.f;
  }
  float qn = 0.f;

  for (int dd = 0; dd < DQK; dd += CW_DTILE) {
    __syncthreads();  // previous tile consumed
    for (int e = tid; e < L * CW_DTILE; e += CW_THREADS) {
      const int t = e / CW_DTILE, c = e - t * CW_DTILE;
      const bool ok = dd + c < DQK;
      sQt[c * L + t] = ok ? to_f32(q[(row0 + t) * DQK + dd + c]) : 0.f;
      sKt[c * L + t] = ok ? to_f32(k[(row0 + t) * DQK + dd + c]) : 0.f;
    }
    for (int e = tid; e < CW_DTILE * CW_TILE; e += CW_THREADS) {
      const int r = e / CW_TILE, c = e - r * CW_TILE;
      sC[r * CW_TILE + c] = (dd + r < DQK && v0 + c < DV) ? Cst[(sidx * DQK + dd + r) * DV + v0 + c] : 0.f;
    }
    if (tid < CW_DTILE) sn[tid] = (dd + tid < DQK) ? nst[sidx * DQK + dd + tid] : 0.f;
    __syncthreads();
#pragma unroll 4
    for (int d = 0; d < CW_DTILE; ++d) {
      float qv[RS], kv[RS], cv[4];
#pragma unroll
      for (int a = 0; a < RS; ++a) qv[a] = sQt[d * L + ty * RS + a];
#pragma unroll
      for (int b = 0; b < RS; ++b) kv[b] = sKt[d * L + tx * RS + b];
#pragma unroll
      for (int c = 0; c < 4; ++c) cv[c] = sC[d * CW_TILE + tx * 4 + c];
#pragma unroll
      for (int a = 0; a < RS; ++a) {
#pragma unroll
        for (int b = 0; b < RS; ++b) accS[a][b] += qv[a] * kv[b];
#pragma unroll
        for (int c = 0; c < 4; ++c) accH[a][c] += qv[a] * cv[c];
      }
    }
    if (tid < L) {
      for (int d = 0; d < CW_DTILE; ++d) qn += sQt[d * L + tid] * sn[d];
    }
  }
  __syncthreads();  // contraction tiles dead; region A becomes V

  // M = (Q K^T s) exp(b_i - b_j + i_j - m_i) on j <= i (fw.py:204-227), stored transposed
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const int i = ty * RS + a;
    const float bi = sb[i], mci = smc[i];
#pragma unroll
    for (int b = 0; b < RS; ++b) {
      const int j = tx * RS + b;
      sMt[j * L + i] = (j <= i) ? accS[a][b] * qk_scale * expf(bi - sb[j] + si[j] - mci) : 0.f;
    }
  }
  for (int e = tid; e < L * CW_TILE; e += CW_THREADS) {
    const int t = e / CW_TILE, c = e - t * CW_TILE;
    sV[t * CW_TILE + c] = (v0 + c < DV) ? to_f32(v[(row0 + t) * DV + v0 + c]) : 0.f;
  }
  __syncthreads();
  if (tid < L) {  // den = qbar (q.n) + sum_j M_ij (fw.py:237-243)
    float rs = 0.f;
    for (int j = 0; j < L; ++j) rs += sMt[j * L + tid];
    const float den = sqb[tid] * qn + rs;
    sden[tid] = fmaxf(fabsf(den), expf(-smc[tid])) + eps;
  }
  // H = qbar (Q C) + M V (fw.py:233-235)
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const float qb = sqb[ty * RS + a];
#pragma unroll
    for (int c = 0; c < 4; ++c) accH[a][c] *= qb;
  }
  for (int j = 0; j < L; ++j) {
    float mv[RS], vv[4];
#pragma unroll
    for (int a = 0; a < RS; ++a) mv[a] = sMt[j * L + ty * RS + a];
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = sV[j * CW_TILE + tx * 4 + c];
#pragma unroll
    for (int a = 0; a < RS; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) accH[a][c] += mv[a] * vv[c];
  }
  __syncthreads();  // sden ready
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const int i = ty * RS + a;
    const float inv = 1.0f / sden[i];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int vv = v0 + tx * 4 + c;
      if (vv < DV) h[(row0 + i) * DV + vv] = from_f32<TQ>(accH[a][c] * inv);
    }
  }
}

// ------------------------------- output pass, float32 on the bf16 matrix cores
// chunk_output_kernel for 64-token chunks and whole 64-wide tiles, on v_mfma_f32_16x16x32_bf16
// in the three-product form (q/k/v of any dtype, read as float32): every operand x is split into
// hi = bf16(x), lo = bf16(x - hi), and a product a b is taken as a_hi b_hi + a_hi b_lo + a_lo b_hi
// (the a_lo b_lo term and the splits leave about 2^-16 of |a b|), accumulated in float32.  One
// workgroup of 4 waves per (head, chunk, 64 columns of DV); wave w owns the tokens
// i in [16 w, 16 w + 16).  Over DQK in blocks of 64, 32 d per MFMA, lane (g, r) at
// d = 8 g .. 8 g + 7 of the step, holding its Q row 16 w + r split in registers:
//   S^T[j][i] += K[j][d] Q[i][d]   (A = K rows hi / lo from LDS, B = Q)
//   Hc[i][v]  += Q[i][d] C[d][v]   (A = Q, B = the C block hi / lo by transposed reads)
//   q.n       += n[d] Q[i][d]      (A rows 0, 1 = n hi, lo, so D[0][i] + D[1][i] = q . n)
// then M[i][j] = S s exp(b_i - b_j + i_j - m_i) on j <= i into LDS as hi / lo rows, the divisor
// max(|qbar q.n + sum_j M_ij|, exp(-m_i)) + eps, and H = (qbar Hc + M V) / divisor (A = M rows,
// B = V by transposed reads) (fw.py:193-245).
constexpr int OX_P = 80;  // bf16 per staged 64-wide row (160 bytes)

// 4 consecutive values as float32
__device__ __forceinline__ mfma::f32x4 ld4f(const float* p) { return *reinterpret_cast<const mfma::f32x4*>(p); }
template <typename T>
__device__ __forceinline__ mfma::f32x4 ld4f(const T* p) {
  const mfma::u32x2 w = *reinterpret_cast<const mfma::u32x2*>(p);
  const T* e = reinterpret_cast<const T*>(&w);
  return mfma::f32x4{to_f32(e[0]), to_f32(e[1]), to_f32(e[2]), to_f32(e[3])};
}

template <typename TQ, typename TG, int NRT>
__global__ __launch_bounds__(256) void chunk_output_x3_kernel(
    const TQ* __restrict__ q, const TQ* __restrict__ k, const TQ* __restrict__ v,
    const TG* __restrict__ ig, const TG* __restrict__ fg, const float* __restrict__ Cst,
    const float* __restrict__ nst, const float* __restrict__ mst, TQ* __restrict__ h, int NC, int DV, int nvt,
    float qk_scale, float eps) {
  using namespace xl::mfma;
  constexpr int L = 64, DQK = 64 * NRT;
  // K block [t][d], then M rows [i][j]; the C block [d][v], then V [j][v]; bf16 hi / lo each
  __shared__ __attribute__((aligned(16))) uint32_t sAh[L * OX_P / 2], sAl[L * OX_P / 2];
  __shared__ __attribute__((aligned(16))) uint32_t sBh[L * OX_P / 2], sBl[L * OX_P / 2];
  __shared__ float sn[64], sb[L], si[L], smc[L], sqb[L], sden[L];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int kk = r >> 2, ka = r & 3;  // transposed reads: row r / 4 of a 4-row block, columns 4 (r % 4)
  const int per_bh = NC * nvt;
  const int blk = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bh = blk / per_bh, rem = blk - bh * per_bh;
  const int kc = rem / nvt, v0 = (rem - kc * nvt) * 64;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  const float* cblk = Cst + sidx * DQK * DV + v0;  // C entering the chunk, columns v0 ..
  // one DQK block in registers: this lane's Q row pieces (d = 32 ks + 8 g + 4 h), K rows and C
  // rows (row p / 16, 4 values at 4 (p % 16)), n; then the V chunk
  f32x4 pq[4], pk[4], pc[4], pv[4];
  float pn = 0.f;
  auto fetch = [&](int db) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      pq[u] = ld4f(q + (row0 + 16 * w + r) * DQK + db + 32 * (u >> 1) + 8 * g + 4 * (u & 1));
      const int p = u * 256 + tid;
      pk[u] = ld4f(k + (row0 + (p >> 4)) * DQK + db + (p & 15) * 4);
      pc[u] = *reinterpret_cast<const f32x4*>(cblk + (size_t)(db + (p >> 4)) * DV + (p & 15) * 4);
    }
    if (tid < 64) pn = nst[sidx * DQK + db + tid];
  };
  auto fetch_v = [&]() {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = u * 256 + tid;
      pv[u] = ld4f(v + (row0 + (p >> 4)) * DV + v0 + (p & 15) * 4);
    }
  };
  // 4 floats of row p / 16, columns 4 (p % 16), as bf16 hi / lo into a pair of staged tiles
  auto stage4 = [&](uint32_t* dh, uint32_t* dl, int p, f32x4 x) {
    const int o = ((p >> 4) * OX_P + (p & 15) * 4) >> 1;
    const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
    *reinterpret_cast<u32x2*>(dh + o) = u32x2{h0, h1};
    *reinterpret_cast<u32x2*>(dl + o) = u32x2{pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1))};
  };
  fetch(0);
  chunk_gate_prefix<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {  // fw.py:204-217, 230
    const float mprev = mst[sidx];
    float mi = -INFINITY;
    for (int j = 0; j <= tid; ++j) mi = fmaxf(mi, sb[tid] - sb[j] + si[j]);
    const float mb = sb[tid] + mprev;
    const float mc = fmaxf(mb, mi);
    smc[tid] = mc;
    sqb[tid] = expf(mb - mc) * qk_scale;
  }
  f32x4 accS[4], accH[4], accN = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    accS[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    accH[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const u32x4 z4 = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int db = 0; db < DQK; db += 64) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      stage4(sAh, sAl, u * 256 + tid, pk[u]);
      stage4(sBh, sBl, u * 256 + tid, pc[u]);
    }
    if (tid < 64) sn[tid] = pn;
    bfx8 qh[2], ql[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const float x[8] = {pq[2 * ks][0], pq[2 * ks][1], pq[2 * ks][2], pq[2 * ks][3],
                          pq[2 * ks + 1][0], pq[2 * ks + 1][1], pq[2 * ks + 1][2], pq[2 * ks + 1][3]};
      u32x4 hh, ll;
      split_bf(x, hh, ll);
      qh[ks] = __builtin_bit_cast(bfx8, hh);
      ql[ks] = __builtin_bit_cast(bfx8, ll);
    }
    __syncthreads();
    if (db + 64 < DQK) fetch(db + 64);
    else fetch_v();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = 32 * ks + 8 * g;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int o = ((16 * jt + r) * OX_P + c) >> 1;
        const bfx8 kh = ld_bf8(sAh + o), kl = ld_bf8(sAl + o);
        accS[jt] = mfma_bf(kh, qh[ks], accS[jt]);
        accS[jt] = mfma_bf(kh, ql[ks], accS[jt]);
        accS[jt] = mfma_bf(kl, qh[ks], accS[jt]);
      }
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int o1 = ((c + kk) * OX_P + 16 * ct + 4 * ka) >> 1, o2 = o1 + 2 * OX_P;
        const bfx8 ch = tr_pair(sBh + o1, sBh + o2), cl = tr_pair(sBl + o1, sBl + o2);
        accH[ct] = mfma_bf(qh[ks], ch, accH[ct]);
        accH[ct] = mfma_bf(qh[ks], cl, accH[ct]);
        accH[ct] = mfma_bf(ql[ks], ch, accH[ct]);
      }
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = sn[c + e];
      u32x4 nh, nl;
      split_bf(x, nh, nl);
      const bfx8 an = __builtin_bit_cast(bfx8, r == 0 ? nh : (r == 1 ? nl : z4));
      accN = mfma_bf(an, qh[ks], accN);
      accN = mfma_bf(an, ql[ks], accN);
    }
    __syncthreads();  // the blocks are read; the next staging may overwrite them
  }
  // lane (g, r), element e of tile jt: S[i = 16 w + r][j = 16 jt + 4 g + e]
  const int i = 16 * w + r;
  float rs = 0.f;
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    float mm[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 16 * jt + 4 * g + e;
      mm[e] = (j <= i) ? accS[jt][e] * qk_scale * expf(sb[i] - sb[j] + si[j] - smc[i]) : 0.f;  // fw.py:219-227
      rs += mm[e];
    }
    const uint32_t h0 = pk_bf(mm[0], mm[1]), h1 = pk_bf(mm[2], mm[3]);
    const int o = (i * OX_P + 16 * jt + 4 * g) >> 1;
    *reinterpret_cast<u32x2*>(sAh + o) = u32x2{h0, h1};
    *reinterpret_cast<u32x2*>(sAl + o) =
        u32x2{pk_bf(mm[0] - bf_l(h0), mm[1] - bf_h(h0)), pk_bf(mm[2] - bf_l(h1), mm[3] - bf_h(h1))};
  }
  rs += __shfl_xor(rs, 16, 64);
  rs += __shfl_xor(rs, 32, 64);
  if (g == 0) {  // den = qbar (q . n) + sum_j M_ij; divisor max(|den|, exp(-m)) + eps (fw.py:237-245)
    const float den = sqb[i] * (accN[0] + accN[1]) + rs;
    sden[i] = fmaxf(fabsf(den), expf(-smc[i])) + eps;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) stage4(sBh, sBl, u * 256 + tid, pv[u]);
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int e = 0; e < 4; ++e) accH[ct][e] *= sqb[16 * w + 4 * g + e];
  __syncthreads();
  // H += M V (fw.py:233-235)
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int c = 32 * ks + 8 * g;
    const int om = (i * OX_P + c) >> 1;
    const bfx8 mh = ld_bf8(sAh + om), ml = ld_bf8(sAl + om);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int o1 = ((c + kk) * OX_P + 16 * ct + 4 * ka) >> 1, o2 = o1 + 2 * OX_P;
      const bfx8 vh = tr_pair(sBh + o1, sBh + o2), vl = tr_pair(sBl + o1, sBl + o2);
      accH[ct] = mfma_bf(mh, vh, accH[ct]);
      accH[ct] = mfma_bf(mh, vl, accH[ct]);
      accH[ct] = mfma_bf(ml, vh, accH[ct]);
    }
  }
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int it = 16 * w + 4 * g + e;
      h[(row0 + it) * DV + v0 + 16 * ct + r] = from_f32<TQ>(accH[ct][e] / sden[it]);
    }
}

// ---------------------------------------------------------------- launchers
template <typename TQ, typename TG, int L>
static int two_pass_t(const ChunkwiseArgs& A) {
  const int NC = A.S / L;
  const int BNH = A.B * A.NH;
  const int ndt = (A.DQK + CW_TILE - 1) / CW_TILE;
  const int nvt = (A.DV + CW_TILE - 1) / CW_TILE;
  float* ws = (float*)A.workspace;
  float* Cst = ws;
  float* nst = Cst + (size_t)BNH * NC * A.DQK * A.DV;
  float* mst = nst + (size_t)BNH * NC * A.DQK;
  hipStream_t s = (hipStream_t)A.stream;

  // 64-token chunks, whole 64-wide tiles: both passes on the matrix cores
  if constexpr (L == 64) {
    const int rc = chunkwise_states_mfma(A, Cst, nst, mst, mst + (size_t)BNH * NC);
    if (rc < 0) return rc;  // a launch error (1: the tiles do not fit, the FMA kernels below)
    if (rc == 0) {
      const dim3 grid((unsigned)(BNH * NC * nvt));
      const TQ *q = (const TQ*)A.q, *k = (const TQ*)A.k, *v = (const TQ*)A.v;
      const TG *ig = (const TG*)A.i, *fg = (const TG*)A.f;
      switch (A.DQK) {
        case 64: hipLaunchKernelGGL((chunk_output_x3_kernel<TQ, TG, 1>), grid, dim3(256), 0, s, q, k, v, ig, fg, Cst, nst, mst, (TQ*)A.h, NC, A.DV, nvt, A.qk_scale, A.eps); break;
        case 128: hipLaunchKernelGGL((chunk_output_x3_kernel<TQ, TG, 2>), grid, dim3(256), 0, s, q, k, v, ig, fg, Cst, nst, mst, (TQ*)A.h, NC, A.DV, nvt, A.qk_scale, A.eps); break;
        default: hipLaunchKernelGGL((chunk_output_x3_kernel<TQ, TG, 4>), grid, dim3(256), 0, s, q, k, v, ig, fg, Cst, nst, mst, (TQ*)A.h, NC, A.DV, nvt, A.qk_scale, A.eps); break;
      }
      return check_launch("xl_mlstm_chunkwise_fwd(output pass)");
    }
  }
  hipLaunchKernelGGL((chunk_states_kernel<TQ, TG, L>), dim3((unsigned)(BNH * ndt * nvt)), dim3(CW_THREADS), 0, s,
                     (const TQ*)A.k, (const TQ*)A.v, (const TG*)A.i, (const TG*)A.f, A.c0, A.n0, A.m0, Cst, nst, mst,
                     A.c_last, A.n_last, A.m_last, NC, A.DQK, A.DV, ndt, nvt);
  int rc = check_launch("xl_mlstm_chunkwise_fwd(states pass)");
  if (rc) return rc;
  auto kout = chunk_output_kernel<TQ, TG, L>;
  const size_t smem = OutSmem<L>::BYTES;
  if (smem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)kout, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess)
      return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd: LDS attribute failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(kout, dim3((unsigned)(BNH * NC * nvt)), dim3(CW_THREADS), smem, s, (const TQ*)A.q,
                     (const TQ*)A.k, (const TQ*)A.v, (const TG*)A.i, (const TG*)A.f, Cst, nst, mst, (TQ*)A.h, NC,
                     A.DQK, A.DV, nvt, A.qk_scale, A.eps);
  return check_launch("xl_mlstm_chunkwise_fwd(output pass)");
}

template <typename TQ, typename TG>
static int two_pass_l(const ChunkwiseArgs& A) {
  switch (A.L) {
    case 16: return two_pass_t<TQ, TG, 16>(A);
    case 32: return two_pass_t<TQ, TG, 32>(A);
    case 64: return two_pass_t<TQ, TG, 64>(A);
    default: return two_pass_t<TQ, TG, 128>(A);
  }
}

template <typename TQ>
static int two_pass_g(const ChunkwiseArgs& A) {
  switch (A.dtype_gates) {
    case XL_DTYPE_F32: return two_pass_l<TQ, float>(A);
    case XL_DTYPE_BF16: return two_pass_l<TQ, bf16_t>(A);
    default: return two_pass_l<TQ, f16_t>(A);
  }
}

template <typename TQ, typename TG>
static int states_pass_l(const ChunkwiseArgs& A, float* Cst, float* nst, float* mst, float* c_fin, float* n_fin,
                         float* m_fin) {
  const int BNH = A.B * A.NH;
  const int ndt = (A.DQK + CW_TILE - 1) / CW_TILE;
  const int nvt = (A.DV + CW_TILE - 1) / CW_TILE;
  const dim3 grid((unsigned)(BNH * ndt * nvt)), blk(CW_THREADS);
  hipStream_t s = (hipStream_t)A.stream;
  const TQ *k = (const TQ*)A.k, *v = (const TQ*)A.v;
  const TG *ig = (const TG*)A.i, *fg = (const TG*)A.f;
  switch (A.L) {
    case 16: hipLaunchKernelGGL((chunk_states_kernel<TQ, TG, 16>), grid, blk, 0, s, k, v, ig, fg, A.c0, A.n0, A.m0, Cst, nst, mst, c_fin, n_fin, m_fin, A.S / 16, A.DQK, A.DV, ndt, nvt); break;
    case 32: hipLaunchKernelGGL((chunk_states_kernel<TQ, TG, 32>), grid, blk, 0, s, k, v, ig, fg, A.c0, A.n0, A.m0, Cst, nst, mst, c_fin, n_fin, m_fin, A.S / 32, A.DQK, A.DV, ndt, nvt); break;
    case 64: hipLaunchKernelGGL((chunk_states_kernel<TQ, TG, 64>), grid, blk, 0, s, k, v, ig, fg, A.c0, A.n0, A.m0, Cst, nst, mst, c_fin, n_fin, m_fin, A.S / 64, A.DQK, A.DV, ndt, nvt); break;
    default: hipLaunchKernelGGL((chunk_states_kernel<TQ, TG, 128>), grid, blk, 0, s, k, v, ig, fg, A.c0, A.n0, A.m0, Cst, nst, mst, c_fin, n_fin, m_fin, A.S / 128, A.DQK, A.DV, ndt, nvt); break;
  }
  return check_launch("chunkwise states pass");
}

template <typename TQ>
static int states_pass_g(const ChunkwiseArgs& A, float* Cst, float* nst, float* mst, float* c_fin, float* n_fin,
                         float* m_fin) {
  switch (A.dtype_gates) {
    case XL_DTYPE_F32: return states_pass_l<TQ, float>(A, Cst, nst, mst, c_fin, n_fin, m_fin);
    case XL_DTYPE_BF16: return states_pass_l<TQ, bf16_t>(A, Cst, nst, mst, c_fin, n_fin, m_fin);
    default: return states_pass_l<TQ, f16_t>(A, Cst, nst, mst, c_fin, n_fin, m_fin);
  }
}

int chunkwise_states_pass(const ChunkwiseArgs& A, float* Cst, float* nst, float* mst, float* c_fin, float* n_fin,
                          float* m_fin) {
  switch (A.dtype_qkv) {
    case XL_DTYPE_F32: return states_pass_g<float>(A, Cst, nst, mst, c_fin, n_fin, m_fin);
    case XL_DTYPE_BF16: return states_pass_g<bf16_t>(A, Cst, nst, mst, c_fin, n_fin, m_fin);
    default: return states_pass_g<f16_t>(A, Cst, nst, mst, c_fin, n_fin, m_fin);
  }
}

size_t chunkwise_two_pass_workspace(int B, int NH, int S, int DQK, int DV, int L) {
  const size_t NC = (size_t)(S / L);
  const size_t BNH = (size_t)B * NH;
  const size_t floats = BNH * NC * ((size_t)DQK * DV + DQK + 1 + kChunkGatePrefix);
  return (floats * sizeof(float) + 255) & ~(size_t)255;
}

int chunkwise_two_pass(const ChunkwiseArgs& A) {
  switch (A.dtype_qkv) {
    case XL_DTYPE_F32: return two_pass_g<float>(A);
    case XL_DTYPE_BF16: return two_pass_g<bf16_t>(A);
    default: return two_pass_g<f16_t>(A);
  }
}

}  // namespace xl
