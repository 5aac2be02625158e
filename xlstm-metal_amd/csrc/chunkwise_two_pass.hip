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
  const size_t floats = BNH * NC * ((size_t)DQK * DV + DQK + 1);
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
