// Chunkwise mLSTM backward (float32 accumulation): the reference's custom backward
// mlstm_chunkwise_bw (kernel_development/xlstm/mlstm_block/mlstm_chunkwise/
// vendored/torch/native/bw.py:198-352), which treats the per-token
// denominator max(|q n|, exp(-m)) + eps as a constant (the mLSTM layer's
// multi-head norm removes any per-row scale of h, so its gradient does not
// reach the loss there).  Five launches after the states pass (named here by
// their FMA forms; the bf16 and float32-MFMA forms further down do the same
// work per launch):
//
//   1. the states pass of the two-pass forward recomputes the state entering
//      every chunk (bw.py:242-258, recompute_states_in_bw);
//   2. bw_stats_kernel: per chunk, the combined stabiliser m_t and the divisor
//      max(|den_t|, exp(-m_t)) + eps of every token (the forward's vecM_out and
//      vecN_out + eps, fw.py:204-253);
//   3. bw_dC_kernel: the reverse recurrence dC_{k-1} = exp(g_k + m_{k-1} - m_k) dC_k
//      + Qbar_k^T (dH_k / (N_k + eps)) over the chunks, one workgroup per 64 x 64
//      tile of dC (bw.py:31-115);
//   4. bw_dv_kernel: dV = Sbar^T dH~ + (K * Abar) dC_k per chunk and 64-column tile
//      of V, and the per-token partial sums v . dV of dI (bw.py:159,182,338);
//   5. bw_dqk_kernel: dQ = (dS K) s + (dH~ * Bbar) (C_{k-1} s)^T and
//      dK = (dS^T Q) s + (V * Abar) dC_k^T per chunk and 64-column tile of DQK,
//      with dS = (dH~ V^T) * Dbar, and the per-token partial sums q . dQ - k . dK
//      (bw.py:161-185, 333);
//   6. bw_gates_kernel: dI = sum of the partials, dF = (reverse cumulative sum of
//      the q . dQ - k . dK partials) * sigmoid(-f) (bw.py:332-338).
//
// Workspace (float32, each region 256-byte aligned): the entering states C, n, m
// [BNH][NC](...), the final state, m_comb and the divisor [BNH][S], dC
// [BNH][NC + 1][DQK][DV] (index k: the gradient of the state after chunk k - 1;
// 0 is dC_initial), the dF partials [BNH][S][ceil(DQK/64)] and the dI partials
// [BNH][S][ceil(DV/64)].  On the path of the fused bf16 dV / dQ / dK pass the C and
// dC states are kept as their upper 24 bits (pack24 below), in the first three
// quarters of their regions.
#include "chunkwise.h"
#include "mfma_bf16.h"

#include <type_traits>

namespace xl {
namespace {
using namespace xl::mfma;  // bf16 MFMA building blocks (mfma_bf16.h)

constexpr int BW_THREADS = 256;
constexpr int BW_T = 64;   // DQK / DV tile
constexpr int BW_KT = 32;  // contraction tile

// Per-chunk states C and dC on the fused bf16 path, 4 values in 12 bytes: the upper 24 bits of
// each float32 (sign, exponent, 15 mantissa bits = 16 significant bits, what the bf16 hi + lo
// pair that consumes them carries), rounded to nearest by adding half of the dropped byte.
// A quarter less state traffic for the scans (which are bound by their state stores) and
// the pass that reads them.  Packed states are blocked by 64 columns: element (row, col) of a
// [DQK][DV] state sits at byte ((col / 64) DQK + row) 192 + (col % 64) 3, so a 64 x 64 block is
// 12 KB contiguous and every access covers whole 128-byte lines (row-major 192-byte rows would
// split lines between neighbouring column blocks, read at different times).
__host__ __device__ constexpr size_t pk24_offset(int row, int col, int DQK) {
  return ((size_t)(col >> 6) * DQK + row) * 192 + (size_t)(col & 63) * 3;
}
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
__device__ __forceinline__ u32x3a pack24(f32x4 x) {
  uint32_t b[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) b[e] = __float_as_uint(x[e]) + 0x80u;
  return u32x3a{(b[0] >> 8) | ((b[1] >> 8) << 24), (b[1] >> 16) | ((b[2] >> 8) << 16),
                (b[2] >> 24) | (b[3] & 0xffffff00u)};
}
__device__ __forceinline__ f32x4 unpack24(u32x3a w) {
  return f32x4{__uint_as_float(w[0] << 8), __uint_as_float(((w[0] >> 24) << 8) | (w[1] << 16)),
               __uint_as_float(((w[1] >> 16) << 8) | (w[2] << 24)), __uint_as_float(w[2] & 0xffffff00u)};
}

// DPP moves inside a row of 16 lanes (VALU only, no LDS traffic)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum16(float v) {  // over the 16 lanes of a tx group (a DPP row)
  v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]: lane ^ 1
  v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2 (every lane holds its quad's sum)
  v += dpp_f<0x141>(v);  // row_half_mirror: the other quad of the half row
  v += dpp_f<0x140>(v);  // row_mirror: the other half row
  return v;
}
// the value of lane r ^ M (M = 1, 2, 4, 8) of the same row of 16 lanes
template <int M>
__device__ __forceinline__ float xor_lane(float x, int lane) {
  if constexpr (M == 1) {
    return dpp_f<0xB1>(x);
  } else if constexpr (M == 2) {
    return dpp_f<0x4E>(x);
  } else {
    const float up = dpp_f<0x100 + M>(x), down = dpp_f<0x110 + M>(x);  // row_shl:M (lane + M), row_shr:M (lane - M)
    return (lane & M) ? down : up;
  }
}

struct BwLayout {
  size_t Cst, nst, mst, cfin, nfin, mfin, vm, vn, dC, dfp, dip, gprep, total;
};

constexpr int GP_STRIDE = kChunkGatePrefix;  // floats per chunk of the scans' gate prefix

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

BwLayout bw_layout(int B, int NH, int S, int DQK, int DV, int L) {
  const size_t BNH = (size_t)B * NH, NC = (size_t)(S / L);
  const size_t ndt = (DQK + BW_T - 1) / BW_T, nvt = (DV + BW_T - 1) / BW_T;
  BwLayout o{};
  size_t off = 0;
  auto take = [&](size_t floats) {
    const size_t at = off;
    off += align256(floats * sizeof(float));
    return at;
  };
  o.Cst = take(BNH * NC * DQK * DV);
  o.nst = take(BNH * NC * DQK);
  o.mst = take(BNH * NC);
  o.cfin = take(BNH * DQK * DV);
  o.nfin = take(BNH * DQK);
  o.mfin = take(BNH);
  o.vm = take(BNH * S);
  o.vn = take(BNH * S);
  o.dC = take(BNH * (NC + 1) * DQK * DV);
  o.dfp = take(BNH * S * ndt);
  o.dip = take(BNH * S * nvt);
  o.gprep = take(BNH * NC * GP_STRIDE);
  o.total = off;
  return o;
}

// inclusive sum over the 64 lanes of a wave (lane order): the DPP row shifts and row broadcasts
// of wave_sum_dpp leave every lane with its prefix
__device__ __forceinline__ float wave_incl_sum(float x, int) { return wave_sum_dpp(x); }

// maximum over the 64 lanes of a wave, in every lane: DPP inside each row of 16, then the four
// row maxima read as scalars
__device__ __forceinline__ float wave_max_rows(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));   // lane ^ 1
  v = fmaxf(v, dpp_f<0x4E>(v));   // lane ^ 2
  v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
  return fmaxf(fmaxf(lane_of(v, 0), lane_of(v, 16)), fmaxf(lane_of(v, 32), lane_of(v, 48)));
}

// Per-chunk gate prefix of the backward kernels: sb[t] = sum_{u<=t} logsig f_u, si[t] = i_t
// for the L tokens from g0, scanned by wave 0 (lane = token); called by every thread, one
// barrier.
template <typename TG, int L>
__device__ __forceinline__ void chunk_gate_scan(const TG* __restrict__ ig, const TG* __restrict__ fg, size_t g0,
                                                float* sb, float* si) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const float x = tid < L ? logsigmoid(to_f32(fg[g0 + tid])) : 0.f;
    const float b = wave_incl_sum(x, tid);
    if (tid < L) {
      sb[tid] = b;
      si[tid] = to_f32(ig[g0 + tid]);
    }
  }
  __syncthreads();
}

// chunk_gate_scan with token t's f and i already loaded by thread t (t < L), so that the
// kernel's first global loads all go out together
template <int L>
__device__ __forceinline__ void chunk_gate_scan_v(float f, float i, float* sb, float* si) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const float b = wave_incl_sum(tid < L ? logsigmoid(f) : 0.f, tid);
    if (tid < L) {
      sb[tid] = b;
      si[tid] = i;
    }
  }
  __syncthreads();
}

// combined stabiliser of token i of a chunk entering with m_prev: max(b_i + m_prev,
// max_{j<=i} b_i - b_j + i_j) (fw.py:204-217)
template <int L>
__device__ __forceinline__ float m_combine(const float* sb, const float* si, int i, float m_prev) {
  float mi = -INFINITY;
  for (int j = 0; j <= i; ++j) mi = fmaxf(mi, sb[i] - sb[j] + si[j]);
  return fmaxf(sb[i] + m_prev, mi);
}

// ------------------------------------------------------------------ 2. stats
template <typename TQ, typename TG, int L>
__global__ __launch_bounds__(BW_THREADS) void bw_stats_kernel(const TQ* __restrict__ q, const TQ* __restrict__ k,
                                                               const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                               const float* __restrict__ nst,
                                                               const float* __restrict__ mst, float* __restrict__ vm,
                                                               float* __restrict__ vn, int NC, int DQK,
                                                               float qk_scale, float eps) {
  constexpr int RS = L / 16;
  __shared__ float sQt[BW_KT][L], sKt[BW_KT][L], sn[BW_KT];
  __shared__ float sM[L][L + 1];
  __shared__ float sb[L], si[L], smc[L], sqb[L];
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int bh = blockIdx.x / NC, kc = blockIdx.x - bh * NC;
  const size_t row0 = (size_t)bh * NC * L + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  chunk_gate_scan<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {
    const float mp = mst[sidx];
    const float mc = m_combine<L>(sb, si, tid, mp);
    smc[tid] = mc;
    sqb[tid] = expf(sb[tid] + mp - mc) * qk_scale;  // fw.py:230-231
  }
  float accS[RS][RS] = {};
  float qn = 0.f;
  for (int dd = 0; dd < DQK; dd += BW_KT) {
    __syncthreads();
    for (int e = tid; e < L * BW_KT; e += BW_THREADS) {
      const int t = e / BW_KT, c = e - t * BW_KT;
      const bool ok = dd + c < DQK;
      sQt[c][t] = ok ? to_f32(q[(row0 + t) * DQK + dd + c]) : 0.f;
      sKt[c][t] = ok ? to_f32(k[(row0 + t) * DQK + dd + c]) : 0.f;
    }
    if (tid < BW_KT) sn[tid] = (dd + tid < DQK) ? nst[sidx * DQK + dd + tid] : 0.f;
    __syncthreads();
#pragma unroll 4
    for (int d = 0; d < BW_KT; ++d) {
      float qv[RS], kv[RS];
#pragma unroll
      for (int a = 0; a < RS; ++a) qv[a] = sQt[d][ty * RS + a];
#pragma unroll
      for (int b = 0; b < RS; ++b) kv[b] = sKt[d][tx * RS + b];
#pragma unroll
      for (int a = 0; a < RS; ++a)
#pragma unroll
        for (int b = 0; b < RS; ++b) accS[a][b] += qv[a] * kv[b];
    }
    if (tid < L)
      for (int d = 0; d < BW_KT; ++d) qn += sQt[d][tid] * sn[d];
  }
  // M = S s exp(b_i - b_j + i_j - m_i) on j <= i (fw.py:219-227)
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const int i = ty * RS + a;
#pragma unroll
    for (int b = 0; b < RS; ++b) {
      const int j = tx * RS + b;
      sM[i][j] = (j <= i) ? accS[a][b] * qk_scale * expf(sb[i] - sb[j] + si[j] - smc[i]) : 0.f;
    }
  }
  __syncthreads();
  if (tid < L) {  // den = qbar (q . n) + sum_j M_ij; divisor max(|den|, exp(-m)) + eps (fw.py:237-245)
    float rs = 0.f;
    for (int j = 0; j < L; ++j) rs += sM[tid][j];
    const float den = sqb[tid] * qn + rs;
    vm[row0 + tid] = smc[tid];
    vn[row0 + tid] = fmaxf(fabsf(den), expf(-smc[tid])) + eps;
  }
}

// --------------------------------------------------------------- 3. dC pass
template <typename TQ, typename TG, int L>
__global__ __launch_bounds__(BW_THREADS) void bw_dC_kernel(const TQ* __restrict__ q, const TQ* __restrict__ dh,
                                                            const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                            const float* __restrict__ mst,
                                                            const float* __restrict__ mfin,
                                                            const float* __restrict__ vm,
                                                            const float* __restrict__ vn,
                                                            const float* __restrict__ dc_last,
                                                            float* __restrict__ dCst, float* __restrict__ dc0,
                                                            int NC, int DQK, int DV, int ndt, int nvt,
                                                            float qk_scale) {
  __shared__ float sQ[L][BW_T + 1], sH[L][BW_T + 1];
  __shared__ float sb[L], si[L], scoef[L];
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int per_bh = ndt * nvt;
  const int bh = blockIdx.x / per_bh, rem = blockIdx.x - bh * per_bh;
  const int d0 = (rem / nvt) * BW_T, v0 = (rem % nvt) * BW_T;
  const size_t S = (size_t)NC * L;
  float dC[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int d = d0 + 4 * ty + a, v = v0 + 4 * tx + b;
      dC[a][b] = (dc_last && d < DQK && v < DV) ? dc_last[((size_t)bh * DQK + d) * DV + v] : 0.f;
    }
  auto store = [&](float* dst) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int d = d0 + 4 * ty + a, v = v0 + 4 * tx + b;
        if (d < DQK && v < DV) dst[(size_t)d * DV + v] = dC[a][b];
      }
  };
  for (int kc = NC - 1; kc >= 0; --kc) {
    store(dCst + ((size_t)bh * (NC + 1) + kc + 1) * DQK * DV);  // bw.py:81
    const size_t row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
    chunk_gate_scan<TG, L>(ig, fg, row0, sb, si);
    const float mp = mst[sidx];
    const float mn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
    // Qbar dH~ = q exp(b + m_{k-1} - m_comb) s / (N + eps) (bw.py:92-101)
    if (tid < L) scoef[tid] = expf(sb[tid] + mp - vm[row0 + tid]) * qk_scale / vn[row0 + tid];
    for (int e = tid; e < L * BW_T; e += BW_THREADS) {
      const int t = e / BW_T, c = e - t * BW_T;
      sQ[t][c] = (d0 + c < DQK) ? to_f32(q[(row0 + t) * DQK + d0 + c]) : 0.f;
      sH[t][c] = (v0 + c < DV) ? to_f32(dh[(row0 + t) * DV + v0 + c]) : 0.f;
    }
    __syncthreads();
    const float gbar = expf(sb[L - 1] + mp - mn);  // bw.py:86-89
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) dC[a][b] *= gbar;
    for (int t = 0; t < L; ++t) {  // bw.py:104
      const float co = scoef[t];
      float qd[4], hv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) qd[a] = sQ[t][4 * ty + a] * co;
#pragma unroll
      for (int b = 0; b < 4; ++b) hv[b] = sH[t][4 * tx + b];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) dC[a][b] += qd[a] * hv[b];
    }
    __syncthreads();  // LDS reused by the next chunk
  }
  store(dCst + (size_t)bh * (NC + 1) * DQK * DV);  // bw.py:110
  if (dc0) store(dc0 + (size_t)bh * DQK * DV);
}

// --------------------------------------------------------------- 4. dV pass
template <int L>
struct DvSmem {
  // phase 1 (contraction over DQK): Q^T, K^T tiles and the dC tile
  static constexpr int QT = 0, KT = QT + BW_KT * L, DC = KT + BW_KT * L, P1 = DC + BW_KT * BW_T;
  // phase 2: Sbar [L][L + 1] and dH~ [L][BW_T + 1]
  static constexpr int SB = 0, H = SB + L * (L + 1), P2 = H + L * (BW_T + 1);
  static constexpr int TOTAL = P1 > P2 ? P1 : P2;
};

template <typename TQ, typename TG, int L>
__global__ __launch_bounds__(BW_THREADS) void bw_dv_kernel(const TQ* __restrict__ q, const TQ* __restrict__ k,
                                                            const TQ* __restrict__ v, const TQ* __restrict__ dh,
                                                            const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                            const float* __restrict__ mst,
                                                            const float* __restrict__ mfin,
                                                            const float* __restrict__ vm,
                                                            const float* __restrict__ vn,
                                                            const float* __restrict__ dCst, TQ* __restrict__ dv,
                                                            float* __restrict__ dip, int NC, int DQK, int DV,
                                                            int nvt, float qk_scale) {
  constexpr int RS = L / 16;
  using SM = DvSmem<L>;
  __shared__ float smem[SM::TOTAL];
  __shared__ float sb[L], si[L], smc[L], sinv[L], sab[L];
  float* sQt = smem + SM::QT;
  float* sKt = smem + SM::KT;
  float* sdC = smem + SM::DC;
  float* sSb = smem + SM::SB;
  float* sH = smem + SM::H;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int per_bh = NC * nvt;
  const int bh = blockIdx.x / per_bh, rem = blockIdx.x - bh * per_bh;
  const int kc = rem / nvt, vt = rem - kc * nvt, v0 = vt * BW_T;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  const float* dCk = dCst + ((size_t)bh * (NC + 1) + kc + 1) * DQK * DV;  // gradient of the state after chunk kc
  chunk_gate_scan<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {
    const float mn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
    smc[tid] = vm[row0 + tid];
    sinv[tid] = 1.0f / vn[row0 + tid];
    sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - mn);  // Abar = exp(b_L - b + i - m_k) (bw.py:168-176)
  }
  float accS[RS][RS] = {}, accV[RS][4] = {};
  for (int dd = 0; dd < DQK; dd += BW_KT) {
    __syncthreads();
    for (int e = tid; e < L * BW_KT; e += BW_THREADS) {
      const int t = e / BW_KT, c = e - t * BW_KT;
      const bool ok = dd + c < DQK;
      sQt[c * L + t] = ok ? to_f32(q[(row0 + t) * DQK + dd + c]) : 0.f;
      sKt[c * L + t] = ok ? to_f32(k[(row0 + t) * DQK + dd + c]) : 0.f;
    }
    for (int e = tid; e < BW_KT * BW_T; e += BW_THREADS) {
      const int r = e / BW_T, c = e - r * BW_T;
      sdC[r * BW_T + c] = (dd + r < DQK && v0 + c < DV) ? dCk[(size_t)(dd + r) * DV + v0 + c] : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int d = 0; d < BW_KT; ++d) {
      float qv[RS], kv[RS], kr[RS], cv[4];
#pragma unroll
      for (int a = 0; a < RS; ++a) {
        qv[a] = sQt[d * L + ty * RS + a];
        kr[a] = sKt[d * L + ty * RS + a];
      }
#pragma unroll
      for (int b = 0; b < RS; ++b) kv[b] = sKt[d * L + tx * RS + b];
#pragma unroll
      for (int c = 0; c < 4; ++c) cv[c] = sdC[d * BW_T + tx * 4 + c];
#pragma unroll
      for (int a = 0; a < RS; ++a) {
#pragma unroll
        for (int b = 0; b < RS; ++b) accS[a][b] += qv[a] * kv[b];
#pragma unroll
        for (int c = 0; c < 4; ++c) accV[a][c] += kr[a] * cv[c];
      }
    }
  }
  __syncthreads();  // phase-1 tiles dead
  // inter: (K * Abar) dC_k (bw.py:179); Sbar = S s Dbar on j <= i (bw.py:146-153)
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const int t = ty * RS + a;
    const float ab = sab[t];
#pragma unroll
    for (int c = 0; c < 4; ++c) accV[a][c] *= ab;
#pragma unroll
    for (int b = 0; b < RS; ++b) {
      const int j = tx * RS + b;
      sSb[t * (L + 1) + j] = (j <= t) ? accS[a][b] * qk_scale * expf(sb[t] - sb[j] + si[j] - smc[t]) : 0.f;
    }
  }
  for (int e = tid; e < L * BW_T; e += BW_THREADS) {
    const int t = e / BW_T, c = e - t * BW_T;
    sH[t * (BW_T + 1) + c] = (v0 + c < DV) ? to_f32(dh[(row0 + t) * DV + v0 + c]) * sinv[t] : 0.f;
  }
  __syncthreads();
  // intra: dV_j = sum_t Sbar_tj dH~_t (bw.py:156)
  for (int t = 0; t < L; ++t) {
    float sv[RS], hv[4];
#pragma unroll
    for (int a = 0; a < RS; ++a) sv[a] = sSb[t * (L + 1) + ty * RS + a];
#pragma unroll
    for (int c = 0; c < 4; ++c) hv[c] = sH[t * (BW_T + 1) + tx * 4 + c];
#pragma unroll
    for (int a = 0; a < RS; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) accV[a][c] += sv[a] * hv[c];
  }
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const size_t row = row0 + ty * RS + a;
    float part = 0.f;  // v . dV over this tile (bw.py:338)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int vv = v0 + tx * 4 + c;
      if (vv < DV) {
        dv[row * DV + vv] = from_f32<TQ>(accV[a][c]);
        part += to_f32(v[row * DV + vv]) * accV[a][c];
      }
    }
    part = sum16(part);
    if (tx == 0) dip[row * nvt + vt] = part;
  }
}

// ------------------------------------------------------------ 5. dQ, dK pass
template <int L>
struct DqkSmem {
  // phase 1 (contraction over DV): dH~^T, V^T tiles, C_{k-1} and dC_k tiles (transposed)
  static constexpr int HT = 0, VT = HT + BW_KT * L, CT = VT + BW_KT * L, DCT = CT + BW_KT * BW_T,
                       P1 = DCT + BW_KT * BW_T;
  // phase 2: dS [L][L + 1], Q and K tiles [L][BW_T + 1]
  static constexpr int DS = 0, Q = DS + L * (L + 1), K = Q + L * (BW_T + 1), P2 = K + L * (BW_T + 1);
  static constexpr int TOTAL = P1 > P2 ? P1 : P2;
};

template <typename TQ, typename TG, int L>
__global__ __launch_bounds__(BW_THREADS) void bw_dqk_kernel(const TQ* __restrict__ q, const TQ* __restrict__ k,
                                                             const TQ* __restrict__ v, const TQ* __restrict__ dh,
                                                             const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                             const float* __restrict__ Cst,
                                                             const float* __restrict__ mst,
                                                             const float* __restrict__ mfin,
                                                             const float* __restrict__ vm,
                                                             const float* __restrict__ vn,
                                                             const float* __restrict__ dCst, TQ* __restrict__ dq,
                                                             TQ* __restrict__ dk, float* __restrict__ dfp, int NC,
                                                             int DQK, int DV, int ndt, float qk_scale) {
  constexpr int RS = L / 16;
  using SM = DqkSmem<L>;
  __shared__ float smem[SM::TOTAL];
  __shared__ float sb[L], si[L], smc[L], sinv[L], sab[L], sbb[L];
  float* sHt = smem + SM::HT;
  float* sVt = smem + SM::VT;
  float* sCt = smem + SM::CT;
  float* sdCt = smem + SM::DCT;
  float* sdS = smem + SM::DS;
  float* sQ = smem + SM::Q;
  float* sK = smem + SM::K;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int per_bh = NC * ndt;
  const int bh = blockIdx.x / per_bh, rem = blockIdx.x - bh * per_bh;
  const int kc = rem / ndt, dt = rem - kc * ndt, d0 = dt * BW_T;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  const float* Ck = Cst + sidx * DQK * DV;                                   // state entering chunk kc
  const float* dCk = dCst + ((size_t)bh * (NC + 1) + kc + 1) * DQK * DV;  // gradient of the state after it
  chunk_gate_scan<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {
    const float mp = mst[sidx];
    const float mn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
    const float mc = vm[row0 + tid];
    smc[tid] = mc;
    sinv[tid] = 1.0f / vn[row0 + tid];
    sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - mn);  // Abar (bw.py:168-176)
    sbb[tid] = expf(sb[tid] + mp - mc) * qk_scale;        // Bbar s (bw.py:175, 182)
  }
  float accS[RS][RS] = {}, accQ[RS][4] = {}, accK[RS][4] = {};
  for (int vv = 0; vv < DV; vv += BW_KT) {
    __syncthreads();
    for (int e = tid; e < L * BW_KT; e += BW_THREADS) {
      const int t = e / BW_KT, c = e - t * BW_KT;
      const bool ok = vv + c < DV;
      sHt[c * L + t] = ok ? to_f32(dh[(row0 + t) * DV + vv + c]) * sinv[t] : 0.f;
      sVt[c * L + t] = ok ? to_f32(v[(row0 + t) * DV + vv + c]) : 0.f;
    }
    for (int e = tid; e < BW_KT * BW_T; e += BW_THREADS) {
      const int r = e / BW_KT, c = e - r * BW_KT;  // r: d row of the tile, c: v column
      const bool ok = d0 + r < DQK && vv + c < DV;
      sCt[c * BW_T + r] = ok ? Ck[(size_t)(d0 + r) * DV + vv + c] : 0.f;
      sdCt[c * BW_T + r] = ok ? dCk[(size_t)(d0 + r) * DV + vv + c] : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int r = 0; r < BW_KT; ++r) {
      float hv[RS], vj[RS], vr[RS], cv[4], dcv[4];
#pragma unroll
      for (int a = 0; a < RS; ++a) {
        hv[a] = sHt[r * L + ty * RS + a];
        vr[a] = sVt[r * L + ty * RS + a];
      }
#pragma unroll
      for (int b = 0; b < RS; ++b) vj[b] = sVt[r * L + tx * RS + b];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        cv[c] = sCt[r * BW_T + tx * 4 + c];
        dcv[c] = sdCt[r * BW_T + tx * 4 + c];
      }
#pragma unroll
      for (int a = 0; a < RS; ++a) {
#pragma unroll
        for (int b = 0; b < RS; ++b) accS[a][b] += hv[a] * vj[b];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          accQ[a][c] += hv[a] * cv[c];
          accK[a][c] += vr[a] * dcv[c];
        }
      }
    }
  }
  __syncthreads();  // phase-1 tiles dead
  // inter terms (bw.py:181-182); dS = (dH~ V^T) Dbar on j <= i (bw.py:158-159)
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const int t = ty * RS + a;
    const float bb = sbb[t], ab = sab[t];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      accQ[a][c] *= bb;
      accK[a][c] *= ab;
    }
#pragma unroll
    for (int b = 0; b < RS; ++b) {
      const int j = tx * RS + b;
      sdS[t * (L + 1) + j] = (j <= t) ? accS[a][b] * expf(sb[t] - sb[j] + si[j] - smc[t]) : 0.f;
    }
  }
  for (int e = tid; e < L * BW_T; e += BW_THREADS) {
    const int t = e / BW_T, c = e - t * BW_T;
    const bool ok = d0 + c < DQK;
    sQ[t * (BW_T + 1) + c] = ok ? to_f32(q[(row0 + t) * DQK + d0 + c]) : 0.f;
    sK[t * (BW_T + 1) + c] = ok ? to_f32(k[(row0 + t) * DQK + d0 + c]) : 0.f;
  }
  __syncthreads();
  // intra: dQ_t = s sum_j dS_tj K_j, dK_j = s sum_t dS_tj Q_t (bw.py:161-162)
  float iq[RS][4] = {}, ik[RS][4] = {};
  for (int j = 0; j < L; ++j) {
    float dsq[RS], dsk[RS], kv[4], qv[4];
#pragma unroll
    for (int a = 0; a < RS; ++a) {
      dsq[a] = sdS[(ty * RS + a) * (L + 1) + j];  // dS[t = row][j]
      dsk[a] = sdS[j * (L + 1) + ty * RS + a];    // dS[t = j][row]
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kv[c] = sK[j * (BW_T + 1) + tx * 4 + c];
      qv[c] = sQ[j * (BW_T + 1) + tx * 4 + c];
    }
#pragma unroll
    for (int a = 0; a < RS; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        iq[a][c] += dsq[a] * kv[c];
        ik[a][c] += dsk[a] * qv[c];
      }
  }
#pragma unroll
  for (int a = 0; a < RS; ++a) {
    const int t = ty * RS + a;
    const size_t row = row0 + t;
    float part = 0.f;  // q . dQ - k . dK over this tile (bw.py:333)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = d0 + tx * 4 + c;
      const float gq = accQ[a][c] + qk_scale * iq[a][c];
      const float gk = accK[a][c] + qk_scale * ik[a][c];
      if (d < DQK) {
        dq[row * DQK + d] = from_f32<TQ>(gq);
        dk[row * DQK + d] = from_f32<TQ>(gk);
        part += sQ[t * (BW_T + 1) + tx * 4 + c] * gq - sK[t * (BW_T + 1) + tx * 4 + c] * gk;
      }
    }
    part = sum16(part);
    if (tx == 0) dfp[row * ndt + dt] = part;
  }
}

// --------------------------------------------------------------- 6. gates
// One workgroup per (head, segment of GSEG tokens): dI_t = sum of its dV partials;
// dF_t = sigmoid(-f_t) times the suffix sum over u >= t of the q . dQ - k . dK partials
// (bw.py:332-338): the segment's own suffix scan (4 consecutive tokens per thread, then a
// reverse scan over the lanes and the 4 waves) plus the total of every later segment, which
// each workgroup sums itself (a plain reduction over contiguous partials).
constexpr int GSEG = 1024;

template <typename TG>
__global__ __launch_bounds__(256) void bw_gates_kernel(const TG* __restrict__ fg, const float* __restrict__ dfp,
                                                       const float* __restrict__ dip, TG* __restrict__ di,
                                                       TG* __restrict__ df, int S, int ndt, int nvt) {
  __shared__ float s_wave[4], s_red[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nseg = (S + GSEG - 1) / GSEG;
  const int bh = blockIdx.x / nseg, sg = blockIdx.x - bh * nseg;
  const size_t base = (size_t)bh * S;
  const int t0 = sg * GSEG, t1 = min(S, t0 + GSEG);
  // total of the later segments' partials
  float c = 0.f;
  const float* later = dfp + (base + t1) * ndt;
  const size_t nl = (size_t)(S - t1) * ndt;
  for (size_t e = tid; e < nl; e += 256) c += later[e];
  // this thread's tokens t0 + 4 tid + u
  float x[4], fv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 4 * tid + u;
    float a = 0.f, sd = 0.f;
    fv[u] = 0.f;
    if (t < t1) {
      for (int j = 0; j < ndt; ++j) a += dfp[(base + t) * ndt + j];
      for (int j = 0; j < nvt; ++j) sd += dip[(base + t) * nvt + j];
      di[base + t] = from_f32<TG>(sd);
      fv[u] = to_f32(fg[base + t]);
    }
    x[u] = a;
  }
  float suf[4];
  suf[3] = x[3];
  suf[2] = x[2] + suf[3];
  suf[1] = x[1] + suf[2];
  suf[0] = x[0] + suf[1];
  // inclusive suffix over the lanes of the wave, and the wave reductions
  float v = suf[0];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_down(v, o, 64);
    if (lane + o < 64) v += y;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
  if (lane == 0) {
    s_wave[w] = v;
    s_red[w] = c;
  }
  __syncthreads();
  float after = v - suf[0] + s_red[0] + s_red[1] + s_red[2] + s_red[3];  // everything past this thread's tokens
  for (int w2 = w + 1; w2 < 4; ++w2) after += s_wave[w2];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 4 * tid + u;
    if (t < t1) df[base + t] = from_f32<TG>((suf[u] + after) / (1.0f + expf(fv[u])));  // * sigmoid(-f)
  }
}

// --------------------------------------------------- MFMA chunk scans (1, 3)
// The two chunk-sequential passes on v_mfma_f32_16x16x4f32: float32 operands and
// accumulation, the arithmetic of the FMA form at the matrix cores' rate.  One
// workgroup of 4 waves per (head, 64 columns of DV); wave w holds rows
// [16 NRT w, 16 NRT (w + 1)) of the DQK x 64 state as NRT x 4 accumulator tiles of
// 16 x 16.  Per chunk, X (K forward, Q reverse) is staged in LDS in its own dtype and
// Y (V forward, dH reverse) in float32 with the per-token coefficient folded in, then
//   state = decay state + sum_t X[t][rows]^T (coef_t Y[t][cols]),
// four tokens per MFMA: lane (g, r) supplies X[t0 + g][row r of the tile] and
// coef Y[t0 + g][column r of the tile] (16x16x4: A[i][k] in lane i + 16 k, B[k][j] in
// lane j + 16 k, D[i][j] in lane j + 16 (i / 4), element i % 4).  The next chunk's
// X, Y and gates are loaded into registers while the MFMAs run.
//  * forward (REV false): X = K, Y = V, coef_t = exp(a_t - m'), decay = exp(g + m - m');
//    stores the state entering every chunk (recurrent_fw_C, fw.py:98-143), with n (v
//    tile 0) and m beside it, and the state after the last chunk;
//  * reverse (REV true): X = Q, Y = dH, coef_t = exp(b_t + m_{k-1} - m_t) s / (N_t + eps),
//    decay = exp(g + m_{k-1} - m_k); stores the gradient of the state after every chunk
//    and, last, of the initial state (bw.py:31-115).
constexpr int SC_V = 64;          // DV columns per workgroup
constexpr int SC_YP = SC_V + 16;  // floats per staged Y row (16 mod 64 dwords: 4 rows, distinct banks)


__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <typename T>
union Piece16 {
  u32x4 raw;
  T v[16 / sizeof(T)];
};

template <typename TQ, typename TG, int L, int NRT, bool REV>
__global__ __launch_bounds__(256) void bw_scan_kernel(
    const TQ* __restrict__ X, const TQ* __restrict__ Y, const TG* __restrict__ ig, const TG* __restrict__ fg,
    const float* __restrict__ s0, const float* __restrict__ n0, const float* __restrict__ m0,
    const float* __restrict__ vm, const float* __restrict__ vn, float* __restrict__ Sst, float* __restrict__ nst,
    float* __restrict__ mst, float* __restrict__ sfin, float* __restrict__ nfin, float* __restrict__ mfin,
    float* __restrict__ s_init, int NC, int DQKf, int DV, int nvt, float qk_scale) {
  constexpr int DQK = 64 * NRT;  // state rows of this workgroup (DQKf / DQK workgroups share a state)
  constexpr int XP = DQK + 16;   // elements per staged X row (see the bank note above)
  constexpr int EPV = 16 / sizeof(TQ);
  constexpr int PRX = DQK / EPV, NX = L * PRX, NXP = (NX + 255) / 256;
  constexpr int PRY = SC_V / EPV, NY = L * PRY, NYP = (NY + 255) / 256;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  TQ* sX = reinterpret_cast<TQ*>(smem_raw);
  float* sY = reinterpret_cast<float*>(smem_raw + (size_t)L * XP * sizeof(TQ));
  __shared__ float scoef[L];
  __shared__ float s_mn, s_g;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int nrs = DQKf / DQK;
  const int bhv = blockIdx.x / nrs, rs = blockIdx.x - bhv * nrs;
  const int bh = bhv / nvt, vt = bhv - bh * nvt, v0 = vt * SC_V;
  const int d_off = rs * DQK;  // this workgroup's first state row
  const size_t S = (size_t)NC * L;
  const int row0 = d_off + w * 16 * NRT;  // this wave's first state row
  const int nslots = REV ? NC + 1 : NC;

  f32x4 acc[NRT][4];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc[rt][ct][e] = s0 ? s0[((size_t)bh * DQKf + row0 + 16 * rt + 4 * g + e) * DV + v0 + 16 * ct + r] : 0.f;
  auto store_state = [&](float* dst) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(size_t)(row0 + 16 * rt + 4 * g + e) * DV + v0 + 16 * ct + r] = acc[rt][ct][e];
  };
  const bool owns_n = !REV && vt == 0 && tid < DQK;
  float nn = (owns_n && n0) ? n0[(size_t)bh * DQKf + d_off + tid] : 0.f;
  float m = (!REV && m0) ? m0[bh] : 0.f;

  // prefetch registers: X, Y pieces and this thread's token gates (tid < L)
  u32x4 px[NXP], py[NYP];
  float pf = 0.f, pi = 0.f, pvm = 0.f, pvn = 1.f, pmp = 0.f;
  auto fetch = [&](int kc) {
    const size_t t0 = (size_t)bh * S + (size_t)kc * L;
#pragma unroll
    for (int u = 0; u < NXP; ++u) {
      const int p = u * 256 + tid;
      if (NX % 256 == 0 || p < NX)
        px[u] = *reinterpret_cast<const u32x4*>(X + (t0 + p / PRX) * DQKf + d_off + (p % PRX) * EPV);
    }
#pragma unroll
    for (int u = 0; u < NYP; ++u) {
      const int p = u * 256 + tid;
      if (NY % 256 == 0 || p < NY)
        py[u] = *reinterpret_cast<const u32x4*>(Y + (t0 + p / PRY) * DV + v0 + (p % PRY) * EPV);
    }
    if (tid < L) {
      pf = to_f32(fg[t0 + tid]);
      pi = to_f32(ig[t0 + tid]);
      if (REV) {
        pvm = vm[t0 + tid];
        pvn = vn[t0 + tid];
      }
    }
    if (REV) pmp = mst[(size_t)bh * NC + kc];  // m entering chunk kc
  };
  float mnext = REV ? mfin[bh] : 0.f;  // reverse: m after the chunk being processed
  const int kfirst = REV ? NC - 1 : 0;
  fetch(kfirst);
  for (int it = 0; it < NC; ++it) {
    const int kc = REV ? NC - 1 - it : it;
    const size_t sidx = (size_t)bh * NC + kc;
    const int slot = REV ? kc + 1 : kc;
    // gates of this chunk from the prefetched values, wave 0 (lane = token): b = cumsum logsig f,
    // then the coefficients and the decay
    const float cvm = pvm, cvn = pvn, cmp = pmp;
    if (w == 0) {
      const float b = wave_incl_sum(lane < L ? logsigmoid(pf) : 0.f, lane);
      const float gl = lane_of(b, L - 1);
      if (!REV) {
        const float a = lane < L ? gl - b + pi : -INFINITY;
        const float mn = fmaxf(gl + m, wave_max_rows(a));  // fw.py:115
        if (lane < L) scoef[lane] = expf(a - mn);     // fw.py:121
        if (lane == 0) {
          s_mn = mn;
          s_g = gl;
        }
      } else {
        if (lane < L) scoef[lane] = expf(b + cmp - cvm) * qk_scale / cvn;  // bw.py:92-101
        if (lane == 0) s_g = gl;
      }
    }
    __syncthreads();
    const float gch = s_g;
    float decay;
    const float m_in = m;
    if (!REV) {
      const float mn = s_mn;
      decay = expf(gch + m - mn);  // fw.py:125
      m = mn;
    } else {
      decay = expf(gch + cmp - mnext);  // bw.py:86-89
      mnext = cmp;
    }
    // stage X (own dtype) and coef Y (float32)
#pragma unroll
    for (int u = 0; u < NXP; ++u) {
      const int p = u * 256 + tid;
      if (NX % 256 == 0 || p < NX) *reinterpret_cast<u32x4*>(sX + (p / PRX) * XP + (p % PRX) * EPV) = px[u];
    }
#pragma unroll
    for (int u = 0; u < NYP; ++u) {
      const int p = u * 256 + tid;
      if (NY % 256 == 0 || p < NY) {
        const int t = p / PRY, c = (p % PRY) * EPV;
        Piece16<TQ> pc;
        pc.raw = py[u];
        const float co = scoef[t];
        float* dst = sY + t * SC_YP + c;
#pragma unroll
        for (int e = 0; e < EPV; e += 4)
          *reinterpret_cast<f32x4*>(dst + e) =
              f32x4{co * to_f32(pc.v[e]), co * to_f32(pc.v[e + 1]), co * to_f32(pc.v[e + 2]), co * to_f32(pc.v[e + 3])};
      }
    }
    if (it + 1 < NC) fetch(REV ? kc - 1 : kc + 1);
    __syncthreads();
    // the state entering this chunk (forward) / after it (reverse), stored here, after the
    // waits for the staged data, so that the next wait (one chunk later) finds them done
    store_state(Sst + ((size_t)bh * nslots + slot) * DQKf * DV);
    if (owns_n) nst[sidx * DQKf + d_off + tid] = nn;
    if (!REV && vt == 0 && rs == 0 && tid == 0) mst[sidx] = m_in;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) acc[rt][ct] *= decay;
#pragma unroll 4
    for (int t0 = 0; t0 < L; t0 += 4) {
      float a[NRT], b[4];
      const TQ* xr = sX + (t0 + g) * XP + (row0 - d_off) + r;
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) a[rt] = to_f32(xr[16 * rt]);
      const float* yr = sY + (t0 + g) * SC_YP + r;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) b[ct] = yr[16 * ct];
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = mfma4(a[rt], b[ct], acc[rt][ct]);
    }
    if (owns_n) {  // n' = decay n + sum_t coef_t k_t (fw.py:133)
      float sacc = 0.f;
      for (int t = 0; t < L; ++t) sacc += scoef[t] * to_f32(sX[t * XP + tid]);
      nn = decay * nn + sacc;
    }
    __syncthreads();  // the staged tiles are read; the next chunk may overwrite them
  }
  if (!REV) {  // the final state (the forward's last states may not be asked for)
    if (sfin) store_state(sfin + (size_t)bh * DQKf * DV);
    if (owns_n && nfin) nfin[(size_t)bh * DQKf + d_off + tid] = nn;
    if (vt == 0 && rs == 0 && tid == 0 && mfin) mfin[bh] = m;
  } else {
    store_state(Sst + (size_t)bh * nslots * DQKf * DV);
    if (s_init) store_state(s_init + (size_t)bh * DQKf * DV);
  }
}

template <typename TQ, int L>
constexpr size_t scan_smem(int NRT) {
  return (size_t)L * (64 * NRT + 16) * sizeof(TQ) + (size_t)L * SC_YP * sizeof(float);
}


// ------------------------------------------------------ bf16 MFMA stats (2)
// bw_stats_kernel for bf16 q / k and 64-token chunks on v_mfma_f32_16x16x32_bf16: one
// workgroup of 4 waves per (head, chunk); wave w owns query rows [16 w, 16 w + 16) and all
// 64 key columns, so every row sum stays in the wave.  Per 32 d: A = Q rows (loaded from
// global memory straight into the operand registers), B = K rows (the chunk's K staged once in
// LDS) for S[i][j]; a fifth tile takes B = n_{k-1} as bf16 hi (column 0) and lo (column 1), so
// q . n = D[i][0] + D[i][1].  Then M = S s exp(b_i - b_j + i_j - m_i) on j <= i, its row sums
// over the tiles and the 16 lanes of a group, and the divisor (fw.py:219-245).
template <typename TG, int NRT>
__global__ __launch_bounds__(256) void bw_stats_bf16_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                             const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                             const float* __restrict__ nst,
                                                             const float* __restrict__ mst, float* __restrict__ vm,
                                                             float* __restrict__ vn, float* __restrict__ gp, int NC,
                                                             float qk_scale, float eps) {
  constexpr int L = 64, DQK = 64 * NRT;
  constexpr int KP = DQK + 16;               // bf16 per staged K row (2 DQK + 32 bytes)
  constexpr int PR = DQK / 8, NP = L * PR / 256;  // 16-byte pieces per row, per thread
  constexpr int NKS = DQK / 32;              // 32-d MFMA steps
  __shared__ __attribute__((aligned(16))) bf16_t sK[L * KP];
  __shared__ __attribute__((aligned(16))) float sn[DQK];
  __shared__ float sb[L], si[L], smc[L], sqb[L];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int bh = blockIdx.x / NC, kc = blockIdx.x - bh * NC;
  const size_t row0 = (size_t)bh * NC * L + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  // every load first: gates, m, the K chunk, n, this lane's Q operands
  float gf = 0.f, gi = 0.f;
  if (tid < L) {
    gf = to_f32(fg[row0 + tid]);
    gi = to_f32(ig[row0 + tid]);
  }
  const float mp = mst[sidx];
  u32x4 pk[NP], pq[NKS];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int p = u * 256 + tid;
    pk[u] = *reinterpret_cast<const u32x4*>(k + (row0 + p / PR) * DQK + (p % PR) * 8);
  }
  const float nv = tid < DQK ? nst[sidx * DQK + tid] : 0.f;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    pq[ks] = *reinterpret_cast<const u32x4*>(q + (row0 + 16 * w + r) * DQK + 32 * ks + 8 * g);
  chunk_gate_scan_v<L>(gf, gi, sb, si);
  if (tid < L) {
    const float mc = m_combine<L>(sb, si, tid, mp);
    smc[tid] = mc;
    sqb[tid] = expf(sb[tid] + mp - mc) * qk_scale;  // fw.py:230-231
  }
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int p = u * 256 + tid;
    *reinterpret_cast<u32x4*>(sK + (p / PR) * KP + (p % PR) * 8) = pk[u];
  }
  if (tid < DQK) sn[tid] = nv;
  __syncthreads();
  f32x4 acc[4], accN = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) acc[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int c = 32 * ks + 8 * g;
    const bfx8 qa = __builtin_bit_cast(bfx8, pq[ks]);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) acc[jt] = mfma_bf(qa, ld_bf8(sK + (16 * jt + r) * KP + c), acc[jt]);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = sn[c + e];
    u32x4 h, l;
    split_bf(x, h, l);
    const u32x4 z = {0u, 0u, 0u, 0u};
    accN = mfma_bf(qa, __builtin_bit_cast(bfx8, r == 0 ? h : (r == 1 ? l : z)), accN);
  }
  // lane (g, r), element e: row i = 16 w + 4 g + e; S[i][16 jt + r], q . n in lanes r = 0, 1
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = 16 * w + 4 * g + e;
    float rs = 0.f;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const int j = 16 * jt + r;
      rs += (j <= i) ? acc[jt][e] * qk_scale * expf(sb[i] - sb[j] + si[j] - smc[i]) : 0.f;
    }
    rs = sum16(rs);
    const float qn = accN[e] + xor_lane<1>(accN[e], lane);
    if (r == 0) {  // den = qbar (q . n) + sum_j M_ij; divisor max(|den|, exp(-m)) + eps (fw.py:237-245)
      const float den = sqb[i] * qn + rs;
      const float dv = fmaxf(fabsf(den), expf(-smc[i])) + eps;
      vm[row0 + i] = smc[i];
      vn[row0 + i] = dv;
      if (gp) {  // the dC scan's per-token factors (bw.py:92-101): b - m_comb and qk_scale / divisor
        float* g = gp + sidx * GP_STRIDE;
        g[64 + i] = sb[i] - smc[i];
        g[132 + i] = qk_scale / dv;
      }
    }
  }
}

// Gate prefix of every chunk for the bf16 chunk scans, all chunks at once (one wave per chunk,
// lane = token): b = sum_{u<=t} logsig f_u, its last value gl, a = gl - b + i and max a
// (fw.py:98, 115).  Every one of these is independent of the running stabiliser, so the scans
// no longer form them chunk after chunk on one wave behind a barrier: per chunk each thread only
// takes m' = max(gl + m, max a) and the exponentials of its own tokens.  The same operations in
// the same order as the scans formed them, so the values are identical.
template <typename TG, int L>
__global__ __launch_bounds__(256) void bw_gate_prep_kernel(const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                           float* __restrict__ gp, int total_chunks) {
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);  // bh * NC + chunk
  if (c >= total_chunks) return;                      // no barrier follows
  const size_t t0 = (size_t)c * L;                    // the chunk's first token (S = NC * L)
  const float f = lane < L ? to_f32(fg[t0 + lane]) : 0.f, i = lane < L ? to_f32(ig[t0 + lane]) : 0.f;
  const float b = wave_incl_sum(lane < L ? logsigmoid(f) : 0.f, lane);
  const float gl = lane_of(b, L - 1);
  const float a = lane < L ? gl - b + i : -INFINITY;
  const float amax = wave_max_rows(a);
  float* p = gp + (size_t)c * GP_STRIDE;
  if (lane < L) {
    p[lane] = b;
    p[64 + lane] = a;
  }
  if (lane == 0) {
    p[128] = gl;
    p[129] = amax;
  }
}

// ----------------------------------------------- bf16 MFMA chunk scans (1, 3)
// bw_scan_kernel for bf16 X and Y on v_mfma_f32_16x16x32_bf16: the same workgroups,
// gates, stores and state layout; per chunk X is staged in LDS as it is and coef_t Y[t] as
// its bf16 hi and lo rows, then per 32-token step
//   state[i][j] += sum_k X[T(k)][row i] (hi + lo)[T(k)][column j],
// lane (g, r) holding k = 8 g .. 8 g + 7 at the tokens T = 4 g + 0..3 and 16 + 4 g + 0..3 of
// the step (two transposed reads of each operand).  Rows of 2 DQK + 32 and 160 bytes put
// the 8 consecutive token rows that half a wave reads in distinct banks.
constexpr int SB_YP = SC_V + 16;  // bf16 per staged hi / lo row (160 bytes)
constexpr int SST_P = SC_V + 4;  // floats per LDS row of a state store (conflict-free 16-byte writes and reads)

// two workgroups per CU (at most 256 registers per lane): the scans are bound by their state
// stores, and two workgroups keep more of them in flight
template <typename TG, int L, int NRT, bool REV, bool PK>
__global__ __launch_bounds__(256, 2) void bw_scan_bf16_kernel(
    const bf16_t* __restrict__ X, const bf16_t* __restrict__ Y, const TG* __restrict__ ig,
    const TG* __restrict__ fg, const float* __restrict__ gp, const float* __restrict__ s0,
    const float* __restrict__ n0, const float* __restrict__ m0, const float* __restrict__ vm,
    const float* __restrict__ vn, float* __restrict__ Sst, float* __restrict__ nst, float* __restrict__ mst,
    float* __restrict__ sfin, float* __restrict__ nfin, float* __restrict__ mfin, float* __restrict__ s_init, int NC,
    int DQKf, int DV, int nvt, float qk_scale) {
  static_assert(L % 32 == 0, "32-token MFMA steps");
  constexpr int DQK = 64 * NRT;  // state rows of this workgroup
  constexpr int XP = DQK + 16;   // bf16 per staged X row
  constexpr int PRX = DQK / 8, NX = L * PRX, NXP = (NX + 255) / 256;
  constexpr int PRY = SC_V / 8, NY = L * PRY, NYP = (NY + 255) / 256;
  __shared__ __attribute__((aligned(16))) bf16_t sX[L * XP];
  __shared__ __attribute__((aligned(16))) bf16_t sYh[L * SB_YP];
  __shared__ __attribute__((aligned(16))) bf16_t sYl[L * SB_YP];
  __shared__ __attribute__((aligned(16))) float sSt[4][16 * NRT * SST_P];  // per wave: its state rows, for the stores
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int nrs = DQKf / DQK;
  const int blk = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bhv = blk / nrs, rs = blk - bhv * nrs;
  const int bh = bhv / nvt, vt = bhv - bh * nvt, v0 = vt * SC_V;
  const int d_off = rs * DQK;
  const size_t S = (size_t)NC * L;
  const int row0 = d_off + w * 16 * NRT;
  const int nslots = REV ? NC + 1 : NC;

  // the state transposed in the accumulators: tile (rt, ct) holds D[column][row], lane (g, r)
  // columns 16 ct + 4 g + 0..3 of row 16 rt + r, so a lane stores 16 contiguous bytes
  f32x4 acc[NRT][4];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      acc[rt][ct] = s0 ? *reinterpret_cast<const f32x4*>(s0 + ((size_t)bh * DQKf + row0 + 16 * rt + r) * DV + v0 +
                                                          16 * ct + 4 * g)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
  // A state store goes through the wave's LDS rows, so that each store instruction writes 4 whole
  // 256-byte rows (16 lanes per row, 128-byte lines): straight from the accumulators every row
  // piece would be 64 bytes, and the stores, sent to L2 as 64-byte requests, capped the scans'
  // write rate at about 2.8 TB/s.  Only this wave touches its rows: no barrier.
  // With PK the per-chunk states (slots) go out as pack24 (12-byte pieces of 192-byte block rows).
  float* const st_w = sSt[w];
  auto store_state = [&](float* dst, bool packed) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        *reinterpret_cast<f32x4*>(st_w + (16 * rt + r) * SST_P + 16 * ct + 4 * g) = acc[rt][ct];
#pragma unroll
    for (int k = 0; k < 4 * NRT; ++k) {
      const int row = 4 * k + (lane >> 4), col = 4 * (lane & 15);
      const f32x4 x = *reinterpret_cast<const f32x4*>(st_w + row * SST_P + col);
      if (packed)
        *reinterpret_cast<u32x3a*>(reinterpret_cast<char*>(dst) + pk24_offset(row0 + row, v0 + col, DQKf)) = pack24(x);
      else
        *reinterpret_cast<f32x4*>(dst + (size_t)(row0 + row) * DV + v0 + col) = x;
    }
  };
  // slot j of this head: float32 [DQKf][DV], or its pack24 form in the first 3/4 of that room
  auto slot_ptr = [&](int j) {
    const size_t off = ((size_t)bh * nslots + j) * DQKf * DV;
    return PK ? reinterpret_cast<float*>(reinterpret_cast<char*>(Sst) + 3 * off) : Sst + off;
  };
  // n (forward, the first column tile's workgroups, which write whole n rows): one more 16 x 16
  // accumulator tile per row tile, whose A operand is columns 64.. of the staged hi rows: coef_t
  // hi in column 64, lo in column 65, zeros after; n[row 16 rt + r] = elements 0 + 1 of lane
  // (0, r)
  const bool owns_n = !REV && vt == 0;  // workgroup-uniform
  f32x4 accN[NRT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
    accN[rt] = f32x4{(owns_n && n0 && g == 0) ? n0[(size_t)bh * DQKf + row0 + 16 * rt + r] : 0.f, 0.f, 0.f, 0.f};
  auto store_n = [&](float* dst) {  // dst: this head's DQKf values
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
      if (g == 0) dst[row0 + 16 * rt + r] = accN[rt][0] + accN[rt][1];
  };
  if (owns_n)
    for (int p = tid; p < L * 16; p += 256) sYh[(p >> 4) * SB_YP + SC_V + (p & 15)] = bf16_t{0};
  float m = (!REV && m0) ? m0[bh] : 0.f;

  u32x4 px[NXP], py[NYP];
  // the chunk's gate prefix (bw_gate_prep_kernel): for this thread's staged tokens a (forward) or
  // b (reverse, with the token's stats), the chunk's gl and max a, and (forward, n column pair)
  // a of token tid
  float ga[NYP], gvm[NYP], gvn[NYP], gl = 0.f, gam = 0.f, gan = 0.f, pmp = 0.f;
  auto fetch = [&](int kc) {
    const size_t t0 = (size_t)bh * S + (size_t)kc * L;
#pragma unroll
    for (int u = 0; u < NXP; ++u) {
      const int p = u * 256 + tid;
      if (NX % 256 == 0 || p < NX)
        px[u] = *reinterpret_cast<const u32x4*>(X + (t0 + p / PRX) * DQKf + d_off + (p % PRX) * 8);
    }
#pragma unroll
    for (int u = 0; u < NYP; ++u) {
      const int p = u * 256 + tid;
      if (NY % 256 == 0 || p < NY) py[u] = *reinterpret_cast<const u32x4*>(Y + (t0 + p / PRY) * DV + v0 + (p % PRY) * 8);
    }
    const float* gb = gp + ((size_t)bh * NC + kc) * GP_STRIDE;
#pragma unroll
    for (int u = 0; u < NYP; ++u) {
      const int t = (u * 256 + tid) / PRY;
      if (NY % 256 == 0 || t < L) {
        if (REV && PK) {  // b - m_comb and qk_scale / divisor, from the stats pass
          ga[u] = gb[64 + t];
          gvn[u] = gb[132 + t];
        } else {
          ga[u] = REV ? gb[t] : gb[64 + t];
          if (REV) {
            gvm[u] = vm[t0 + t];
            gvn[u] = vn[t0 + t];
          }
        }
      }
    }
    gl = gb[128];
    if (!REV) {
      gam = gb[129];
      if (owns_n && tid < L) gan = gb[64 + tid];
    }
    if (REV) pmp = mst[(size_t)bh * NC + kc];
  };
  float mnext = REV ? mfin[bh] : 0.f;
  fetch(REV ? NC - 1 : 0);
  // this lane's transposed-read addresses: row r / 4 of a 4-row block, columns 4 (r % 4)
  const int kk = r >> 2, ka = r & 3;
  for (int it = 0; it < NC; ++it) {
    const int kc = REV ? NC - 1 - it : it;
    const size_t sidx = (size_t)bh * NC + kc;
    const int slot = REV ? kc + 1 : kc;
    // the chunk's decay and the coefficients of this thread's own tokens: every thread carries
    // the running stabiliser, so no wave scans the gates and no barrier waits for it
    float decay, co[NYP], con = 0.f;
    const float m_in = m;
    if (!REV) {
      const float mn = fmaxf(gl + m, gam);  // fw.py:115
      decay = expf(gl + m - mn);            // fw.py:125
      m = mn;
#pragma unroll
      for (int u = 0; u < NYP; ++u) co[u] = expf(ga[u] - mn);  // fw.py:121
      if (owns_n && tid < L) con = expf(gan - mn);
    } else {
      const float cmp = pmp;
      decay = expf(gl + cmp - mnext);  // bw.py:86-89
      mnext = cmp;
#pragma unroll
      for (int u = 0; u < NYP; ++u)  // bw.py:92-101
        co[u] = PK ? expf(ga[u] + cmp) * gvn[u] : expf(ga[u] + cmp - gvm[u]) * qk_scale / gvn[u];
    }
#pragma unroll
    for (int u = 0; u < NXP; ++u) {
      const int p = u * 256 + tid;
      if (NX % 256 == 0 || p < NX) *reinterpret_cast<u32x4*>(sX + (p / PRX) * XP + (p % PRX) * 8) = px[u];
    }
#pragma unroll
    for (int u = 0; u < NYP; ++u) {
      const int p = u * 256 + tid;
      if (NY % 256 == 0 || p < NY) {
        const int t = p / PRY, c = (p % PRY) * 8;
        Piece16<bf16_t> pc;
        pc.raw = py[u];
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = co[u] * to_f32(pc.v[e]);
        u32x4 h, l;
        split_bf(x, h, l);
        *reinterpret_cast<u32x4*>(sYh + t * SB_YP + c) = h;
        *reinterpret_cast<u32x4*>(sYl + t * SB_YP + c) = l;
      }
    }
    if (owns_n && tid < L) {  // the n column pair
      const uint32_t h = pk_bf(con, 0.f);
      *reinterpret_cast<uint32_t*>(sYh + tid * SB_YP + SC_V) = (h & 0xffffu) | (pk_bf(con - bf_l(h), 0.f) << 16);
    }
    if (it + 1 < NC) fetch(REV ? kc - 1 : kc + 1);
    __syncthreads();
    store_state(slot_ptr(slot), PK);
    if (owns_n) store_n(nst + sidx * DQKf);
    if (!REV && vt == 0 && rs == 0 && tid == 0) mst[sidx] = m_in;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) acc[rt][ct] *= decay;
      accN[rt] *= decay;
    }
#pragma unroll
    for (int ks = 0; ks < L / 32; ++ks) {
      const int t1 = 32 * ks + 4 * g + kk, t2 = t1 + 16;
      bfx8 a[NRT];
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        const int c = (row0 - d_off) + 16 * rt + 4 * ka;
        a[rt] = tr_pair(sX + t1 * XP + c, sX + t2 * XP + c);
      }
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int c = 16 * ct + 4 * ka;
        const bfx8 bh8 = tr_pair(sYh + t1 * SB_YP + c, sYh + t2 * SB_YP + c);
        const bfx8 bl8 = tr_pair(sYl + t1 * SB_YP + c, sYl + t2 * SB_YP + c);
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {  // D[column][row] += (hi + lo)[T][column] X[T][row]
          acc[rt][ct] = mfma_bf(bh8, a[rt], acc[rt][ct]);
          acc[rt][ct] = mfma_bf(bl8, a[rt], acc[rt][ct]);
        }
      }
      if (owns_n) {  // n' = decay n + sum_t coef_t k_t (fw.py:133)
        const int c = SC_V + 4 * ka;
        const bfx8 bn = tr_pair(sYh + t1 * SB_YP + c, sYh + t2 * SB_YP + c);
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) accN[rt] = mfma_bf(bn, a[rt], accN[rt]);
      }
    }
    __syncthreads();
  }
  if (!REV) {  // the final state (the forward's last states may not be asked for)
    if (sfin) store_state(sfin + (size_t)bh * DQKf * DV, false);
    if (owns_n && nfin) store_n(nfin + (size_t)bh * DQKf);
    if (vt == 0 && rs == 0 && tid == 0 && mfin) mfin[bh] = m;
  } else {
    store_state(slot_ptr(0), PK);
    if (s_init) store_state(s_init + (size_t)bh * DQKf * DV, false);
  }
}

// ---------------------------------------------------------------- launchers
struct BwArgs {
  ChunkwiseArgs fw;
  const void* dh;
  const float* dc_last;
  void *dq, *dk, *dv, *di, *df;
  float* dc0;
};

// ------------------------------------------------------- MFMA dV pass (4)
// dV on v_mfma_f32_16x16x4f32 for 16-bit q/k/v/dH and 64-token chunks: one workgroup of
// 4 waves per (head, chunk, 64 columns of DV) as in bw_dv_kernel.  Wave w owns columns
// [16 w, 16 w + 16) of the tile and the j-tile w of Sbar, for all 64 tokens (4 row tiles):
//   over DQK in blocks of 64 (K and Q of the block staged in LDS, the dC_k column values
//   of a lane and the next block's tiles loaded a block ahead), 4 d per MFMA:
//     A = K[t][d], B = Q[16 w + r][d] (Sbar^T) and dC_k[d][v] (the inter term);
//   Sbar^T gated (fw.py:204-227) into LDS; dV rows scaled by Abar_t (bw.py:179);
//   over j: A = Sbar^T[t][j] (LDS), B = dH[j][v] / (N_j + eps) (bw.py:156).
// Lane (g, r) ends with dV[16 tt + 4 g + e][16 w + r]; the v . dV partials of dI are summed
// over the 16 lanes of a column group, then over the 4 waves in LDS.
constexpr int DVM_P = 72;   // elements per staged 64-wide 16-bit row (36 mod 64 dwords)
constexpr int DVM_SP = 68;  // floats per row of the staged Sbar^T

template <typename TQ, typename TG, int NRT>
__global__ __launch_bounds__(256) void bw_dv_mfma_kernel(const TQ* __restrict__ q, const TQ* __restrict__ k,
                                                          const TQ* __restrict__ v, const TQ* __restrict__ dh,
                                                          const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                          const float* __restrict__ mst,
                                                          const float* __restrict__ mfin,
                                                          const float* __restrict__ vm,
                                                          const float* __restrict__ vn,
                                                          const float* __restrict__ dCst, TQ* __restrict__ dv,
                                                          float* __restrict__ dip, int NC, int DV, int nvt,
                                                          float qk_scale) {
  constexpr int L = 64;
  constexpr int DQK = 64 * NRT;
  static_assert(sizeof(TQ) == 2, "16-bit operands");
  __shared__ __attribute__((aligned(16))) TQ sK[L * DVM_P];
  __shared__ __attribute__((aligned(16))) TQ sQ[L * DVM_P];
  __shared__ float sS[L * DVM_SP];
  __shared__ float sb[L], si[L], smc[L], sinv[L], sab[L];
  __shared__ float s_part[4][L];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int per_bh = NC * nvt;
  const int bh = blockIdx.x / per_bh, rem = blockIdx.x - bh * per_bh;
  const int kc = rem / nvt, vt = rem - kc * nvt, v0 = vt * 64;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  // this lane's column of dC_k (the gradient of the state after chunk kc)
  const float* dcol = dCst + ((size_t)bh * (NC + 1) + kc + 1) * DQK * DV + v0 + 16 * w + r;
  // K, Q blocks of 64 x 64: 512 pieces of 16 bytes, 2 per thread; dC values d = db + 4 ks + g
  u32x4 pk[2], pq[2];
  float pc[16];
  auto fetch = [&](int db) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      pk[u] = *reinterpret_cast<const u32x4*>(k + (row0 + t) * DQK + db + c);
      pq[u] = *reinterpret_cast<const u32x4*>(q + (row0 + t) * DQK + db + c);
    }
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) pc[ks] = dcol[(size_t)(db + 4 * ks + g) * DV];
  };
  // the intra term's dH operands, j = 4 ks + g
  float ph[16];
  auto fetch_h = [&]() {
    const TQ* hcol = dh + row0 * DV + v0 + 16 * w + r;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) ph[ks] = to_f32(hcol[(size_t)(4 * ks + g) * DV]);
  };
  chunk_gate_scan<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {
    const float mn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
    smc[tid] = vm[row0 + tid];
    sinv[tid] = 1.0f / vn[row0 + tid];
    sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - mn);  // Abar (bw.py:168-176)
  }
  f32x4 accS[4], accV[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    accS[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    accV[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  fetch(0);
  for (int db = 0; db < DQK; db += 64) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      *reinterpret_cast<u32x4*>(sK + t * DVM_P + c) = pk[u];
      *reinterpret_cast<u32x4*>(sQ + t * DVM_P + c) = pq[u];
    }
    float cc[16];
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) cc[ks] = pc[ks];
    __syncthreads();
    if (db + 64 < DQK) fetch(db + 64);
    else fetch_h();
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const int dd = 4 * ks + g;
      const float bq = to_f32(sQ[(16 * w + r) * DVM_P + dd]);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float a = to_f32(sK[(16 * tt + r) * DVM_P + dd]);
        accS[tt] = mfma4(a, bq, accS[tt]);
        accV[tt] = mfma4(a, cc[ks], accV[tt]);
      }
    }
    __syncthreads();  // the blocks are read; the next staging may overwrite them
  }
  // Sbar^T[t][j] = S[j][t] Dbar[j][t] on t <= j; inter rows scaled by Abar_t
  const int j = 16 * w + r;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * g + e;
      sS[t * DVM_SP + j] = (t <= j) ? accS[tt][e] * qk_scale * expf(sb[j] - sb[t] + si[t] - smc[j]) : 0.f;
      accV[tt][e] *= sab[t];
    }
  __syncthreads();
  // intra: dV[t][v] += sum_j Sbar^T[t][j] dH[j][v] / (N_j + eps)
#pragma unroll
  for (int ks = 0; ks < 16; ++ks) {
    const int j0 = 4 * ks + g;
    const float b = ph[ks] * sinv[j0];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) accV[tt] = mfma4(sS[(16 * tt + r) * DVM_SP + j0], b, accV[tt]);
  }
  // store dV; v . dV partials of dI (bw.py:338)
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * g + e;
      const size_t off = (row0 + t) * DV + v0 + 16 * w + r;
      dv[off] = from_f32<TQ>(accV[tt][e]);
      const float part = sum16(to_f32(v[off]) * accV[tt][e]);
      if (r == 0) s_part[w][t] = part;
    }
  __syncthreads();
  if (tid < L) dip[(row0 + tid) * nvt + vt] = s_part[0][tid] + s_part[1][tid] + s_part[2][tid] + s_part[3][tid];
}

// ---------------------------------------------------- MFMA dQ, dK pass (5)
// dQ and dK on v_mfma_f32_16x16x4f32 for 16-bit q/k/v/dH and 64-token chunks: one workgroup
// of 4 waves per (head, chunk, 64 columns of DQK) as in bw_dqk_kernel.  Wave w owns columns
// [16 w, 16 w + 16) of the tile and the j-tile w of dS~, for all 64 tokens.
//  Phase 1, over DV in blocks of 64 (dH and V staged in LDS, C_{k-1} and dC_k rows from
//  global memory one block ahead), 4 v per MFMA in the order v = 16 g + ks of a block
//  (lane group g, k-step ks; any order of the contraction serves, and this one makes the
//  C / dC operands of a lane 16 consecutive floats):
//    dS~[t][j] = sum_v dH[t][v] V[j][v],  Q~[t][d] = sum_v dH[t][v] C[d][v],
//    K~[t][d] = sum_v V[t][v] dC[d][v].
//  Then dS = dS~ / (N_t + eps) Dbar[t][j] s (bw.py:158-159) into LDS, dQ = Q~ Bbar_t s /
//  (N_t + eps) (bw.py:182), dK = K~ Abar_t (bw.py:181), and phase 2 adds dS K and dS^T Q over
//  the chunk's tokens (bw.py:161-162), K and Q of the tile staged in LDS.
constexpr int DQM_P = 72;   // elements per staged 64-wide bf16 row (144 bytes: 36 mod 64 dwords)
constexpr int DQM_SP = 68;  // floats per staged dS row

template <typename TQ, typename TG, int NRT>
__global__ __launch_bounds__(256) void bw_dqk_mfma_kernel(const TQ* __restrict__ q, const TQ* __restrict__ k,
                                                           const TQ* __restrict__ v, const TQ* __restrict__ dh,
                                                           const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                           const float* __restrict__ Cst,
                                                           const float* __restrict__ mst,
                                                           const float* __restrict__ mfin,
                                                           const float* __restrict__ vm,
                                                           const float* __restrict__ vn,
                                                           const float* __restrict__ dCst, TQ* __restrict__ dq,
                                                           TQ* __restrict__ dk, float* __restrict__ dfp, int NC, int DV,
                                                           int ndt, float qk_scale) {
  constexpr int L = 64;
  constexpr int DQK = 64 * NRT;
  static_assert(sizeof(TQ) == 2, "16-bit operands");
  // phase 1: sA = dH block, sB = V block; phase 2: sA = K tile, sB = Q tile
  __shared__ __attribute__((aligned(16))) TQ sA[L * DQM_P];
  __shared__ __attribute__((aligned(16))) TQ sB[L * DQM_P];
  __shared__ float sdS[L * DQM_SP];
  __shared__ float sb[L], si[L], smc[L], sinv[L], sab[L], sbb[L];
  __shared__ float s_part[4][L];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int per_bh = NC * ndt;
  const int bh = blockIdx.x / per_bh, rem = blockIdx.x - bh * per_bh;
  const int kc = rem / ndt, dt = rem - kc * ndt, d0 = dt * 64;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  const float* crow = Cst + sidx * DQK * DV + (size_t)(d0 + 16 * w + r) * DV;  // C_{k-1} row d
  const float* dcrow = dCst + (((size_t)bh * (NC + 1) + kc + 1) * DQK + d0 + 16 * w + r) * DV;  // dC_k row d
  // 64 x 64 bf16 tiles: 512 pieces of 16 bytes, 2 per thread (rows p / 8, 8 elements at 8 (p % 8))
  u32x4 pa[2], pb[2];
  auto fetch_tiles = [&](const TQ* A, const TQ* Bm, int stride, int col) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      pa[u] = *reinterpret_cast<const u32x4*>(A + (row0 + t) * stride + col + c);
      pb[u] = *reinterpret_cast<const u32x4*>(Bm + (row0 + t) * stride + col + c);
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      *reinterpret_cast<u32x4*>(sA + t * DQM_P + c) = pa[u];
      *reinterpret_cast<u32x4*>(sB + t * DQM_P + c) = pb[u];
    }
  };
  // this lane's C and dC operands of a block: v = vb + 16 g + 0..15
  f32x4 pc[4], pd[4];
  auto fetch_cd = [&](int vb) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      pc[u] = *reinterpret_cast<const f32x4*>(crow + vb + 16 * g + 4 * u);
      pd[u] = *reinterpret_cast<const f32x4*>(dcrow + vb + 16 * g + 4 * u);
    }
  };
  chunk_gate_scan<TG, L>(ig, fg, row0, sb, si);
  if (tid < L) {
    const float mp = mst[sidx];
    const float mn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
    const float mc = vm[row0 + tid];
    smc[tid] = mc;
    sinv[tid] = 1.0f / vn[row0 + tid];
    sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - mn);  // Abar (bw.py:168-176)
    sbb[tid] = expf(sb[tid] + mp - mc) * qk_scale;        // Bbar s (bw.py:175, 182)
  }
  f32x4 accS[4], accQ[4], accK[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    accS[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    accQ[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    accK[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  fetch_tiles(dh, v, DV, 0);
  fetch_cd(0);
  for (int vb = 0; vb < DV; vb += 64) {
    store_tiles();
    const f32x4 cc[4] = {pc[0], pc[1], pc[2], pc[3]}, cd[4] = {pd[0], pd[1], pd[2], pd[3]};
    __syncthreads();
    if (vb + 64 < DV) {
      fetch_tiles(dh, v, DV, vb + 64);
      fetch_cd(vb + 64);
    } else {  // phase 2's K and Q tiles
      fetch_tiles(k, q, DQK, d0);
    }
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const int vv = 16 * g + ks;
      const float bV = to_f32(sB[(16 * w + r) * DQM_P + vv]);
      const float bC = cc[ks >> 2][ks & 3], bD = cd[ks >> 2][ks & 3];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const float aH = to_f32(sA[(16 * tt + r) * DQM_P + vv]);
        const float aV = to_f32(sB[(16 * tt + r) * DQM_P + vv]);
        accS[tt] = mfma4(aH, bV, accS[tt]);
        accQ[tt] = mfma4(aH, bC, accQ[tt]);
        accK[tt] = mfma4(aV, bD, accK[tt]);
      }
    }
    __syncthreads();  // the blocks are read; the next staging may overwrite them
  }
  // dS into LDS; inter terms scaled
  const int j = 16 * w + r;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * g + e;
      sdS[t * DQM_SP + j] =
          (j <= t) ? accS[tt][e] * sinv[t] * expf(sb[t] - sb[j] + si[j] - smc[t]) * qk_scale : 0.f;
      accQ[tt][e] *= sbb[t] * sinv[t];
      accK[tt][e] *= sab[t];
    }
  store_tiles();  // sA = K[t][d0 ..], sB = Q[t][d0 ..]
  __syncthreads();
  const int dc = 16 * w + r;  // this lane's column of the tile
#pragma unroll 4
  for (int c0 = 0; c0 < L; c0 += 4) {
    const float bK = to_f32(sA[(c0 + g) * DQM_P + dc]);
    const float bQ = to_f32(sB[(c0 + g) * DQM_P + dc]);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      accQ[tt] = mfma4(sdS[(16 * tt + r) * DQM_SP + c0 + g], bK, accQ[tt]);  // dS[t][j] K[j][d]
      accK[tt] = mfma4(sdS[(c0 + g) * DQM_SP + 16 * tt + r], bQ, accK[tt]);  // dS[t][j'] Q[t][d]
    }
  }
  // store dQ, dK; q . dQ - k . dK partials of dF (bw.py:333)
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * g + e;
      const size_t off = (row0 + t) * DQK + d0 + dc;
      dq[off] = from_f32<TQ>(accQ[tt][e]);
      dk[off] = from_f32<TQ>(accK[tt][e]);
      const float part = sum16(to_f32(sB[t * DQM_P + dc]) * accQ[tt][e] - to_f32(sA[t * DQM_P + dc]) * accK[tt][e]);
      if (r == 0) s_part[w][t] = part;
    }
  __syncthreads();
  if (tid < L) dfp[(row0 + tid) * ndt + dt] = s_part[0][tid] + s_part[1][tid] + s_part[2][tid] + s_part[3][tid];
}

// -------------------------------------------------- bf16 MFMA dV pass (4)
// bw_dv_mfma_kernel for bf16 on v_mfma_f32_16x16x32_bf16: the same workgroups and outputs.
// Wave w owns rows [16 w, 16 w + 16) of S[j][t] and columns [16 w, 16 w + 16) of the dV tile.
//   Over DQK in blocks of 64 (K and Q rows and the dC_k block, as bf16 hi / lo rows, staged in
//   LDS from 16-byte loads issued two blocks ahead, together with the gates, stats and the dH
//   block at the start), 32 d per MFMA, lane (g, r) at d = 8 g .. 8 g + 7 of the step:
//     S[j][t] += Q[j][d] K[t][d]            (A = Q rows, B = K rows: one product)
//     dV[t][v] += K[t][d] dC_k[d][v]        (B = dC hi, lo by transposed reads)
//   Sbar^T[t][j] = S[j][t] s Dbar[j][t] / (N_j + eps) on t <= j (fw.py:204-227, bw.py:156)
//   into LDS as bf16 hi / lo rows; dV rows scaled by Abar_t (bw.py:179); then, with the dH
//   block staged in place of K,
//     dV[t][v] += Sbar^T[t][j] dH[j][v]     (A = Sbar^T hi, lo rows; B = dH by transposed reads).
constexpr int BFP = 80;  // bf16 per staged 64-wide row (160 bytes)

template <typename TG, int NRT>
__global__ __launch_bounds__(256, 3) void bw_dv_bf16_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                          const bf16_t* __restrict__ v, const bf16_t* __restrict__ dh,
                                                          const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                          const float* __restrict__ mst,
                                                          const float* __restrict__ mfin,
                                                          const float* __restrict__ vm,
                                                          const float* __restrict__ vn,
                                                          const float* __restrict__ dCst, bf16_t* __restrict__ dv,
                                                          float* __restrict__ dip, int NC, int DV, int nvt,
                                                          float qk_scale) {
  constexpr int L = 64;
  constexpr int DQK = 64 * NRT;
  __shared__ __attribute__((aligned(16))) bf16_t sK[L * BFP];
  __shared__ __attribute__((aligned(16))) bf16_t sV[L * BFP];  // the V tile, for the dI partials
  // the dC_k block [d][v] as bf16 hi / lo rows; after the DQK loop, Sbar^T [t][j] hi / lo
  __shared__ __attribute__((aligned(16))) uint32_t sCh[L * BFP / 2];
  __shared__ __attribute__((aligned(16))) uint32_t sCl[L * BFP / 2];
  uint32_t* const sSh = sCh;
  uint32_t* const sSl = sCl;
  __shared__ float sb[L], si[L], smc[L], sinv[L], sab[L];
  __shared__ float s_part[4][L];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int per_bh = NC * nvt;
  const int blk = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bh = blk / per_bh, rem = blk - bh * per_bh;
  const int kc = rem / nvt, vt = rem - kc * nvt, v0 = vt * 64;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  // dC_k (the gradient of the state after chunk kc), columns v0 .. v0 + 63
  const float* dcb = dCst + ((size_t)bh * (NC + 1) + kc + 1) * DQK * DV + v0;
  // two register slots of a DQK block: K rows (t = p / 8, 8 d at 8 (p % 8)), this lane's Q
  // operands (row 16 w + r, d = 32 ks + 8 g + 0..7: each wave reads only its own rows of Q) and
  // the dC_k block (d = p / 16, 4 v at 4 (p % 16)); block b + 2 is loaded while block b is computed
  u32x4 pk[2][2], pq[2][2];
  f32x4 pc[2][4];
  auto fetch = [&](auto slot, int db) {
    constexpr int sl = decltype(slot)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      pk[sl][u] = *reinterpret_cast<const u32x4*>(k + (row0 + t) * DQK + db + c);
      pq[sl][u] = *reinterpret_cast<const u32x4*>(q + (row0 + 16 * w + r) * DQK + db + 32 * u + 8 * g);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = u * 256 + tid;
      pc[sl][u] = *reinterpret_cast<const f32x4*>(dcb + (size_t)(db + (p >> 4)) * DV + (p & 15) * 4);
    }
  };
  // the intra term's dH block [j][v], staged into sK after the last DQK block, and the V tile
  u32x4 ph[2], pv[2];
  const int kk = r >> 2, ka = r & 3;  // transposed reads: row r / 4 of a 4-row block, columns 4 (r % 4)
  // every load that does not depend on another goes out first: gates, stats, blocks 0 and 1, dH
  float gf = 0.f, gi = 0.f, gvm = 0.f, gvn = 1.f, gmn = 0.f;
  if (tid < L) {
    gf = to_f32(fg[row0 + tid]);
    gi = to_f32(ig[row0 + tid]);
    gvm = vm[row0 + tid];
    gvn = vn[row0 + tid];
    gmn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
  }
  const std::integral_constant<int, 0> S0{};
  const std::integral_constant<int, 1> S1{};
  fetch(S0, 0);
  if (NRT > 1) fetch(S1, 64);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
    ph[u] = *reinterpret_cast<const u32x4*>(dh + (row0 + t) * DV + v0 + c);
    pv[u] = *reinterpret_cast<const u32x4*>(v + (row0 + t) * DV + v0 + c);
  }
  chunk_gate_scan_v<L>(gf, gi, sb, si);
  if (tid < L) {
    smc[tid] = gvm;
    sinv[tid] = 1.0f / gvn;
    sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - gmn);  // Abar (bw.py:168-176)
  }
  f32x4 accS[4], accV[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    accS[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    accV[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto step = [&](auto slot, int bi) {
    constexpr int sl = decltype(slot)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      *reinterpret_cast<u32x4*>(sK + t * BFP + c) = pk[sl][u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = u * 256 + tid, o = ((p >> 4) * BFP + (p & 15) * 4) >> 1;
      const f32x4 x = pc[sl][u];
      const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
      *reinterpret_cast<u32x2*>(sCh + o) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(sCl + o) = u32x2{pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1))};
    }
    const u32x4 qv[2] = {pq[sl][0], pq[sl][1]};  // this block's Q operands, before the slot is reloaded
    __syncthreads();
    if (bi + 2 < NRT) fetch(slot, (bi + 2) * 64);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = 32 * ks + 8 * g;
      // dC_k[d][16 w + r] at d = c + 0..7 (the k of the K operand)
      const int o1 = ((c + kk) * BFP + 16 * w + 4 * ka) >> 1, o2 = o1 + 2 * BFP;
      const bfx8 dch = tr_pair(sCh + o1, sCh + o2), dcl = tr_pair(sCl + o1, sCl + o2);
      const bfx8 qa = __builtin_bit_cast(bfx8, qv[ks]);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const bfx8 kb = ld_bf8(sK + (16 * tt + r) * BFP + c);
        accS[tt] = mfma_bf(qa, kb, accS[tt]);
        accV[tt] = mfma_bf(kb, dch, accV[tt]);
        accV[tt] = mfma_bf(kb, dcl, accV[tt]);
      }
    }
    __syncthreads();  // the blocks are read; the next staging may overwrite them
  };
#pragma unroll
  for (int bi = 0; bi < NRT; bi += 2) {
    step(S0, bi);
    if (bi + 1 < NRT) step(S1, bi + 1);
  }
  // lane (g, r), element e of tile tt: S[j = 16 w + 4 g + e][t = 16 tt + r]
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = 16 * tt + r;
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 16 * w + 4 * g + e;
      x[e] = (t <= j) ? accS[tt][e] * qk_scale * expf(sb[j] - sb[t] + si[t] - smc[j]) * sinv[j] : 0.f;
    }
    const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
    const uint32_t l0 = pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), l1 = pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1));
    const int o = (t * BFP + 16 * w + 4 * g) >> 1;
    *reinterpret_cast<u32x2*>(sSh + o) = u32x2{h0, h1};
    *reinterpret_cast<u32x2*>(sSl + o) = u32x2{l0, l1};
#pragma unroll
    for (int e = 0; e < 4; ++e) accV[tt][e] *= sab[16 * tt + 4 * g + e];
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {  // dH block into sK (read by every wave before the last barrier)
    const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
    *reinterpret_cast<u32x4*>(sK + t * BFP + c) = ph[u];
    *reinterpret_cast<u32x4*>(sV + t * BFP + c) = pv[u];
  }
  __syncthreads();
  // intra: dV[t][v] += sum_j Sbar^T[t][j] dH[j][v]
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int c = 32 * ks + 8 * g + kk;  // dH[j][16 w + r] at j = 32 ks + 8 g + 0..7
    const bfx8 bh8 = tr_pair(sK + c * BFP + 16 * w + 4 * ka, sK + (c + 4) * BFP + 16 * w + 4 * ka);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int o = ((16 * tt + r) * BFP + 32 * ks + 8 * g) >> 1;
      accV[tt] = mfma_bf(ld_bf8(sSh + o), bh8, accV[tt]);
      accV[tt] = mfma_bf(ld_bf8(sSl + o), bh8, accV[tt]);
    }
  }
  // store dV; v . dV partials of dI (bw.py:338)
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * g + e;
      const size_t off = (row0 + t) * DV + v0 + 16 * w + r;
      dv[off] = from_f32<bf16_t>(accV[tt][e]);
      const float part = sum16(to_f32(sV[t * BFP + 16 * w + r]) * accV[tt][e]);
      if (r == 0) s_part[w][t] = part;
    }
  __syncthreads();
  if (tid < L) dip[(row0 + tid) * nvt + vt] = s_part[0][tid] + s_part[1][tid] + s_part[2][tid] + s_part[3][tid];
}

// ---------------------------------------------- bf16 MFMA dQ, dK pass (5)
// bw_dqk_mfma_kernel for bf16 on v_mfma_f32_16x16x32_bf16: the same workgroups and outputs.
// Wave w owns rows [16 w, 16 w + 16) of dS~[j][t] and columns [16 w, 16 w + 16) of the DQK tile.
//  Phase 1, over DV in blocks of 64 (dH and V rows staged in LDS; the lane's C_{k-1} and dC_k
//  row pieces in registers; loads issued two blocks ahead, the first two with the gates and
//  stats at the start), 32 v per MFMA, lane (g, r) at v = 8 g .. 8 g + 7 of the step:
//    dS~[j][t] += V[j][v] dH[t][v]     (A = V rows, B = dH rows: one product)
//    Q~[t][d]  += dH[t][v] C[d][v]     (B = C hi, lo)
//    K~[t][d]  += V[t][v] dC[d][v]     (B = dC hi, lo)
//  dS[t][j] = dS~ / (N_t + eps) Dbar[t][j] s on j <= t (bw.py:158-159) into LDS as bf16 hi / lo
//  rows, dQ = Q~ Bbar_t s / (N_t + eps) (bw.py:182), dK = K~ Abar_t (bw.py:181); phase 2, K and
//  Q rows of the tile staged, 32 tokens per MFMA at j = 4 g + 0..3 and 16 + 4 g + 0..3 of the
//  step (bw.py:161-162):
//    dQ[t][d] += dS[t][j] K[j][d]      (A = dS rows hi, lo; B = K by transposed reads)
//    dK[t][d] += dS[j][t] Q[j][d]      (A = dS columns hi, lo by transposed reads; B = Q likewise)
template <typename TG, int NRT>
__global__ __launch_bounds__(256, 2) void bw_dqk_bf16_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                           const bf16_t* __restrict__ v, const bf16_t* __restrict__ dh,
                                                           const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                           const float* __restrict__ Cst,
                                                           const float* __restrict__ mst,
                                                           const float* __restrict__ mfin,
                                                           const float* __restrict__ vm,
                                                           const float* __restrict__ vn,
                                                           const float* __restrict__ dCst, bf16_t* __restrict__ dq,
                                                           bf16_t* __restrict__ dk, float* __restrict__ dfp, int NC,
                                                           int DV, int ndt, float qk_scale) {
  constexpr int L = 64;
  constexpr int DQK = 64 * NRT;
  // phase 1: sA = dH block, sB = V block; phase 2: sA = K tile, sB = Q tile
  __shared__ __attribute__((aligned(16))) bf16_t sA[L * BFP];
  __shared__ __attribute__((aligned(16))) bf16_t sB[L * BFP];
  __shared__ __attribute__((aligned(16))) bf16_t sDh[L * BFP];
  __shared__ __attribute__((aligned(16))) bf16_t sDl[L * BFP];
  __shared__ float sb[L], si[L], smc[L], sinv[L], sab[L], sbb[L];
  __shared__ float s_part[4][L];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int per_bh = NC * ndt;
  const int blk = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bh = blk / per_bh, rem = blk - bh * per_bh;
  const int kc = rem / ndt, dt = rem - kc * ndt, d0 = dt * 64;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  const float* crow = Cst + sidx * DQK * DV + (size_t)(d0 + 16 * w + r) * DV;                    // C_{k-1} row d
  const float* dcrow = dCst + (((size_t)bh * (NC + 1) + kc + 1) * DQK + d0 + 16 * w + r) * DV;  // dC_k row d
  // two register slots of a DV block: dH, V rows (t = p / 8, 8 v at 8 (p % 8)) and this lane's
  // C, dC pieces (v = vb + 32 ks + 8 g + 0..7); block b + 2 is loaded while block b is computed,
  // and phase 2's K and Q tiles go into the slot the last block frees
  u32x4 pa[2][2], pb[2][2];
  f32x4 pc[2][2][2], pd[2][2][2];
  auto fetch = [&](auto slot, int vb) {
    constexpr int sl = decltype(slot)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      pa[sl][u] = *reinterpret_cast<const u32x4*>(dh + (row0 + t) * DV + vb + c);
      pb[sl][u] = *reinterpret_cast<const u32x4*>(v + (row0 + t) * DV + vb + c);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        pc[sl][ks][h] = *reinterpret_cast<const f32x4*>(crow + vb + 32 * ks + 8 * g + 4 * h);
        pd[sl][ks][h] = *reinterpret_cast<const f32x4*>(dcrow + vb + 32 * ks + 8 * g + 4 * h);
      }
  };
  auto fetch_kq = [&](auto slot) {
    constexpr int sl = decltype(slot)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      pa[sl][u] = *reinterpret_cast<const u32x4*>(k + (row0 + t) * DQK + d0 + c);
      pb[sl][u] = *reinterpret_cast<const u32x4*>(q + (row0 + t) * DQK + d0 + c);
    }
  };
  auto store_tiles = [&](auto slot) {
    constexpr int sl = decltype(slot)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * 256 + tid, t = p >> 3, c = (p & 7) * 8;
      *reinterpret_cast<u32x4*>(sA + t * BFP + c) = pa[sl][u];
      *reinterpret_cast<u32x4*>(sB + t * BFP + c) = pb[sl][u];
    }
  };
  const int nb = DV / 64;
  // every load that does not depend on another goes out first: gates, stats, blocks 0 and 1
  float gf = 0.f, gi = 0.f, gvm = 0.f, gvn = 1.f, gmp = 0.f, gmn = 0.f;
  if (tid < L) {
    gf = to_f32(fg[row0 + tid]);
    gi = to_f32(ig[row0 + tid]);
    gvm = vm[row0 + tid];
    gvn = vn[row0 + tid];
    gmp = mst[sidx];
    gmn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
  }
  const std::integral_constant<int, 0> S0{};
  const std::integral_constant<int, 1> S1{};
  fetch(S0, 0);
  if (nb > 1) fetch(S1, 64);
  else fetch_kq(S1);
  chunk_gate_scan_v<L>(gf, gi, sb, si);
  if (tid < L) {
    smc[tid] = gvm;
    sinv[tid] = 1.0f / gvn;
    sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - gmn);  // Abar (bw.py:168-176)
    sbb[tid] = expf(sb[tid] + gmp - gvm) * qk_scale;       // Bbar s (bw.py:175, 182)
  }
  f32x4 accS[4], accQ[4], accK[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    accS[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    accQ[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    accK[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto step = [&](auto slot, int bi) {
    constexpr int sl = decltype(slot)::value;
    store_tiles(slot);
    bfx8 ch[2], cl[2], dch[2], dcl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float x[8], y[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = pc[sl][ks][0][e];
        x[4 + e] = pc[sl][ks][1][e];
        y[e] = pd[sl][ks][0][e];
        y[4 + e] = pd[sl][ks][1][e];
      }
      u32x4 h, l;
      split_bf(x, h, l);
      ch[ks] = __builtin_bit_cast(bfx8, h);
      cl[ks] = __builtin_bit_cast(bfx8, l);
      split_bf(y, h, l);
      dch[ks] = __builtin_bit_cast(bfx8, h);
      dcl[ks] = __builtin_bit_cast(bfx8, l);
    }
    __syncthreads();
    if (bi + 2 < nb) fetch(slot, (bi + 2) * 64);
    else if (bi + 2 == nb) fetch_kq(slot);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = 32 * ks + 8 * g;
      const bfx8 va = ld_bf8(sB + (16 * w + r) * BFP + c);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const bfx8 hb = ld_bf8(sA + (16 * tt + r) * BFP + c);
        const bfx8 vb8 = ld_bf8(sB + (16 * tt + r) * BFP + c);
        accS[tt] = mfma_bf(va, hb, accS[tt]);
        accQ[tt] = mfma_bf(hb, ch[ks], accQ[tt]);
        accQ[tt] = mfma_bf(hb, cl[ks], accQ[tt]);
        accK[tt] = mfma_bf(vb8, dch[ks], accK[tt]);
        accK[tt] = mfma_bf(vb8, dcl[ks], accK[tt]);
      }
    }
    __syncthreads();  // the blocks are read; the next staging may overwrite them
  };
  for (int bi = 0; bi < nb; bi += 2) {
    step(S0, bi);
    if (bi + 1 < nb) step(S1, bi + 1);
  }
  // lane (g, r), element e of tile tt: dS~[j = 16 w + 4 g + e][t = 16 tt + r]
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = 16 * tt + r;
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 16 * w + 4 * g + e;
      x[e] = (j <= t) ? accS[tt][e] * sinv[t] * expf(sb[t] - sb[j] + si[j] - smc[t]) * qk_scale : 0.f;
    }
    const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
    const uint32_t l0 = pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), l1 = pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1));
    const int o = t * BFP + 16 * w + 4 * g;
    *reinterpret_cast<u32x2*>(sDh + o) = u32x2{h0, h1};
    *reinterpret_cast<u32x2*>(sDl + o) = u32x2{l0, l1};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tq = 16 * tt + 4 * g + e;
      accQ[tt][e] *= sbb[tq] * sinv[tq];
      accK[tt][e] *= sab[tq];
    }
  }
  if (nb & 1) store_tiles(S1);  // sA = K[t][d0 ..], sB = Q[t][d0 ..], in the slot block nb - 2 freed
  else store_tiles(S0);
  __syncthreads();
  const int kk = r >> 2, ka = r & 3;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int j1 = 32 * ks + 4 * g + kk, j2 = j1 + 16;  // this lane's transposed-read rows
    const int cd = 16 * w + 4 * ka;
    const bfx8 bK = tr_pair(sA + j1 * BFP + cd, sA + j2 * BFP + cd);  // K[j][d0 + 16 w + r]
    const bfx8 bQ = tr_pair(sB + j1 * BFP + cd, sB + j2 * BFP + cd);  // Q[j][d0 + 16 w + r]
    const int jr = 32 * ks + 4 * g;  // the row pieces: j = jr + 0..3, jr + 16 + 0..3
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int rowo = (16 * tt + r) * BFP + jr;
      const u32x2 h0 = *reinterpret_cast<const u32x2*>(sDh + rowo), h1 = *reinterpret_cast<const u32x2*>(sDh + rowo + 16);
      const u32x2 l0 = *reinterpret_cast<const u32x2*>(sDl + rowo), l1 = *reinterpret_cast<const u32x2*>(sDl + rowo + 16);
      const bfx8 ah = __builtin_bit_cast(bfx8, (u32x4{h0[0], h0[1], h1[0], h1[1]}));
      const bfx8 al = __builtin_bit_cast(bfx8, (u32x4{l0[0], l0[1], l1[0], l1[1]}));
      accQ[tt] = mfma_bf(ah, bK, accQ[tt]);  // dS[t][j] K[j][d]
      accQ[tt] = mfma_bf(al, bK, accQ[tt]);
      const int ct = 16 * tt + 4 * ka;
      const bfx8 th = tr_pair(sDh + j1 * BFP + ct, sDh + j2 * BFP + ct);  // dS[j][16 tt + r]
      const bfx8 tl = tr_pair(sDl + j1 * BFP + ct, sDl + j2 * BFP + ct);
      accK[tt] = mfma_bf(th, bQ, accK[tt]);  // dS[j][t] Q[j][d]
      accK[tt] = mfma_bf(tl, bQ, accK[tt]);
    }
  }
  // store dQ, dK; q . dQ - k . dK partials of dF (bw.py:333)
  const int dc = 16 * w + r;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * tt + 4 * g + e;
      const size_t off = (row0 + t) * DQK + d0 + dc;
      dq[off] = from_f32<bf16_t>(accQ[tt][e]);
      dk[off] = from_f32<bf16_t>(accK[tt][e]);
      const float part = sum16(to_f32(sB[t * BFP + dc]) * accQ[tt][e] - to_f32(sA[t * BFP + dc]) * accK[tt][e]);
      if (r == 0) s_part[w][t] = part;
    }
  __syncthreads();
  if (tid < L) dfp[(row0 + tid) * ndt + dt] = s_part[0][tid] + s_part[1][tid] + s_part[2][tid] + s_part[3][tid];
}

// ------------------------------------------- bf16 MFMA dV, dQ, dK in one pass (4, 5)
// The dV and dQ/dK passes fused per (head, chunk), so C_{k-1} and dC_k stream from HBM once
// (the separate passes read dC_k twice).  One workgroup of 8 waves; every 64 x 64 product is
// 16 tiles of 16 x 16, wave w owning row tile R = w / 2 and column tiles 2 (w % 2) + {0, 1}.
//  * Q and K of the chunk are staged in LDS once; S^T[j][t] = Q[j] . K[t] over DQK, then
//    Sbar^T[t][j] = S s Dbar[j][t] / (N_j + eps) on t <= j (fw.py:204-227, bw.py:156) into LDS
//    as bf16 hi / lo rows.
//  * Over the v-blocks vb (64 columns), dH[:, vb] and V[:, vb] staged once, and in each over the
//    d-tiles dt (64 rows of the state), the blocks C[dt, vb], dC[dt, vb] staged as bf16 hi / lo
//    (their loads issued two blocks ahead, dH and V a v-block ahead):
//      Q~[dt][t][d] += dH[t] . C[d],  K~[dt][t][d] += V[t] . dC[d]    (32 v per MFMA)
//      dV[t][v] += K[t] . dC[:, v]                                   (32 d per MFMA, transposed reads)
//    with, at the first d-tile, the intra term Sbar^T/N dH of the v-block (bw.py:156) in its own
//    accumulator and dS~^T[j][t] += V[j] . dH[t]; after the last d-tile dV of the v-block is
//    Abar_t (bw.py:179) times the inter term plus the intra term, stored with its v . dV partial
//    of dI.
//  * At the end dS = dS~ Dbar s / (N_t + eps) (bw.py:158-159) and, per d-tile,
//      dQ = Q~ Bbar_t s / (N_t + eps) + dS K,  dK = K~ Abar_t + dS^T Q   (bw.py:161-185)
//    stored with their q . dQ - k . dK partial of dF.
// float32 operands enter as bf16 hi / lo pairs, q, k, v, dH once; float32 accumulation.
constexpr int FV_THREADS = 512;
constexpr int FV_TILE = 64 * BFP * 2;  // bytes of one staged 64 x 64 bf16 tile

template <int NDT>
constexpr size_t dvqk_qk_bytes() { return (size_t)64 * (64 * NDT + 16) * 2; }  // one full Q or K tile
template <int NDT>
constexpr size_t dvqk_smem() { return 2 * dvqk_qk_bytes<NDT>() + (size_t)8 * FV_TILE + (size_t)(6 + 16) * 64 * sizeof(float); }

template <typename TG, int NDT, int NVB>
__global__ __launch_bounds__(FV_THREADS) void bw_dvqk_bf16_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ dh, const TG* __restrict__ ig, const TG* __restrict__ fg,
    const float* __restrict__ Cst, const float* __restrict__ mst, const float* __restrict__ mfin,
    const float* __restrict__ vm, const float* __restrict__ vn, const float* __restrict__ dCst,
    bf16_t* __restrict__ dq, bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, float* __restrict__ dfp,
    float* __restrict__ dip, int NC, float qk_scale) {
  constexpr int L = 64, DQK = 64 * NDT, DV = 64 * NVB;
  constexpr int QP = DQK + 16;   // bf16 per staged Q / K row (2 DQK + 32 bytes)
  constexpr int NKQ = DQK / 32;  // 32-deep k-steps over DQK
  constexpr int NQP = L * (DQK / 8) / FV_THREADS;  // 16-byte Q / K pieces per thread
  extern __shared__ __attribute__((aligned(16))) char fv_smem[];
  bf16_t* sQ = reinterpret_cast<bf16_t*>(fv_smem);                                   // Q [t][d]
  bf16_t* sK = reinterpret_cast<bf16_t*>(fv_smem + dvqk_qk_bytes<NDT>());            // K [t][d]
  char* tiles = fv_smem + 2 * dvqk_qk_bytes<NDT>();
  bf16_t* sH = reinterpret_cast<bf16_t*>(tiles);                  // dH[:, vb] [t][v]
  bf16_t* sV = reinterpret_cast<bf16_t*>(tiles + FV_TILE);        // V[:, vb]  [t][v]
  uint32_t* sCh = reinterpret_cast<uint32_t*>(tiles + 2 * FV_TILE);  // C[dt, vb] [d][v] hi / lo
  uint32_t* sCl = reinterpret_cast<uint32_t*>(tiles + 3 * FV_TILE);
  uint32_t* sDh = reinterpret_cast<uint32_t*>(tiles + 4 * FV_TILE);  // dC[dt, vb] [d][v] hi / lo
  uint32_t* sDl = reinterpret_cast<uint32_t*>(tiles + 5 * FV_TILE);
  uint32_t* sBh = reinterpret_cast<uint32_t*>(tiles + 6 * FV_TILE);  // Sbar^T / N [t][j] hi / lo
  uint32_t* sBl = reinterpret_cast<uint32_t*>(tiles + 7 * FV_TILE);
  uint32_t* sSh = sCh;  // dS [t][j] hi / lo, after the last C block
  uint32_t* sSl = sCl;
  float* sb = reinterpret_cast<float*>(tiles + 8 * FV_TILE);
  float* si = sb + L;
  float* smc = si + L;
  float* sinv = smc + L;
  float* sab = sinv + L;
  float* sbb = sab + L;
  float* s_part = sbb + L;  // [8 waves][L] dI partials; then [2][8 waves][L] dF partials, by d-tile parity
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
  const int kk = r >> 2, ka = r & 3;  // transposed reads: row r / 4 of a 4-row block, columns 4 (r % 4)
  const int R = w >> 1, C0 = 2 * (w & 1);
  const int blk = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bh = blk / NC, kc = blk - bh * NC;
  const size_t S = (size_t)NC * L, row0 = (size_t)bh * S + (size_t)kc * L, sidx = (size_t)bh * NC + kc;
  // C_{k-1} and dC_k as pack24 (3 bytes per value)
  const char* cbase = reinterpret_cast<const char*>(Cst) + 3 * (sidx * DQK * DV);
  const char* dcbase = reinterpret_cast<const char*>(dCst) + 3 * (((size_t)bh * (NC + 1) + kc + 1) * DQK * DV);

  // C / dC block (dt, vb) in two register slots (row p / 16, 4 columns at 4 (p % 16)); dH, V of
  // a v-block in one (row tid / 8, 8 columns at 8 (tid % 8))
  u32x3a pc[2][2], pd[2][2];
  u32x4 ph, pv;
  auto fetch = [&](auto slot, int st) {  // block st = vb NDT + dt
    constexpr int sl = decltype(slot)::value;
    if (st >= NDT * NVB) return;
    const int vb = st / NDT, dt = st - vb * NDT;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = u * FV_THREADS + tid;
      const size_t off = pk24_offset(64 * dt + (p >> 4), 64 * vb + (p & 15) * 4, DQK);
      pc[sl][u] = *reinterpret_cast<const u32x3a*>(cbase + off);
      pd[sl][u] = *reinterpret_cast<const u32x3a*>(dcbase + off);
    }
  };
  auto fetch_hv = [&](int vb) {
    if (vb >= NVB) return;
    const int t = tid >> 3, c = (tid & 7) * 8;
    ph = *reinterpret_cast<const u32x4*>(dh + (row0 + t) * DV + 64 * vb + c);
    pv = *reinterpret_cast<const u32x4*>(v + (row0 + t) * DV + 64 * vb + c);
  };
  auto stage4 = [&](uint32_t* th, uint32_t* tl, int p, f32x4 x) {
    const int o = ((p >> 4) * BFP + (p & 15) * 4) >> 1;
    const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
    *reinterpret_cast<u32x2*>(th + o) = u32x2{h0, h1};
    *reinterpret_cast<u32x2*>(tl + o) = u32x2{pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1))};
  };
  const std::integral_constant<int, 0> S0{};
  const std::integral_constant<int, 1> S1{};

  // ---- every independent load first: gates, stats, Q and K of the chunk, blocks 0 and 1, dH / V of vb 0
  float gf = 0.f, gi = 0.f, gvm = 0.f, gvn = 1.f, gmp = 0.f, gmn = 0.f;
  if (tid < L) {
    gf = to_f32(fg[row0 + tid]);
    gi = to_f32(ig[row0 + tid]);
    gvm = vm[row0 + tid];
    gvn = vn[row0 + tid];
    gmp = mst[sidx];
    gmn = (kc + 1 < NC) ? mst[sidx + 1] : mfin[bh];
  }
  {
    u32x4 pq[NQP], pk[NQP];
#pragma unroll
    for (int u = 0; u < NQP; ++u) {
      const int p = u * FV_THREADS + tid, t = p / (DQK / 8), c = (p % (DQK / 8)) * 8;
      pq[u] = *reinterpret_cast<const u32x4*>(q + (row0 + t) * DQK + c);
      pk[u] = *reinterpret_cast<const u32x4*>(k + (row0 + t) * DQK + c);
    }
    fetch(S0, 0);
    fetch(S1, 1);
    fetch_hv(0);
    chunk_gate_scan_v<L>(gf, gi, sb, si);
    if (tid < L) {
      smc[tid] = gvm;
      sinv[tid] = 1.0f / gvn;
      sab[tid] = expf(sb[L - 1] - sb[tid] + si[tid] - gmn);  // Abar (bw.py:168-176)
      sbb[tid] = expf(sb[tid] + gmp - gvm) * qk_scale;       // Bbar s (bw.py:175, 182)
    }
#pragma unroll
    for (int u = 0; u < NQP; ++u) {
      const int p = u * FV_THREADS + tid, t = p / (DQK / 8), c = (p % (DQK / 8)) * 8;
      *reinterpret_cast<u32x4*>(sQ + t * QP + c) = pq[u];
      *reinterpret_cast<u32x4*>(sK + t * QP + c) = pk[u];
    }
  }
  __syncthreads();  // gate rows, stats, Q, K
  {  // S^T[j][t] (A = Q rows j = 16 R + r, B = K rows t), then Sbar^T / N into LDS rows t
    f32x4 Sa[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < NKQ; ++ks) {
      const int c = 32 * ks + 8 * g;
      const bfx8 aq = ld_bf8(sQ + (16 * R + r) * QP + c);
#pragma unroll
      for (int i = 0; i < 2; ++i) Sa[i] = mfma_bf(aq, ld_bf8(sK + (16 * (C0 + i) + r) * QP + c), Sa[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int t = 16 * (C0 + i) + r;
      float x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 16 * R + 4 * g + e;
        x[e] = (t <= j) ? Sa[i][e] * qk_scale * expf(sb[j] - sb[t] + si[t] - smc[j]) * sinv[j] : 0.f;
      }
      const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
      const int o = (t * BFP + 16 * R + 4 * g) >> 1;
      *reinterpret_cast<u32x2*>(sBh + o) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(sBl + o) =
          u32x2{pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1))};
    }
  }

  // ---- accumulators: Q~, K~ of every d-tile (t = 16 R + 4 g + e, d = 64 dt + 16 (C0 + i) + r);
  // dV of the v-block (t as above, v = 64 vb + 16 (C0 + i) + r); dS~^T (j = 16 R + 4 g + e,
  // t = 16 (C0 + i) + r)
  f32x4 Qa[NDT][2], Ka[NDT][2], dSa[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int d = 0; d < NDT; ++d) Qa[d][i] = Ka[d][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    dSa[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  static_for<0, NVB>([&](auto vbc) {
    constexpr int vb = decltype(vbc)::value;
    {  // dH and V of this v-block (every wave is past its last read of them)
      const int t = tid >> 3, c = (tid & 7) * 8;
      *reinterpret_cast<u32x4*>(sH + t * BFP + c) = ph;
      *reinterpret_cast<u32x4*>(sV + t * BFP + c) = pv;
    }
    fetch_hv(vb + 1);
    f32x4 dVa[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    f32x4 dVi[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // the intra term of dV
    static_for<0, NDT>([&](auto dtc) {
      constexpr int dt = decltype(dtc)::value;
      constexpr int st = vb * NDT + dt, sl = st & 1;
      const auto slot = std::integral_constant<int, sl>{};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        stage4(sCh, sCl, u * FV_THREADS + tid, unpack24(pc[sl][u]));
        stage4(sDh, sDl, u * FV_THREADS + tid, unpack24(pd[sl][u]));
      }
      __syncthreads();  // the block's tiles (and, at dt 0, dH / V of the v-block)
      fetch(slot, st + 2);
      if (dt == 0) {  // needing only dH and V: dV intra = Sbar^T / N . dH, dS~ += V . dH (32 j per step),
                      // early, so that the v-block's finish waits on no MFMA chain of its own
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int c = 32 * ks + 8 * g;
          const int ob = ((16 * R + r) * BFP + c) >> 1;
          const bfx8 bh8 = ld_bf8(sBh + ob), bl8 = ld_bf8(sBl + ob);
          const bfx8 av = ld_bf8(sV + (16 * R + r) * BFP + c);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const bfx8 hj = tr_pair(sH + (c + kk) * BFP + 16 * (C0 + i) + 4 * ka, sH + (c + kk + 4) * BFP + 16 * (C0 + i) + 4 * ka);
            dVi[i] = mfma_bf(bh8, hj, dVi[i]);
            dVi[i] = mfma_bf(bl8, hj, dVi[i]);
            dSa[i] = mfma_bf(av, ld_bf8(sH + (16 * (C0 + i) + r) * BFP + c), dSa[i]);
          }
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {  // 32 v per step: Q~ += dH . C, K~ += V . dC
        const int c = 32 * ks + 8 * g;
        const bfx8 ah = ld_bf8(sH + (16 * R + r) * BFP + c);
        const bfx8 av = ld_bf8(sV + (16 * R + r) * BFP + c);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int o = ((16 * (C0 + i) + r) * BFP + c) >> 1;
          Qa[dt][i] = mfma_bf(ah, ld_bf8(sCh + o), Qa[dt][i]);
          Qa[dt][i] = mfma_bf(ah, ld_bf8(sCl + o), Qa[dt][i]);
          Ka[dt][i] = mfma_bf(av, ld_bf8(sDh + o), Ka[dt][i]);
          Ka[dt][i] = mfma_bf(av, ld_bf8(sDl + o), Ka[dt][i]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {  // 32 d per step: dV += K . dC
        const int c = 32 * ks + 8 * g;
        const bfx8 ak = ld_bf8(sK + (16 * R + r) * QP + 64 * dt + c);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int o1 = ((c + kk) * BFP + 16 * (C0 + i) + 4 * ka) >> 1, o2 = o1 + 2 * BFP;
          dVa[i] = mfma_bf(ak, tr_pair(sDh + o1, sDh + o2), dVa[i]);
          dVa[i] = mfma_bf(ak, tr_pair(sDl + o1, sDl + o2), dVa[i]);
        }
      }
      if (dt == NDT - 1) {  // the v-block of dV: Abar times the inter term plus the intra term, store
        // x[i][e]: row 16 R + 4 g + e, column 16 (C0 + i) + r.  Three swaps of a lane bit with a
        // register bit inside each 16 lanes (r bit 0 with e bit 0, r bit 1 with e bit 1, r bit 2
        // with i) leave lane (g, r) with row 16 R + 4 g + (r & 3) and the 8 consecutive columns
        // 16 (C0 + ((r >> 2) & 1)) + 8 (r >> 3) + 4 i + e: one 16-byte store, one 16-byte V read
        float x[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) x[i][e] = dVa[i][e] * sab[16 * R + 4 * g + e] + dVi[i][e];
        // swap of lane bit M with a register bit: the lane with the bit clear keeps register bit 0
        // and takes its partner's register bit 0 into bit 1; the partner the other way round
        auto swap_bit = [&](auto mc, auto ref) {
          constexpr int M = decltype(mc)::value;
          const bool up = (lane & M) != 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float& a = ref(k, 0);
            float& b = ref(k, 1);
            const float y = xor_lane<M>(up ? a : b, lane);
            if (up) a = y; else b = y;
          }
        };
        swap_bit(std::integral_constant<int, 1>{}, [&](int k, int b) -> float& { return x[k >> 1][2 * (k & 1) + b]; });
        swap_bit(std::integral_constant<int, 2>{}, [&](int k, int b) -> float& { return x[k >> 1][(k & 1) + 2 * b]; });
        swap_bit(std::integral_constant<int, 4>{}, [&](int k, int b) -> float& { return x[b][k]; });
        const int t = 16 * R + 4 * g + (r & 3), vc = 16 * (C0 + ((r >> 2) & 1)) + 8 * (r >> 3);
        *reinterpret_cast<u32x4*>(dv + (row0 + t) * DV + 64 * vb + vc) =
            u32x4{pk_bf(x[0][0], x[0][1]), pk_bf(x[0][2], x[0][3]), pk_bf(x[1][0], x[1][1]), pk_bf(x[1][2], x[1][3])};
        // v . dV partial of dI over this v-block (bw.py:338): 8 columns here, the row's other 24 in
        // the lanes r ^ 4, r ^ 8, r ^ 12
        const u32x4 vw = *reinterpret_cast<const u32x4*>(sV + t * BFP + vc);
        float part = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) part += bf_l(vw[k]) * x[k >> 1][2 * (k & 1)] + bf_h(vw[k]) * x[k >> 1][2 * (k & 1) + 1];
        part += xor_lane<4>(part, lane);
        part += xor_lane<8>(part, lane);
        if ((r >> 2) == 0) s_part[w * L + t] = part;
      }
      __syncthreads();  // the block's tiles are read (and, at the last d-tile, dH / V and the dI partials)
      if (dt == NDT - 1 && tid < L)
        dip[(row0 + tid) * NVB + vb] = s_part[(2 * (tid >> 4)) * L + tid] + s_part[(2 * (tid >> 4) + 1) * L + tid];
    });
  });
  // ---- dS = dS~ Dbar s / (N_t + eps) on j <= t into LDS rows t (over the C block buffers)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = 16 * (C0 + i) + r;
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 16 * R + 4 * g + e;
      x[e] = (j <= t) ? dSa[i][e] * sinv[t] * expf(sb[t] - sb[j] + si[j] - smc[t]) * qk_scale : 0.f;
    }
    const uint32_t h0 = pk_bf(x[0], x[1]), h1 = pk_bf(x[2], x[3]);
    const int o = (t * BFP + 16 * R + 4 * g) >> 1;
    *reinterpret_cast<u32x2*>(sSh + o) = u32x2{h0, h1};
    *reinterpret_cast<u32x2*>(sSl + o) =
        u32x2{pk_bf(x[0] - bf_l(h0), x[1] - bf_h(h0)), pk_bf(x[2] - bf_l(h1), x[3] - bf_h(h1))};
  }
  __syncthreads();
  // ---- per d-tile: dQ = Q~ Bbar s / N + dS K, dK = K~ Abar + dS^T Q; store with the dF partials.
  // Each wave passes its 16 x 32 pieces of dQ and dK through its own part of the (now free) dC
  // tiles, so that they leave as 16-byte row pieces instead of 2-byte ones
  bf16_t* const oq = reinterpret_cast<bf16_t*>(sDh);
  bf16_t* const ok = reinterpret_cast<bf16_t*>(sDl);
  static_for<0, NDT>([&](auto dtc) {
    constexpr int dt = decltype(dtc)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * R + 4 * g + e;
        Qa[dt][i][e] *= sbb[t] * sinv[t];
        Ka[dt][i][e] *= sab[t];
      }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {  // 32 j per step
      const int c = 32 * ks + 8 * g;
      const int os = ((16 * R + r) * BFP + c) >> 1;
      const bfx8 sh8 = ld_bf8(sSh + os), sl8 = ld_bf8(sSl + os);  // dS rows t
      const int ot1 = ((c + kk) * BFP + 16 * R + 4 * ka) >> 1, ot2 = ot1 + 2 * BFP;
      const bfx8 th8 = tr_pair(sSh + ot1, sSh + ot2), tl8 = tr_pair(sSl + ot1, sSl + ot2);  // dS[j][t]
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int cd = 64 * dt + 16 * (C0 + i) + 4 * ka;
        const bfx8 kj = tr_pair(sK + (c + kk) * QP + cd, sK + (c + kk + 4) * QP + cd);  // K[j][d]
        const bfx8 qj = tr_pair(sQ + (c + kk) * QP + cd, sQ + (c + kk + 4) * QP + cd);  // Q[j][d]
        Qa[dt][i] = mfma_bf(sh8, kj, Qa[dt][i]);
        Qa[dt][i] = mfma_bf(sl8, kj, Qa[dt][i]);
        Ka[dt][i] = mfma_bf(th8, qj, Ka[dt][i]);
        Ka[dt][i] = mfma_bf(tl8, qj, Ka[dt][i]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * R + 4 * g + e;
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int dc = 64 * dt + 16 * (C0 + i) + r;
        oq[t * BFP + 16 * (C0 + i) + r] = from_f32<bf16_t>(Qa[dt][i][e]);
        ok[t * BFP + 16 * (C0 + i) + r] = from_f32<bf16_t>(Ka[dt][i][e]);
        part += to_f32(sQ[t * QP + dc]) * Qa[dt][i][e] - to_f32(sK[t * QP + dc]) * Ka[dt][i][e];
      }
      part = sum16(part);
      if (r == 0) s_part[(dt & 1) * 8 * L + w * L + t] = part;
    }
    {  // the wave's own rows back out of LDS (no other wave touches them): 8 columns per lane
      const int t = 16 * R + (lane >> 2), c = 16 * C0 + 8 * (lane & 3);
      const size_t off = (row0 + t) * DQK + 64 * dt + c;
      *reinterpret_cast<u32x4*>(dq + off) = *reinterpret_cast<const u32x4*>(oq + t * BFP + c);
      *reinterpret_cast<u32x4*>(dk + off) = *reinterpret_cast<const u32x4*>(ok + t * BFP + c);
    }
    __syncthreads();  // the dF partials of this d-tile
    if (tid < L)
      dfp[(row0 + tid) * NDT + dt] =
          s_part[(dt & 1) * 8 * L + (2 * (tid >> 4)) * L + tid] + s_part[(dt & 1) * 8 * L + (2 * (tid >> 4) + 1) * L + tid];
  });
}


template <typename TQ, typename TG, int L, bool REV, bool PK = false>
int launch_scan(int DQK, const TQ* X, const TQ* Y, const TG* ig, const TG* fg, const float* gp, const float* s0,
                const float* n0, const float* m0, const float* vm, const float* vn, float* Sst, float* nst, float* mst,
                float* sfin, float* nfin, float* mfin, float* s_init, int BNH, int NC, int DV, float qk_scale,
                hipStream_t st) {
  const int nvt = DV / SC_V;
  // 128 state rows per workgroup (64 for DQK 64): two workgroups share a DQK 256 state, so
  // the chunk-sequential scan keeps two waves on every SIMD
  auto go = [&](auto kern, size_t smem, int nrs, auto... gprep) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess)
      return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_bwd: LDS attribute failed: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3((unsigned)(BNH * nvt * nrs)), dim3(256), smem, st, X, Y, ig, fg, gprep..., s0, n0, m0,
                       vm, vn, Sst, nst, mst, sfin, nfin, mfin, s_init, NC, DQK, DV, nvt, qk_scale);
    return check_launch(REV ? "xl_mlstm_chunkwise_bwd(dC scan)" : "xl_mlstm_chunkwise_bwd(states scan)");
  };
  if constexpr (std::is_same<TQ, bf16_t>::value && L % 32 == 0) {  // bf16 operands, static LDS, gate prefix in gp
    if (DQK == 64) return go(bw_scan_bf16_kernel<TG, L, 1, REV, PK>, 0, 1, gp);
    return go(bw_scan_bf16_kernel<TG, L, 2, REV, PK>, 0, DQK / 128, gp);
  } else {
    static_assert(!PK, "pack24 states come from the bf16 scans only");
    if (DQK == 64) return go(bw_scan_kernel<TQ, TG, L, 1, REV>, scan_smem<TQ, L>(1), 1);
    return go(bw_scan_kernel<TQ, TG, L, 2, REV>, scan_smem<TQ, L>(2), DQK / 128);
  }
}

template <typename TQ, typename TG, int L>
int bw_launch(const BwArgs& A, const BwLayout& lay) {
  const ChunkwiseArgs& F = A.fw;
  const int BNH = F.B * F.NH, NC = F.S / L;
  const int ndt = (F.DQK + BW_T - 1) / BW_T, nvt = (F.DV + BW_T - 1) / BW_T;
  char* ws = (char*)F.workspace;
  float *Cst = (float*)(ws + lay.Cst), *nst = (float*)(ws + lay.nst), *mst = (float*)(ws + lay.mst);
  float *cfin = (float*)(ws + lay.cfin), *nfin = (float*)(ws + lay.nfin), *mfin = (float*)(ws + lay.mfin);
  float *vm = (float*)(ws + lay.vm), *vn = (float*)(ws + lay.vn), *dC = (float*)(ws + lay.dC);
  float *dfp = (float*)(ws + lay.dfp), *dip = (float*)(ws + lay.dip), *gpr = (float*)(ws + lay.gprep);
  hipStream_t s = (hipStream_t)F.stream;
  const TQ *q = (const TQ*)F.q, *k = (const TQ*)F.k, *v = (const TQ*)F.v, *dh = (const TQ*)A.dh;
  const TG *ig = (const TG*)F.i, *fg = (const TG*)F.f;
  // the chunk scans on the matrix cores when the state tiles fit their layout
  const bool scan_mfma = F.DV % SC_V == 0 && (F.DQK == 64 || F.DQK == 128 || F.DQK == 256);
  // the fused dV / dQ / dK pass (bf16, 64-token chunks, DV 256 or 512) reads C and dC as pack24
  constexpr bool fused_types = std::is_same<TQ, bf16_t>::value && L == 64;
  const bool fused_dvqk = fused_types && scan_mfma && (F.DV == 256 || F.DV == 512);
  int rc = XL_OK;
  // the bf16 chunk scans take every chunk's gate prefix from gpr
  if constexpr (std::is_same<TQ, bf16_t>::value && L % 32 == 0) {
    if (scan_mfma) {
      hipLaunchKernelGGL((bw_gate_prep_kernel<TG, L>), dim3((unsigned)((BNH * NC + 3) / 4)), dim3(256), 0, s, ig, fg,
                         gpr, BNH * NC);
      if ((rc = check_launch("xl_mlstm_chunkwise_bwd(gate prefix)"))) return rc;
    }
  }
  if constexpr (fused_types) {
    if (fused_dvqk)
      rc = launch_scan<TQ, TG, L, false, true>(F.DQK, k, v, ig, fg, gpr, F.c0, F.n0, F.m0, nullptr, nullptr, Cst, nst,
                                               mst, cfin, nfin, mfin, nullptr, BNH, NC, F.DV, F.qk_scale, s);
  }
  if (!fused_dvqk)
    rc = scan_mfma ? launch_scan<TQ, TG, L, false>(F.DQK, k, v, ig, fg, gpr, F.c0, F.n0, F.m0, nullptr, nullptr, Cst,
                                                   nst, mst, cfin, nfin, mfin, nullptr, BNH, NC, F.DV, F.qk_scale, s)
                   : chunkwise_states_pass(F, Cst, nst, mst, cfin, nfin, mfin);
  if (rc) return rc;
  bool stats_mfma = false;
  if constexpr (std::is_same<TQ, bf16_t>::value && L == 64) {
    stats_mfma = F.DQK == 64 || F.DQK == 128 || F.DQK == 256;
    const dim3 grid((unsigned)(BNH * NC));
    switch (stats_mfma ? F.DQK : 0) {
      case 64: hipLaunchKernelGGL((bw_stats_bf16_kernel<TG, 1>), grid, dim3(256), 0, s, q, k, ig, fg, nst, mst, vm, vn, fused_dvqk ? gpr : nullptr, NC, F.qk_scale, F.eps); break;
      case 128: hipLaunchKernelGGL((bw_stats_bf16_kernel<TG, 2>), grid, dim3(256), 0, s, q, k, ig, fg, nst, mst, vm, vn, fused_dvqk ? gpr : nullptr, NC, F.qk_scale, F.eps); break;
      case 256: hipLaunchKernelGGL((bw_stats_bf16_kernel<TG, 4>), grid, dim3(256), 0, s, q, k, ig, fg, nst, mst, vm, vn, fused_dvqk ? gpr : nullptr, NC, F.qk_scale, F.eps); break;
      default: break;
    }
  }
  if (!stats_mfma)
    hipLaunchKernelGGL((bw_stats_kernel<TQ, TG, L>), dim3((unsigned)(BNH * NC)), dim3(BW_THREADS), 0, s, q, k, ig, fg,
                       nst, mst, vm, vn, NC, F.DQK, F.qk_scale, F.eps);
  if ((rc = check_launch("xl_mlstm_chunkwise_bwd(stats)"))) return rc;
  if constexpr (fused_types) {
    if (fused_dvqk)
      rc = launch_scan<TQ, TG, L, true, true>(F.DQK, q, dh, ig, fg, gpr, A.dc_last, nullptr, nullptr, vm, vn, dC,
                                              nullptr, mst, nullptr, nullptr, mfin, A.dc0, BNH, NC, F.DV, F.qk_scale, s);
  }
  if (fused_dvqk) {
  } else if (scan_mfma) {
    rc = launch_scan<TQ, TG, L, true>(F.DQK, q, dh, ig, fg, gpr, A.dc_last, nullptr, nullptr, vm, vn, dC, nullptr,
                                      mst, nullptr, nullptr, mfin, A.dc0, BNH, NC, F.DV, F.qk_scale, s);
  } else {
    hipLaunchKernelGGL((bw_dC_kernel<TQ, TG, L>), dim3((unsigned)(BNH * ndt * nvt)), dim3(BW_THREADS), 0, s, q, dh,
                       ig, fg, mst, mfin, vm, vn, A.dc_last, dC, A.dc0, NC, F.DQK, F.DV, ndt, nvt, F.qk_scale);
    rc = check_launch("xl_mlstm_chunkwise_bwd(dC)");
  }
  if (rc) return rc;
  // dV, dQ and dK in one pass for bf16 with DV 256 or 512 (C and dC streamed once)
  if constexpr (fused_types) {
    if (fused_dvqk) {
      auto go = [&](auto kern, size_t smem) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess)
          return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_bwd: LDS attribute failed: %s", hipGetErrorString(e));
        hipLaunchKernelGGL(kern, dim3((unsigned)(BNH * NC)), dim3(FV_THREADS), smem, s, q, k, v, dh, ig, fg,
                           Cst, mst, mfin, vm, vn, dC, (bf16_t*)A.dq, (bf16_t*)A.dk, (bf16_t*)A.dv, dfp, dip, NC,
                           F.qk_scale);
        return check_launch("xl_mlstm_chunkwise_bwd(dV, dQ, dK)");
      };
      const bool wide = F.DV == 512;
      switch (F.DQK) {
        case 64: rc = wide ? go(bw_dvqk_bf16_kernel<TG, 1, 8>, dvqk_smem<1>()) : go(bw_dvqk_bf16_kernel<TG, 1, 4>, dvqk_smem<1>()); break;
        case 128: rc = wide ? go(bw_dvqk_bf16_kernel<TG, 2, 8>, dvqk_smem<2>()) : go(bw_dvqk_bf16_kernel<TG, 2, 4>, dvqk_smem<2>()); break;
        default: rc = wide ? go(bw_dvqk_bf16_kernel<TG, 4, 8>, dvqk_smem<4>()) : go(bw_dvqk_bf16_kernel<TG, 4, 4>, dvqk_smem<4>()); break;
      }
      if (rc) return rc;
      hipLaunchKernelGGL((bw_gates_kernel<TG>), dim3((unsigned)(BNH * ((F.S + GSEG - 1) / GSEG))), dim3(256), 0, s,
                         fg, dfp, dip, (TG*)A.di, (TG*)A.df, F.S, ndt, nvt);
      return check_launch("xl_mlstm_chunkwise_bwd(gates)");
    }
  }
  // dV and dQ/dK on the matrix cores for 16-bit operands, 64-token chunks and whole 64-wide tiles
  bool tiles_mfma = false;
  if constexpr (sizeof(TQ) == 2 && L == 64) {
    tiles_mfma = scan_mfma;
    if (tiles_mfma && std::is_same<TQ, bf16_t>::value) {
      const dim3 grid((unsigned)(BNH * NC * nvt));
      const bf16_t *qb = (const bf16_t*)q, *kb = (const bf16_t*)k, *vb = (const bf16_t*)v, *hb = (const bf16_t*)dh;
      switch (F.DQK) {
        case 64: hipLaunchKernelGGL((bw_dv_bf16_kernel<TG, 1>), grid, dim3(256), 0, s, qb, kb, vb, hb, ig, fg, mst, mfin, vm, vn, dC, (bf16_t*)A.dv, dip, NC, F.DV, nvt, F.qk_scale); break;
        case 128: hipLaunchKernelGGL((bw_dv_bf16_kernel<TG, 2>), grid, dim3(256), 0, s, qb, kb, vb, hb, ig, fg, mst, mfin, vm, vn, dC, (bf16_t*)A.dv, dip, NC, F.DV, nvt, F.qk_scale); break;
        default: hipLaunchKernelGGL((bw_dv_bf16_kernel<TG, 4>), grid, dim3(256), 0, s, qb, kb, vb, hb, ig, fg, mst, mfin, vm, vn, dC, (bf16_t*)A.dv, dip, NC, F.DV, nvt, F.qk_scale); break;
      }
    } else if (tiles_mfma) {
      const dim3 grid((unsigned)(BNH * NC * nvt));
      switch (F.DQK) {
        case 64: hipLaunchKernelGGL((bw_dv_mfma_kernel<TQ, TG, 1>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, mst, mfin, vm, vn, dC, (TQ*)A.dv, dip, NC, F.DV, nvt, F.qk_scale); break;
        case 128: hipLaunchKernelGGL((bw_dv_mfma_kernel<TQ, TG, 2>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, mst, mfin, vm, vn, dC, (TQ*)A.dv, dip, NC, F.DV, nvt, F.qk_scale); break;
        default: hipLaunchKernelGGL((bw_dv_mfma_kernel<TQ, TG, 4>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, mst, mfin, vm, vn, dC, (TQ*)A.dv, dip, NC, F.DV, nvt, F.qk_scale); break;
      }
    }
  }
  if (!tiles_mfma) {
    hipLaunchKernelGGL((bw_dv_kernel<TQ, TG, L>), dim3((unsigned)(BNH * NC * nvt)), dim3(BW_THREADS), 0, s, q, k, v,
                       dh, ig, fg, mst, mfin, vm, vn, dC, (TQ*)A.dv, dip, NC, F.DQK, F.DV, nvt, F.qk_scale);
  }
  if ((rc = check_launch("xl_mlstm_chunkwise_bwd(dV)"))) return rc;
  if (tiles_mfma) {
    if constexpr (std::is_same<TQ, bf16_t>::value && L == 64) {
      const dim3 grid((unsigned)(BNH * NC * ndt));
      switch (F.DQK) {
        case 64: hipLaunchKernelGGL((bw_dqk_bf16_kernel<TG, 1>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DV, ndt, F.qk_scale); break;
        case 128: hipLaunchKernelGGL((bw_dqk_bf16_kernel<TG, 2>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DV, ndt, F.qk_scale); break;
        default: hipLaunchKernelGGL((bw_dqk_bf16_kernel<TG, 4>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DV, ndt, F.qk_scale); break;
      }
    } else if constexpr (sizeof(TQ) == 2 && L == 64) {
      const dim3 grid((unsigned)(BNH * NC * ndt));
      switch (F.DQK) {
        case 64: hipLaunchKernelGGL((bw_dqk_mfma_kernel<TQ, TG, 1>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DV, ndt, F.qk_scale); break;
        case 128: hipLaunchKernelGGL((bw_dqk_mfma_kernel<TQ, TG, 2>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DV, ndt, F.qk_scale); break;
        default: hipLaunchKernelGGL((bw_dqk_mfma_kernel<TQ, TG, 4>), grid, dim3(256), 0, s, q, k, v, dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DV, ndt, F.qk_scale); break;
      }
    }
  } else {
    hipLaunchKernelGGL((bw_dqk_kernel<TQ, TG, L>), dim3((unsigned)(BNH * NC * ndt)), dim3(BW_THREADS), 0, s, q, k, v,
                       dh, ig, fg, Cst, mst, mfin, vm, vn, dC, (TQ*)A.dq, (TQ*)A.dk, dfp, NC, F.DQK, F.DV, ndt,
                       F.qk_scale);
  }
  if ((rc = check_launch("xl_mlstm_chunkwise_bwd(dQ, dK)"))) return rc;
  hipLaunchKernelGGL((bw_gates_kernel<TG>), dim3((unsigned)(BNH * ((F.S + GSEG - 1) / GSEG))), dim3(256), 0, s, fg,
                     dfp, dip, (TG*)A.di, (TG*)A.df, F.S, ndt, nvt);
  return check_launch("xl_mlstm_chunkwise_bwd(gates)");
}

template <typename TQ, typename TG>
int bw_l(const BwArgs& A, const BwLayout& lay) {
  switch (A.fw.L) {
    case 16: return bw_launch<TQ, TG, 16>(A, lay);
    case 32: return bw_launch<TQ, TG, 32>(A, lay);
    default: return bw_launch<TQ, TG, 64>(A, lay);
  }
}

template <typename TQ>
int bw_g(const BwArgs& A, const BwLayout& lay) {
  switch (A.fw.dtype_gates) {
    case XL_DTYPE_F32: return bw_l<TQ, float>(A, lay);
    case XL_DTYPE_BF16: return bw_l<TQ, bf16_t>(A, lay);
    default: return bw_l<TQ, f16_t>(A, lay);
  }
}

bool bw_shape_ok(int B, int NH, int S, int DQK, int DV, int L) {
  return B > 0 && NH > 0 && S > 0 && DQK > 0 && DV > 0 && (L == 16 || L == 32 || L == 64) && S % L == 0;
}

}  // namespace
}  // namespace xl

namespace xl {
// The two-pass forward's states pass on the matrix cores: the backward's states scan in forward
// mode (float32 and f16 q/k/v on float32 MFMA; bf16 on bf16 MFMA with the coefficients as hi /
// lo pairs), writing C, n, m entering every chunk and the last states (each may be null).
// Returns 1, launching nothing, where the tiles do not fit (DV % 64, DQK not in {64, 128, 256},
// L not in {16, 32, 64}); otherwise XL_OK or a negative XL_ERR_* code.
int chunkwise_states_mfma(const ChunkwiseArgs& A, float* Cst, float* nst, float* mst, float* gprep) {
  if (A.DV % SC_V != 0 || !(A.DQK == 64 || A.DQK == 128 || A.DQK == 256) || !(A.L == 16 || A.L == 32 || A.L == 64))
    return 1;
  auto go = [&](auto tq, auto tg, auto lc) {
    using TQ = decltype(tq);
    using TG = decltype(tg);
    constexpr int L = decltype(lc)::value;
    const int BNH = A.B * A.NH, NC = A.S / L;
    if constexpr (std::is_same<TQ, bf16_t>::value && L % 32 == 0) {  // the bf16 scan reads the gate prefix
      hipLaunchKernelGGL((bw_gate_prep_kernel<TG, L>), dim3((unsigned)((BNH * NC + 3) / 4)), dim3(256), 0,
                         (hipStream_t)A.stream, (const TG*)A.i, (const TG*)A.f, gprep, BNH * NC);
      if (const int rc = check_launch("xl_mlstm_chunkwise_fwd(gate prefix)")) return rc;
    }
    return launch_scan<TQ, TG, L, false>(A.DQK, (const TQ*)A.k, (const TQ*)A.v, (const TG*)A.i, (const TG*)A.f,
                                         gprep, A.c0, A.n0, A.m0, nullptr, nullptr, Cst, nst, mst, A.c_last,
                                         A.n_last, A.m_last, nullptr, BNH, NC, A.DV, A.qk_scale,
                                         (hipStream_t)A.stream);
  };
  auto by_l = [&](auto tq, auto tg) {
    switch (A.L) {
      case 16: return go(tq, tg, std::integral_constant<int, 16>{});
      case 32: return go(tq, tg, std::integral_constant<int, 32>{});
      default: return go(tq, tg, std::integral_constant<int, 64>{});
    }
  };
  auto by_g = [&](auto tq) {
    switch (A.dtype_gates) {
      case XL_DTYPE_F32: return by_l(tq, float{});
      case XL_DTYPE_BF16: return by_l(tq, bf16_t{});
      default: return by_l(tq, f16_t{});
    }
  };
  switch (A.dtype_qkv) {
    case XL_DTYPE_F32: return by_g(float{});
    case XL_DTYPE_BF16: return by_g(bf16_t{});
    default: return by_g(f16_t{});
  }
}
}  // namespace xl

extern "C" size_t xl_mlstm_chunkwise_bwd_workspace_size(int B, int NH, int S, int DQK, int DV, int L) {
  using namespace xl;
  if (!bw_shape_ok(B, NH, S, DQK, DV, L)) return 0;
  return bw_layout(B, NH, S, DQK, DV, L).total;
}

extern "C" int xl_mlstm_chunkwise_bwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                                      const float* c0, const float* n0, const float* m0, const void* dh,
                                      const float* dc_last, void* dq, void* dk, void* dv, void* di, void* df,
                                      float* dc0, int B, int NH, int S, int DQK, int DV, int L, float qk_scale,
                                      float eps, int dtype_qkv, int dtype_gates, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_mlstm_chunkwise_bwd";
  if (B <= 0 || NH <= 0 || S <= 0 || DQK <= 0 || DV <= 0)
    return set_error(XL_ERR_INVALID_ARG, "%s: dimensions must be positive (B=%d NH=%d S=%d DQK=%d DV=%d)", who, B, NH,
                     S, DQK, DV);
  if (L != 16 && L != 32 && L != 64) return set_error(XL_ERR_UNSUPPORTED, "%s: chunk_size=%d not in {16,32,64}", who, L);
  if (S % L) return set_error(XL_ERR_INVALID_ARG, "%s: Sequence length %d is not divisible by chunk size %d.", who, S, L);
  if (!dtype_ok(dtype_qkv) || !dtype_ok(dtype_gates)) return set_error(XL_ERR_INVALID_ARG, "%s: unknown dtype", who);
  if (!q || !k || !v || !i || !f || !dh || !dq || !dk || !dv || !di || !df)
    return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!((c0 && n0 && m0) || (!c0 && !n0 && !m0)))
    return set_error(XL_ERR_INVALID_ARG, "%s: initial states must be given together", who);
  if (dc0 && !c0) return set_error(XL_ERR_INVALID_ARG, "%s: dc0 asks for the gradient of an initial state not given", who);
  // the tile kernels move q, k, v, dH, dq, dk, dv and the float32 states in 16-byte pieces
  if ((((uintptr_t)q) | ((uintptr_t)k) | ((uintptr_t)v) | ((uintptr_t)dh) | ((uintptr_t)dq) | ((uintptr_t)dk) |
       ((uintptr_t)dv) | ((uintptr_t)c0) | ((uintptr_t)n0) | ((uintptr_t)dc_last) | ((uintptr_t)dc0)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "%s: q, k, v, dh, dq, dk, dv, c0, n0, dc_last and dc0 must be 16-byte aligned",
                     who);
  const long long BNH = (long long)B * NH;
  if (BNH * (S / L) * ((DV + 63) / 64) > 0x7fffffffLL || BNH * (S / L) * ((DQK + 63) / 64) > 0x7fffffffLL)
    return set_error(XL_ERR_INVALID_ARG, "%s: too large", who);
  const BwLayout lay = bw_layout(B, NH, S, DQK, DV, L);
  if (!workspace || workspace_bytes < lay.total)
    return set_error(XL_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", who, lay.total,
                     workspace ? workspace_bytes : (size_t)0);
  if (((uintptr_t)workspace) & 255u) return set_error(XL_ERR_INVALID_ARG, "%s: workspace must be 256-byte aligned", who);
  BwArgs A;
  A.fw = ChunkwiseArgs{q, k, v, i, f, c0, n0, m0, nullptr, nullptr, nullptr, nullptr, B, NH, S, DQK, DV, L,
                       qk_scale, eps, dtype_qkv, dtype_gates, workspace, workspace_bytes, stream, 1};
  A.dh = dh;
  A.dc_last = dc_last;
  A.dq = dq;
  A.dk = dk;
  A.dv = dv;
  A.di = di;
  A.df = df;
  A.dc0 = dc0;
  switch (dtype_qkv) {
    case XL_DTYPE_F32: return bw_g<float>(A, lay);
    case XL_DTYPE_BF16: return bw_g<bf16_t>(A, lay);
    default: return bw_g<f16_t>(A, lay);
  }
}
