// Recurrent mLSTM: one decode step (xl_mlstm_step_fwd) and a whole sequence
// in one launch (xl_mlstm_sequence_fwd).
//
// Reference math (kernel_development/xlstm/mlstm_block/mlstm_recurrent/
// recurrent/native_step.py:69-101), per (b, h) and step t:
//   m' = max(logsig(f) + m, i);  fa = exp(logsig(f) + m - m');  ia = exp(i - m')
//   C' = fa C + ia k v^T;        n' = fa n + ia k
//   h  = (q s)^T C' / (max(|(q s) . n'|, exp(-m')) + eps),   s = qk_scale
// With a 16-bit q the reference rounds q s, k v^T, and the two products
// (q s)^T C'.to(q.dtype) and (q s) . n'.to(q.dtype) to q's dtype
// (native_step.py:78-96); the kernel reproduces those roundings.
//
// Layout (both kernels): one workgroup per (b*NH + h, 64-column tile of DV),
// 1024 threads as 16 column groups (4 consecutive floats each, one 16-byte
// access) x 64 row groups; a thread owns rows d = ty + 64 r of its 4 columns.
// The decode step widens the tile to 256 columns (64 column groups x 16 row
// groups) when DV allows it and that still gives >= 256 workgroups: a wave
// then reads and writes one contiguous 1 KB row piece of C per instruction
// (cfg1: 24.6 us per step against 26.8 us with 64-column tiles; a plain copy
// of the same bytes in the same geometry takes 22.9 us).
// The column partials of (q s)^T C' are reduced across the 64 row groups
// through LDS.  n' is recomputed by every tile of a head (DQK values, L2
// resident) and written by tile 0 only.  In the sequence kernel C' lives in
// registers for the whole sequence (every C byte crosses HBM once per launch),
// the gates of 64 steps are formed together (lane = step), the next
// steps' q, k and v are loaded several steps ahead (a step is far shorter than
// a memory latency), and the LDS buffers alternate with the step's parity, so a
// step costs two workgroup barriers.
#include "common.h"

#include <type_traits>

namespace xl {

constexpr int REC_COLS = 64;       // DV columns per workgroup
constexpr int REC_MAX_DQK = 512;   // rows per thread RPT = DQK / 64 <= 8
// 1024 threads = 16 column groups x 64 row groups
constexpr int STEP_THREADS = 1024;
constexpr int STEP_RG = STEP_THREADS / 16;
constexpr int STEP_COLS_WIDE = 256;  // decode step tile width when DV allows it

// f(integral_constant<int, I>) for I = I0 .. N - 1, unrolled at compile time
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <typename TQ, typename TG, int RPT>
__global__ __launch_bounds__(STEP_THREADS) void mlstm_recurrent_kernel(
    const TQ* __restrict__ q, const TQ* __restrict__ k, const TQ* __restrict__ v,
    const TG* __restrict__ ig, const TG* __restrict__ fg,
    const float* c_old, const float* __restrict__ n_old, const float* __restrict__ m_old,
    TQ* __restrict__ h, float* c_new, float* __restrict__ n_new, float* __restrict__ m_new,
    int S, int DQK, int DV, int ntile, float qk_scale, float eps) {
  constexpr bool LOWP = !is_f32<TQ>::value;
  constexpr int NR = RPT * STEP_RG;                                  // rows covered (>= DQK)
  constexpr int NPT = (NR + STEP_THREADS - 1) / STEP_THREADS;        // n entries per thread (d = tid + 1024 j)
  // double-buffered by step parity: two barriers per step
  __shared__ float s_q[2][NR];
  __shared__ float s_k[2][NR];
  __shared__ float s_red[2][STEP_RG][REC_COLS + 4];
  __shared__ float s_wsum[2][STEP_THREADS / 64];

  const int bh = blockIdx.x / ntile;
  const int tile = blockIdx.x - bh * ntile;
  const int tid = threadIdx.x, lane = tid & 63;
  const int tx = tid & 15, ty = tid >> 4;
  const int col0 = tile * REC_COLS + tx * 4;
  const bool col_ok = col0 < DV;  // DV % 4 == 0, so a group is all in or all out
  const int colc = col_ok ? col0 : 0;
  const size_t cbase = (size_t)bh * DQK * DV;

  // ---- the state: C rows d = ty + 64 r of this thread's 4 columns, n entries, m
  float4 C[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int d = ty + STEP_RG * r;
    C[r] = (c_old && col_ok && d < DQK) ? *reinterpret_cast<const float4*>(c_old + cbase + (size_t)d * DV + col0)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float nst[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int d = tid + STEP_THREADS * j;
    nst[j] = (n_old && d < DQK) ? n_old[(size_t)bh * DQK + d] : 0.f;
  }
  float m = m_old ? m_old[bh] : 0.f;

  // ---- operands of PF steps in flight, raw (converted when used): slot s holds the step t with
  // t % PF == s, loaded PF steps before it runs (a step lasts well under one memory latency)
  constexpr int PF = (RPT <= 2 || (RPT <= 4 && sizeof(TQ) == 2)) ? 8 : 4;  // within 128 VGPRs
  TQ qr[PF][NPT], kr[PF][NPT], vr[PF][4];
  auto fetch = [&](auto sc, int t) {
    constexpr int sl = decltype(sc)::value;
    if (t >= S) return;
    const size_t tok = (size_t)bh * S + t;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int d = tid + STEP_THREADS * j;
      const int dc = d < DQK ? d : 0;
      qr[sl][j] = q[tok * DQK + dc];
      kr[sl][j] = k[tok * DQK + dc];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) vr[sl][j] = v[tok * DV + colc + j];
  };
  static_for<0, PF>([&](auto sc) { fetch(sc, decltype(sc)::value); });

  // ---- gates, 64 steps at a time with lane = step: logsig f and i per lane,
  // the stabiliser m' = max(logsig f + m, i) step by step exactly as the
  // reference forms it (two dependent operations per step, so m is bit-equal
  // to the step recurrence: with 16-bit q the reference rounds q.n' and
  // (q s)^T C' to bf16, and a 1-ulp change of m can flip those roundings),
  // then fa, ia and exp(-m') of every step, read back per step with v_readlane
  float gfa = 0.f, gia = 0.f, gem = 0.f;
  auto step = [&](auto sc, int t) {
    constexpr int sl = decltype(sc)::value;
    const int jg = t & 63;
    if (jg == 0) {  // uniform
      const int tg = t + lane;
      const bool ok = tg < S;
      const size_t gtok = (size_t)bh * S + (ok ? tg : t);
      const float lsf = ok ? round_to<TG>(logsigmoid(to_f32(fg[gtok]))) : 0.f;  // torch keeps logsigmoid in f's dtype
      const float ipre = to_f32(ig[gtok]);
      const int cnt = S - t < 64 ? S - t : 64;
      float mt = 0.f, mc = m;
      for (int j = 0; j < cnt; ++j) {
        mc = fmaxf(lane_of(lsf, j) + mc, lane_of(ipre, j));
        mt = lane == j ? mc : mt;
      }
      float mp = __shfl_up(mt, 1, 64);
      if (lane == 0) mp = m;
      gfa = expf(lsf + mp - mt);
      gia = expf(ipre - mt);
      gem = expf(-mt);
      m = mc;
    }
    const int buf = t & 1;
    const size_t tok = (size_t)bh * S + t;
    float qv[NPT], kv_[NPT], vv[4];
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      qv[j] = to_f32(qr[sl][j]);
      kv_[j] = to_f32(kr[sl][j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) vv[j] = to_f32(vr[sl][j]);
    fetch(sc, t + PF);  // the operands PF steps ahead, into the slot just read
    const float fa = lane_of(gfa, jg), ia = lane_of(gia, jg), emn = lane_of(gem, jg);

    // ---- n', q s and k to LDS, and the partial of (q s) . n'
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int d = tid + STEP_THREADS * j;
      float qs = qv[j] * qk_scale;
      if (LOWP) qs = round_to<TQ>(qs);
      const float kd = kv_[j];
      const bool ok = d < DQK;
      nst[j] = fa * nst[j] + ia * kd;
      part += ok ? qs * (LOWP ? round_to<TQ>(nst[j]) : nst[j]) : 0.f;
      if (d < NR) {
        s_q[buf][d] = ok ? qs : 0.f;
        s_k[buf][d] = ok ? kd : 0.f;
      }
    }
    part = wave_sum_dpp(part);
    if (lane == 63) s_wsum[buf][tid >> 6] = part;
    __syncthreads();  // s_q, s_k, s_wsum of this step ready

    // ---- C' = fa C + ia k v^T in registers, column partials of (q s)^T C'
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int d = ty + STEP_RG * r;
      const float qd = s_q[buf][d], kd = s_k[buf][d];  // 0 past DQK: the row adds nothing
      float kv[4] = {kd * vv[0], kd * vv[1], kd * vv[2], kd * vv[3]};
      if (LOWP) {
        round2_to<TQ>(kv[0], kv[1]);
        round2_to<TQ>(kv[2], kv[3]);
      }
      C[r].x = fa * C[r].x + ia * kv[0];
      C[r].y = fa * C[r].y + ia * kv[1];
      C[r].z = fa * C[r].z + ia * kv[2];
      C[r].w = fa * C[r].w + ia * kv[3];
      float cr[4] = {C[r].x, C[r].y, C[r].z, C[r].w};
      if (LOWP) {
        round2_to<TQ>(cr[0], cr[1]);
        round2_to<TQ>(cr[2], cr[3]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += qd * cr[j];
    }
    *reinterpret_cast<float4*>(&s_red[buf][ty][tx * 4]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();  // s_red of this step ready

    // ---- column c = tid / 16: 16 lanes add 4 row groups each, then a 16-lane DPP sum
    {
      const int c = tid >> 4, pr = tid & 15;
      float hs = (s_red[buf][pr][c] + s_red[buf][pr + 16][c]) + (s_red[buf][pr + 32][c] + s_red[buf][pr + 48][c]);
#define XL_ROW_ADD(CTRL) hs += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(hs), CTRL, 0xf, 0xf, false));
      XL_ROW_ADD(0x111)  // row_shr:1
      XL_ROW_ADD(0x112)  // row_shr:2
      XL_ROW_ADD(0x114)  // row_shr:4
      XL_ROW_ADD(0x118)  // row_shr:8
#undef XL_ROW_ADD
      if (pr == 15 && tile * REC_COLS + c < DV) {
        float qn = 0.f;
#pragma unroll
        for (int w = 0; w < STEP_THREADS / 64; ++w) qn += s_wsum[buf][w];
        if (LOWP) qn = round_to<TQ>(qn);
        const float den = fmaxf(fabsf(qn), emn) + eps;
        if (LOWP) hs = round_to<TQ>(hs);
        h[tok * DV + tile * REC_COLS + c] = from_f32<TQ>(hs / den);
      }
    }
  };
  for (int t0 = 0; t0 < S; t0 += PF)
    static_for<0, PF>([&](auto sc) {
      const int t = t0 + decltype(sc)::value;
      if (t < S) step(sc, t);  // uniform
    });

  // ---- write the state
  if (c_new) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int d = ty + STEP_RG * r;
      if (col_ok && d < DQK) *reinterpret_cast<float4*>(c_new + cbase + (size_t)d * DV + col0) = C[r];
    }
  }
  if (tile == 0) {
    if (n_new) {
#pragma unroll
      for (int j = 0; j < NPT; ++j) {
        const int d = tid + STEP_THREADS * j;
        if (d < DQK) n_new[(size_t)bh * DQK + d] = nst[j];
      }
    }
    if (m_new && tid == 0) m_new[bh] = m;
  }
}

// Single decode step, straight-line.  Every small operand (gates, m, q, k, n,
// v) is requested first and the whole C tile of the thread right behind it;
// the thread then waits for all of it before the first store, so each wave
// reads its C rows and then writes them (measured on MI355X at cfg1: per-wave
// read-then-write phases beat storing each row as it lands by ~2 us of 27).
// q s and k go to LDS once (one element per thread), so the row loop reads
// them as LDS broadcasts.  Workgroups of 1024 threads (16 column groups x 64
// row groups, 4 rows per thread at DQK = 256): at cfg1 this runs as fast as a
// plain copy with the same access pattern, where 256 threads x 16 rows left a
// VALU phase exposed.  Column partials are reduced through LDS as in
// mlstm_recurrent_kernel.
typedef float nt_f4 __attribute__((ext_vector_type(4)));

template <typename TQ, typename TG, int RPT, int COLS>
__global__ __launch_bounds__(STEP_THREADS) void mlstm_step_kernel(
    const TQ* __restrict__ q, const TQ* __restrict__ k, const TQ* __restrict__ v,
    const TG* __restrict__ ig, const TG* __restrict__ fg,
    const float* c_old, const float* __restrict__ n_old, const float* __restrict__ m_old,
    TQ* __restrict__ h, float* c_new, float* __restrict__ n_new, float* __restrict__ m_new,
    int DQK, int DV, int ntile, float qk_scale, float eps) {
  constexpr bool LOWP = !is_f32<TQ>::value;
  constexpr int CG = COLS / 4;              // 16-byte column groups of the tile
  constexpr int RG = STEP_THREADS / CG;     // row groups
  constexpr int NPT = (RPT * RG + STEP_THREADS - 1) / STEP_THREADS;  // n entries per thread (d = tid + 1024 j)
  __shared__ float s_q[RPT * RG];
  __shared__ float s_k[RPT * RG];
  __shared__ float s_red[RG][COLS + 4];
  __shared__ float s_wsum[STEP_THREADS / 64];

  const int bh = blockIdx.x / ntile;
  const int tile = blockIdx.x - bh * ntile;
  const int tid = threadIdx.x;
  const int tx = tid % CG, ty = tid / CG;
  const int col0 = tile * COLS + tx * 4;
  const bool col_ok = col0 < DV;
  const int colc = col_ok ? col0 : 0;  // clamped: every load below is unconditional and in bounds
  const size_t cbase = (size_t)bh * DQK * DV;

  // ---- small operands first (no branches, so the wait counts stay exact)
  const TG fraw = fg[bh], iraw = ig[bh];
  const float mo = m_old[bh];
  const TQ* qp = q + (size_t)bh * DQK;
  const TQ* kp = k + (size_t)bh * DQK;
  TQ qr[NPT], kr[NPT];
  float nr[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int d = tid + STEP_THREADS * j;
    const int dc = d < DQK ? d : 0;
    qr[j] = qp[dc];
    kr[j] = kp[dc];
    nr[j] = n_old[(size_t)bh * DQK + dc];
  }
  TQ vr[4];
  {
    const TQ* vp = v + (size_t)bh * DV + colc;
#pragma unroll
    for (int j = 0; j < 4; ++j) vr[j] = vp[j];
  }
  asm volatile("" ::: "memory");  // keep the small loads ahead of the C stream
  // ---- then the C stream (rows past DQK re-read row 0 and are never stored)
  float4 C[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int d = ty + RG * r;
    const int dc = d < DQK ? d : 0;
    const nt_f4 x = __builtin_nontemporal_load(reinterpret_cast<const nt_f4*>(c_old + cbase + (size_t)dc * DV + colc));
    C[r] = make_float4(x[0], x[1], x[2], x[3]);
  }

  // gates (identical in every thread)
  const float lsf = round_to<TG>(logsigmoid(to_f32(fraw)));
  const float ipre = to_f32(iraw);
  const float mn = fmaxf(lsf + mo, ipre);
  const float fa = expf(lsf + mo - mn);
  const float ia = expf(ipre - mn);

  // n', q s and k to LDS, and the partial of (q s) . n'
  float part = 0.f, nn[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int d = tid + STEP_THREADS * j;
    float qs = to_f32(qr[j]) * qk_scale;
    if (LOWP) qs = round_to<TQ>(qs);
    const float kd = to_f32(kr[j]);
    nn[j] = fa * nr[j] + ia * kd;
    const bool ok = d < DQK;
    part += ok ? qs * (LOWP ? round_to<TQ>(nn[j]) : nn[j]) : 0.f;
    if (d < RPT * RG) {
      s_q[d] = ok ? qs : 0.f;
      s_k[d] = ok ? kd : 0.f;
    }
  }
  part = wave_sum_dpp(part);
  if ((tid & 63) == 63) s_wsum[tid >> 6] = part;
  float vv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) vv[j] = to_f32(vr[j]);
  // the gate and n work above only waited for the small loads; the barrier
  // publishes s_q, s_k and s_wsum without waiting for the C stream, and each
  // wave's read phase of the C stream ends after it (all of the wave's rows
  // land before its first store)
  __syncthreads();  // s_q, s_k, s_wsum ready
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // C' row by row: store as soon as computed, accumulate (q s)^T C'
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int d = ty + RG * r;
    const float qd = s_q[d], kd = s_k[d];  // 0 past DQK: the row adds nothing
    float kv[4] = {kd * vv[0], kd * vv[1], kd * vv[2], kd * vv[3]};
    if (LOWP) {
      round2_to<TQ>(kv[0], kv[1]);
      round2_to<TQ>(kv[2], kv[3]);
    }
    float4 c = C[r];
    c.x = fa * c.x + ia * kv[0];
    c.y = fa * c.y + ia * kv[1];
    c.z = fa * c.z + ia * kv[2];
    c.w = fa * c.w + ia * kv[3];
    if (col_ok && d < DQK) {
      const nt_f4 x = {c.x, c.y, c.z, c.w};
      __builtin_nontemporal_store(x, reinterpret_cast<nt_f4*>(c_new + cbase + (size_t)d * DV + col0));
    }
    float cr[4] = {c.x, c.y, c.z, c.w};
    if (LOWP) {
      round2_to<TQ>(cr[0], cr[1]);
      round2_to<TQ>(cr[2], cr[3]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] += qd * cr[j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) s_red[ty][tx * 4 + j] = acc[j];
  __syncthreads();
  if (tid < COLS && tile * COLS + tid < DV) {
    float qn = 0.f;
#pragma unroll
    for (int w = 0; w < STEP_THREADS / 64; ++w) qn += s_wsum[w];
    if (LOWP) qn = round_to<TQ>(qn);
    const float den = fmaxf(fabsf(qn), expf(-mn)) + eps;
    float hn = 0.f;
#pragma unroll
    for (int r = 0; r < RG; ++r) hn += s_red[r][tid];
    if (LOWP) hn = round_to<TQ>(hn);
    h[(size_t)bh * DV + tile * COLS + tid] = from_f32<TQ>(hn / den);
  }
  if (tile == 0) {  // n' and m' once per head, after the C stream
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int d = tid + STEP_THREADS * j;
      if (d < DQK) n_new[(size_t)bh * DQK + d] = nn[j];
    }
    if (tid == 0) m_new[bh] = mn;
  }
}

// HBM ceiling of the decode step's state stream: mlstm_step_kernel's grid, block,
// thread -> (row, 16-byte column group) map, nontemporal 16-byte loads, barrier,
// whole-tile wait and stores, with its small operands, arithmetic and reductions
// taken out.  c_new may be c_old (the step updates C in place).
template <int RPT, int COLS>
__global__ __launch_bounds__(STEP_THREADS) void step_copy_kernel(const float* c_old, float* c_new, int DQK, int DV,
                                                                 int ntile) {
  constexpr int CG = COLS / 4;
  constexpr int RG = STEP_THREADS / CG;
  const int bh = blockIdx.x / ntile;
  const int tile = blockIdx.x - bh * ntile;
  const int tid = threadIdx.x;
  const int tx = tid % CG, ty = tid / CG;
  const int col0 = tile * COLS + tx * 4;
  const bool col_ok = col0 < DV;
  const int colc = col_ok ? col0 : 0;
  const size_t cbase = (size_t)bh * DQK * DV;
  nt_f4 C[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int d = ty + RG * r;
    const int dc = d < DQK ? d : 0;
    C[r] = __builtin_nontemporal_load(reinterpret_cast<const nt_f4*>(c_old + cbase + (size_t)dc * DV + colc));
  }
  __syncthreads();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int d = ty + RG * r;
    if (col_ok && d < DQK)
      __builtin_nontemporal_store(C[r], reinterpret_cast<nt_f4*>(c_new + cbase + (size_t)d * DV + col0));
  }
}

// The decode step's tile choice: STEP_COLS_WIDE columns (a wave reads and writes whole
// 1 KB row pieces of C) when DV is a multiple of it, that still gives >= 256 workgroups
// and DQK fits 16 rows per thread; else REC_COLS columns.
static bool step_wide(int BNH, int DQK, int DV) {
  constexpr int RGW = STEP_THREADS / (STEP_COLS_WIDE / 4);
  return DV % STEP_COLS_WIDE == 0 && (long long)BNH * (DV / STEP_COLS_WIDE) >= 256 && DQK <= 16 * RGW;
}

template <typename TQ, typename TG>
static int launch_rec_t(const void* q, const void* k, const void* v, const void* i, const void* f,
                        const float* c0, const float* n0, const float* m0, void* h, float* c1, float* n1,
                        float* m1, int BNH, int S, int DQK, int DV, float qk_scale, float eps, hipStream_t s,
                        const char* who) {
  const int ntile = (DV + REC_COLS - 1) / REC_COLS;
  dim3 grid((unsigned)(BNH * ntile));
  if (S == 1 && c0 && n0 && m0 && c1 && n1 && m1) {  // decode step: straight-line kernel
    // tile width: STEP_COLS_WIDE columns (a wave reads and writes whole 1 KB row pieces of C)
    // when DV is a multiple of it, else 64
    constexpr int RGW = STEP_THREADS / (STEP_COLS_WIDE / 4);
    if (step_wide(BNH, DQK, DV)) {
      const int rps = (DQK + RGW - 1) / RGW;
      const dim3 gw((unsigned)(BNH * (DV / STEP_COLS_WIDE)));
#define XL_STEPW_LAUNCH(R)                                                                                     \
  hipLaunchKernelGGL((mlstm_step_kernel<TQ, TG, R, STEP_COLS_WIDE>), gw, dim3(STEP_THREADS), 0, s, (const TQ*)q, \
                     (const TQ*)k, (const TQ*)v, (const TG*)i, (const TG*)f, c0, n0, m0, (TQ*)h, c1, n1, m1,    \
                     DQK, DV, DV / STEP_COLS_WIDE, qk_scale, eps)
      if (rps <= 4) XL_STEPW_LAUNCH(4);
      else if (rps <= 8) XL_STEPW_LAUNCH(8);
      else XL_STEPW_LAUNCH(16);
#undef XL_STEPW_LAUNCH
      return check_launch(who);
    }
    const int rps = (DQK + STEP_RG - 1) / STEP_RG;
#define XL_STEP_LAUNCH(R)                                                                                      \
  hipLaunchKernelGGL((mlstm_step_kernel<TQ, TG, R, REC_COLS>), grid, dim3(STEP_THREADS), 0, s, (const TQ*)q, \
                     (const TQ*)k, (const TQ*)v, (const TG*)i, (const TG*)f, c0, n0, m0, (TQ*)h, c1, n1, m1,    \
                     DQK, DV, ntile, qk_scale, eps)
    if (rps <= 1) XL_STEP_LAUNCH(1);
    else if (rps <= 2) XL_STEP_LAUNCH(2);
    else if (rps <= 4) XL_STEP_LAUNCH(4);
    else XL_STEP_LAUNCH(8);
#undef XL_STEP_LAUNCH
    return check_launch(who);
  }
  const int rps = (DQK + STEP_RG - 1) / STEP_RG;
#define XL_REC_LAUNCH(R)                                                                                       \
  hipLaunchKernelGGL((mlstm_recurrent_kernel<TQ, TG, R>), grid, dim3(STEP_THREADS), 0, s, (const TQ*)q,      \
                     (const TQ*)k, (const TQ*)v, (const TG*)i, (const TG*)f, c0, n0, m0, (TQ*)h, c1, n1, m1,    \
                     S, DQK, DV, ntile, qk_scale, eps)
  if (rps <= 1) XL_REC_LAUNCH(1);
  else if (rps <= 2) XL_REC_LAUNCH(2);
  else if (rps <= 4) XL_REC_LAUNCH(4);
  else XL_REC_LAUNCH(8);
#undef XL_REC_LAUNCH
  return check_launch(who);
}

template <typename TQ>
static int launch_rec_g(int dtg, const void* q, const void* k, const void* v, const void* i, const void* f,
                        const float* c0, const float* n0, const float* m0, void* h, float* c1, float* n1,
                        float* m1, int BNH, int S, int DQK, int DV, float qk_scale, float eps, hipStream_t s,
                        const char* who) {
  switch (dtg) {
    case XL_DTYPE_F32:
      return launch_rec_t<TQ, float>(q, k, v, i, f, c0, n0, m0, h, c1, n1, m1, BNH, S, DQK, DV, qk_scale, eps, s, who);
    case XL_DTYPE_BF16:
      return launch_rec_t<TQ, bf16_t>(q, k, v, i, f, c0, n0, m0, h, c1, n1, m1, BNH, S, DQK, DV, qk_scale, eps, s, who);
    default:
      return launch_rec_t<TQ, f16_t>(q, k, v, i, f, c0, n0, m0, h, c1, n1, m1, BNH, S, DQK, DV, qk_scale, eps, s, who);
  }
}

static int launch_rec(int dtq, int dtg, const void* q, const void* k, const void* v, const void* i, const void* f,
                      const float* c0, const float* n0, const float* m0, void* h, float* c1, float* n1, float* m1,
                      int BNH, int S, int DQK, int DV, float qk_scale, float eps, hipStream_t s, const char* who) {
  switch (dtq) {
    case XL_DTYPE_F32:
      return launch_rec_g<float>(dtg, q, k, v, i, f, c0, n0, m0, h, c1, n1, m1, BNH, S, DQK, DV, qk_scale, eps, s, who);
    case XL_DTYPE_BF16:
      return launch_rec_g<bf16_t>(dtg, q, k, v, i, f, c0, n0, m0, h, c1, n1, m1, BNH, S, DQK, DV, qk_scale, eps, s, who);
    default:
      return launch_rec_g<f16_t>(dtg, q, k, v, i, f, c0, n0, m0, h, c1, n1, m1, BNH, S, DQK, DV, qk_scale, eps, s, who);
  }
}

static int check_rec_args(const char* who, int B, int NH, int S, int DQK, int DV, int dtq, int dtg) {
  if (B <= 0 || NH <= 0 || S <= 0 || DQK <= 0 || DV <= 0)
    return set_error(XL_ERR_INVALID_ARG, "%s: dimensions must be positive (B=%d NH=%d S=%d DQK=%d DV=%d)", who, B,
                     NH, S, DQK, DV);
  if ((long long)B * NH * ((DV + REC_COLS - 1) / REC_COLS) > 0x7fffffffLL)
    return set_error(XL_ERR_INVALID_ARG, "%s: grid too large", who);
  if (DV % 4 != 0) return set_error(XL_ERR_UNSUPPORTED, "%s: DV=%d must be a multiple of 4", who, DV);
  if (DQK > REC_MAX_DQK) return set_error(XL_ERR_UNSUPPORTED, "%s: DQK=%d exceeds %d", who, DQK, REC_MAX_DQK);
  if (!dtype_ok(dtq) || !dtype_ok(dtg)) return set_error(XL_ERR_INVALID_ARG, "%s: unknown dtype", who);
  return XL_OK;
}

}  // namespace xl

extern "C" int xl_mlstm_step_fwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                                 const float* c_old, const float* n_old, const float* m_old, void* h,
                                 float* c_new, float* n_new, float* m_new, int B, int NH, int DQK, int DV,
                                 float qk_scale, float eps, int dtype_qkv, int dtype_gates, void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_mlstm_step_fwd";
  int rc = check_rec_args(who, B, NH, 1, DQK, DV, dtype_qkv, dtype_gates);
  if (rc) return rc;
  if (!q || !k || !v || !i || !f || !c_old || !n_old || !m_old || !h || !c_new || !n_new || !m_new)
    return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if ((((uintptr_t)c_old) | ((uintptr_t)c_new)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "%s: c_old / c_new must be 16-byte aligned", who);
  if (n_new == n_old || m_new == m_old)
    return set_error(XL_ERR_INVALID_ARG, "%s: n_new / m_new must not alias n_old / m_old", who);
  return launch_rec(dtype_qkv, dtype_gates, q, k, v, i, f, c_old, n_old, m_old, h, c_new, n_new, m_new, B * NH, 1,
                    DQK, DV, qk_scale, eps, (hipStream_t)stream, who);
}

extern "C" int xl_mlstm_step_copy_ceiling(const float* c_old, float* c_new, int B, int NH, int DQK, int DV,
                                          void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_mlstm_step_copy_ceiling";
  int rc = check_rec_args(who, B, NH, 1, DQK, DV, XL_DTYPE_F32, XL_DTYPE_F32);
  if (rc) return rc;
  if (!c_old || !c_new) return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if ((((uintptr_t)c_old) | ((uintptr_t)c_new)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "%s: c_old / c_new must be 16-byte aligned", who);
  const int BNH = B * NH;
  const hipStream_t s = (hipStream_t)stream;
  if (step_wide(BNH, DQK, DV)) {
    constexpr int RGW = STEP_THREADS / (STEP_COLS_WIDE / 4);
    const int rps = (DQK + RGW - 1) / RGW;
    const dim3 gw((unsigned)(BNH * (DV / STEP_COLS_WIDE)));
    if (rps <= 4) hipLaunchKernelGGL((step_copy_kernel<4, STEP_COLS_WIDE>), gw, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, DV / STEP_COLS_WIDE);
    else if (rps <= 8) hipLaunchKernelGGL((step_copy_kernel<8, STEP_COLS_WIDE>), gw, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, DV / STEP_COLS_WIDE);
    else hipLaunchKernelGGL((step_copy_kernel<16, STEP_COLS_WIDE>), gw, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, DV / STEP_COLS_WIDE);
    return check_launch(who);
  }
  const int ntile = (DV + REC_COLS - 1) / REC_COLS;
  const dim3 grid((unsigned)(BNH * ntile));
  const int rps = (DQK + STEP_RG - 1) / STEP_RG;
  if (rps <= 1) hipLaunchKernelGGL((step_copy_kernel<1, REC_COLS>), grid, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, ntile);
  else if (rps <= 2) hipLaunchKernelGGL((step_copy_kernel<2, REC_COLS>), grid, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, ntile);
  else if (rps <= 4) hipLaunchKernelGGL((step_copy_kernel<4, REC_COLS>), grid, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, ntile);
  else hipLaunchKernelGGL((step_copy_kernel<8, REC_COLS>), grid, dim3(STEP_THREADS), 0, s, c_old, c_new, DQK, DV, ntile);
  return check_launch(who);
}

extern "C" int xl_mlstm_sequence_fwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                                     const float* c0, const float* n0, const float* m0, void* h, float* c_last,
                                     float* n_last, float* m_last, int B, int NH, int S, int DQK, int DV,
                                     float qk_scale, float eps, int dtype_qkv, int dtype_gates, void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_mlstm_sequence_fwd";
  int rc = check_rec_args(who, B, NH, S, DQK, DV, dtype_qkv, dtype_gates);
  if (rc) return rc;
  if (!q || !k || !v || !i || !f || !h) return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!((c0 && n0 && m0) || (!c0 && !n0 && !m0)))
    return set_error(XL_ERR_INVALID_ARG, "%s: initial states must be given together", who);
  if (!((c_last && n_last && m_last) || (!c_last && !n_last && !m_last)))
    return set_error(XL_ERR_INVALID_ARG, "%s: last states must be requested together", who);
  if ((((uintptr_t)c0) | ((uintptr_t)c_last)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "%s: c0 / c_last must be 16-byte aligned", who);
  if (n_last && (n_last == n0 || m_last == m0))
    return set_error(XL_ERR_INVALID_ARG, "%s: n_last / m_last must not alias n0 / m0", who);
  return launch_rec(dtype_qkv, dtype_gates, q, k, v, i, f, c0, n0, m0, h, c_last, n_last, m_last, B * NH, S, DQK, DV,
                    qk_scale, eps, (hipStream_t)stream, who);
}
