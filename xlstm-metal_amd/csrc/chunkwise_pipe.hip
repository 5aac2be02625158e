// Pipelined single-pass chunkwise mLSTM forward for bf16 q/k/v on gfx950.
//
// Same math, data layout in HBM and work split over the chip as the fused
// kernel (chunkwise_fused.hip): one workgroup = one (b, h) pair x one 64-column
// tile of DV, 4 state waves holding C (DQK x 64, float32) in MFMA accumulators,
// 4 output waves owning 16 output rows each, the chunk math of
// kernel_development/xlstm/mlstm_block/mlstm_chunkwise/vendored/torch/native/
// fw.py:98-143 (inter-chunk recurrence) and :193-245 (outputs).  What differs is
// the schedule of a chunk, which the fused kernel spends mostly in barrier waits
// (its state waves ran q C, the partial stores and the update back to back
// before the output waves could finish a single row).  Here each chunk is two
// phases, one barrier each:
//
//   phase A (after the chunk's tiles are staged):
//     state waves:  partial q C over their rows (bf16 hi + lo of the state,
//                   two MFMAs) -> LDS; then read their K^T operands of the
//                   update into registers (8 x 16 bytes per lane)
//     output waves: alpha' V of the chunk (formed in the previous phase B) ->
//                   LDS, S^T = K Q^T (with q.n from a fifth tile), gating,
//                   M [V | 1]
//   phase B (after the partials are complete):
//     state waves:  renormalise if the chunk asks for it, C += K^T (alpha' V)
//                   from the captured K^T and the alpha' V tile, and the
//                   normaliser n += K^T alpha' on 4 x 4 x 4 MFMA blocks over the
//                   same K^T registers (alpha' as bf16 hi + lo rows) -- the n
//                   rows a state wave carries are its own C rows; n goes to LDS
//                   as bf16 hi | lo rows for the next chunk's q.n
//     output waves: add the four partials, normalise and store h; write the
//                   next chunk's K and V tiles (loaded from HBM a whole chunk
//                   earlier) into LDS; step the gate recurrence (every output
//                   wave; wave 0 writes the next chunk's gate rows) and form
//                   the next chunk's alpha' V in registers from the V pieces
//                   just staged
//
// The update no longer sits between a chunk's partials and its outputs, so the
// output waves' finish overlaps the state waves' update MFMAs, and every LDS
// tile is single-buffered: K and V of the next chunk are written only in
// phase B, after the last reads of the current ones (the state waves took
// their K^T operands in phase A).  The deferred forget rescale (state stored
// as C e^{-G}, renormalised when G < -30), the ragged last chunk, the
// sequence segments and the XCD-aware grid are those of the fused kernel.
#include "fused_common.h"

#include <type_traits>

namespace xl {
namespace fused {
namespace pipe {


constexpr int NOT = 64 * NOW;  // output-wave threads

// The 16-bit element type of q, k, v and h, and of every MFMA operand: bf16 (the reference's
// usual dtype) or f16.  Float32 operands enter as hi + lo pairs of that type (16 or 22
// significant bits).  f16 keeps no deferred forget rescale (RENORM 0: the stored state is
// renormalised at every chunk whose decay is below 1), so that the state, alpha' <= 1 and
// alpha' V stay within f16's range as they do in the reference's f16 arithmetic.
template <typename T> struct Elt;
template <> struct Elt<bf16_t> {
  typedef bf16x8 V8;
  static constexpr uint32_t ONE2 = 0x3f803f80u;  // {1, 1}
  static constexpr float RENORM = fused::RENORM;
  __device__ static f32x4 mma16(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
  __device__ static f32x16 mma32(V8 a, V8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
  __device__ static f32x4 mma4(s16x4 a, s16x4 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack(float lo, float hi) { return pack_bf16(lo, hi); }
  __device__ static float lo(uint32_t w) { return bf_lo(w); }
  __device__ static float hi(uint32_t w) { return bf_hi(w); }
};
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <> struct Elt<f16_t> {
  typedef f16x8 V8;
  static constexpr uint32_t ONE2 = 0x3c003c00u;  // {1, 1}
  static constexpr float RENORM = 0.f;
  __device__ static f32x4 mma16(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
  __device__ static f32x16 mma32(V8 a, V8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
  __device__ static f32x4 mma4(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  __device__ static float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[0]; }
  __device__ static float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[1]; }
};
// hi + lo split of a pair: hi = T(x), lo = T(x - hi) (the subtraction exact in float32)
template <typename E>
__device__ __forceinline__ uint32_t pack_lo_t(uint32_t hi, float x0, float x1) {
  return E::pack(x0 - E::lo(hi), x1 - E::hi(hi));
}
template <typename E>
__device__ __forceinline__ void split8_t(f32x4 a, f32x4 b, typename E::V8& hi, typename E::V8& lo) {
  const u32x4 h = {E::pack(a[0], a[1]), E::pack(a[2], a[3]), E::pack(b[0], b[1]), E::pack(b[2], b[3])};
  const u32x4 l = {pack_lo_t<E>(h[0], a[0], a[1]), pack_lo_t<E>(h[1], a[2], a[3]), pack_lo_t<E>(h[2], b[0], b[1]),
                   pack_lo_t<E>(h[3], b[2], b[3])};
  hi = __builtin_bit_cast(typename E::V8, h);
  lo = __builtin_bit_cast(typename E::V8, l);
}

// Row of the C tile held by row l32 of 32-row tile dt of state wave rows
// [dw0, dw0 + DW): the order of the transposed K^T reads (within each 16 rows,
// row 4a + c holds state row 8 (a & 1) + 4 (a >> 1) + c); the same row as
// accumulator element e of lane half hh where l32 = 8 (e >> 2) + 4 hh + (e & 3).
__device__ __forceinline__ int state_row(int dw0, int dt, int l32) {
  const int x = l32 & 15;
  return dw0 + 32 * dt + 16 * (l32 >> 4) + 8 * ((x >> 2) & 1) + 4 * (x >> 3) + (x & 3);
}

template <typename T, int DQK, bool STATES_ONLY>
__global__ __launch_bounds__(NTHREADS, 1) void chunkwise_pipe_kernel(MainArgs a) {
  using SM = Smem<DQK>;
  using E = Elt<T>;
  typedef typename E::V8 V8;
  constexpr int KPD = SM::KPD;
  constexpr int DW = DQK / NSW;   // C rows per state wave (64 or 32)
  constexpr int NKO = DQK / 32;   // K staging: 16-byte pieces per output thread (64 rows x DQK / 256 threads / 8)
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int ws = w & 3;  // index within the state or output group
  const SegArgs& sg = a.sg;
  const int S = a.S, NC = a.NC, DV = a.DV, BNH = a.BNH, nvtile = a.nvtile;
  // the head's q / k width in memory: DQK, or less (a multiple of DW) with the tile's rows and
  // columns past it zero (state waves past it idle, q and k read as zero there)
  const int dq = a.dq;

  // ---- XCD-aware workgroup -> (head, column tile): consecutive tiles of a head share an XCD
  const int nwg = BNH * nvtile * sg.nseg;
  int lin = blockIdx.x;
  if ((nwg & 7) == 0) lin = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int bhs = lin / nvtile;  // segment * BNH + head
  const int v0 = (lin - bhs * nvtile) * DVT;
  const int seg = bhs / BNH, bh = bhs - seg * BNH;
  const int kc0 = seg * sg.kc_per_seg, kc1 = min(NC, kc0 + sg.kc_per_seg);  // this segment's chunks
  const size_t cst = (size_t)BNH * dq * DV, nst = (size_t)BNH * dq;
  const float* ci = seg == 0 ? a.c0 : (sg.sc ? sg.sc + (seg - 1) * cst : nullptr);
  const float* ni = seg == 0 ? a.n0 : (sg.sn ? sg.sn + (seg - 1) * nst : nullptr);
  const float m_init = seg == 0 ? (a.m0 ? a.m0[bh] : 0.f) : (sg.sm ? sg.sm[(seg - 1) * BNH + bh] : -INFINITY);
  float* ce = sg.ec ? sg.ec + seg * cst : (seg == sg.nseg - 1 ? a.c_last : nullptr);
  float* ne = sg.ec ? sg.en + seg * nst : a.n_last;
  float* me = sg.ec ? sg.em + (size_t)seg * BNH : a.m_last;

  char* kn = smem + SM::KN;
  char* vn = smem + SM::VN;
  char* av = smem + SM::AV;
  float* hp = (float*)(smem + SM::HP);
  bf16_t* nbuf = (bf16_t*)(smem + SM::NB);   // [2][4][NB_PITCH]: n parts entering chunk kc live in buffer kc & 1
  float* gbuf = (float*)(smem + SM::GATES);  // [2][GROWS][64]: rows of chunk kc live in buffer kc & 1

  const bf16_t* qh = a.q + (size_t)bh * S * dq;
  const bf16_t* kh = a.k + (size_t)bh * S * dq;
  const bf16_t* vh = a.v + (size_t)bh * S * DV;
  bf16_t* hh = a.h + (size_t)bh * S * DV;
  // valid rows of chunk kc (0 past the sequence: a chunk past the end gets a buffer resource
  // with no records, so its prefetches return zeros without touching memory; they are issued
  // unconditionally, which keeps the compiler's load counters exact)
  auto rows_of = [&](int kc) { return __builtin_amdgcn_readfirstlane(max(0, min(L, S - kc * L))); };
  auto q_rsrc = [&](int kc) { return chunk_rsrc(qh + (size_t)kc * L * dq, rows_of(kc), dq * 2); };

  if (w < NSW) {
    // =====================================================================
    // state waves: rows [dw0, dw0 + DW) of C and n, stored as C e^{-G}, n e^{-G}
    // =====================================================================
    // 32 x 32 accumulator tiles acc[dt][vt]: lane (hh, l32) holds column
    // 32 vt + l32 and, in element e = 4i + j, state row
    //   dw0 + 32 dt + 16 (i >> 1) + 8 hh + 4 (i & 1) + j,
    // so the 8 elements 8s' .. 8s'+7 of a lane are the 8 consecutive rows
    // 16 s' + 8 hh .. +7 of the tile: a q C k-step of 16 rows is one split of
    // 8 accumulator values per lane and one 16-byte q load.
    constexpr int NDT = DW / 32;   // 32-row tiles per state wave (1 or 2)
    constexpr int QKS = DW / 16;   // 16-deep k-steps of q C over the wave's rows
    const int dw0 = ws * DW;
    const int l32 = lane & 31, hh = lane >> 5;
    const int kk = r16 >> 2, ka = r16 & 3;
    auto srow = [&](int dt, int e) {
      const int i = e >> 2;
      return dw0 + 32 * dt + 16 * (i >> 1) + 8 * hh + 4 * (i & 1) + (e & 3);
    };
    f32x16 acc[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int vt = 0; vt < 2; ++vt)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          acc[dt][vt][e] = (ci && dw0 < dq) ? ci[((size_t)bh * dq + srow(dt, e)) * DV + v0 + 32 * vt + l32] : 0.f;
    // n of state row state_row(dw0, dt, l32): lane halves hh = 0, 1 sum the
    // tokens of their half of every 16-token k-step
    float nacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      nacc[dt] = (ni && hh == 0 && dw0 < dq) ? ni[(size_t)bh * dq + state_row(dw0, dt, l32)] : 0.f;
    // n entering chunk kc as two bf16 rows (hi, lo) of buffer kc & 1 (rows 2, 3 stay zero):
    // the fifth A tile of the output waves' S product
    auto store_nparts = [&](int buf) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const float x = nacc[dt] + __shfl_xor(nacc[dt], 32);
        if (hh == 0) {
          const uint32_t hi = E::pack(x, 0.f);
          bf16_t* nb = nbuf + buf * 4 * SM::NB_PITCH + state_row(dw0, dt, l32);
          reinterpret_cast<uint16_t*>(nb)[0] = (uint16_t)hi;
          reinterpret_cast<uint16_t*>(nb)[SM::NB_PITCH] = (uint16_t)E::pack(x - E::lo(hi), 0.f);
        }
      }
    };
    for (int e = tid; e < 2 * 4 * DQK; e += 64 * NSW) {  // rows 2, 3, and rows 0, 1 past dq
      const int buf = e / (4 * DQK), part = (e / DQK) % 4, d = e % DQK;
      if (part >= 2 || d >= dq) reinterpret_cast<uint16_t*>(nbuf)[(buf * 4 + part) * SM::NB_PITCH + d] = 0;
    }
    if (dw0 >= dq) {
      // state rows past the head's width: zero partials for the output waves' sums, then only
      // the workgroup's barriers (B0, and B2, B1 of every chunk)
      for (int e = lane; e < 64 * HP_PITCH; e += 64) hp[ws * 64 * HP_PITCH + e] = 0.f;
      __syncthreads();  // B0
      for (int kc = kc0; kc < kc1; ++kc) {
        __syncthreads();  // B2
        __syncthreads();  // B1
      }
      return;
    }
    store_nparts(kc0 & 1);

    // q fragments (B operand of the transposed product C^T Q^T): token 32 tt + l32,
    // rows dw0 + 16 s + 8 hh .. +7
    u32x4 Qs[2][QKS];
    const uint32_t qs_off = (uint32_t)((l32 * dq + dw0 + 8 * hh) * 2);
    auto load_qs = [&](int kc) {
      const auto rq = q_rsrc(kc);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int s = 0; s < QKS; ++s)
          Qs[tt][s] = ld16s(rq, qs_off, (uint32_t)((32 * tt * dq + 16 * s) * 2));
    };
    if (!STATES_ONLY) load_qs(kc0);
    __syncthreads();  // B0: tiles, gate rows and n parts of the first chunk

    for (int kc = kc0; kc < kc1; ++kc) {
      const float* gb = gbuf + (kc & 1) * GROWS * 64;
      // ---------------- phase A: partial q C; the update's K^T and alpha' operands are
      // requested first and consumed in phase B, so their LDS latency hides behind q C.
      // K^T: A = K^T, row l32 of tile dt = state row state_row(dw0, dt, l32), 16-token
      // k-steps, tokens 16 ks + 8 hh + jj (jj = 0..7 in element order).  Transposed
      // reads: within 16 lanes, source lane 4kk + a reads token 16 ks + 8 hh + kk (+4
      // for the second read) at 4 consecutive columns.
      V8 Kt[NDT][4];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const char* base = kn + (16 * ks + 8 * hh + kk) * SM::KN_PITCH +
                             2 * (dw0 + 32 * dt + 16 * (g & 1) + 8 * (ka & 1) + 4 * (ka >> 1));
          Kt[dt][ks] = __builtin_bit_cast(V8, tr8(base, base + 4 * SM::KN_PITCH));
        }
      // A operand of the n update (4 x 4 x 4 MFMA blocks of 4 lanes): lane 4b + m holds
      // alpha' of tokens 16 ks + 8 hh + 4 j .. +3 as bf16 hi (m = 0), lo (m = 1) or zeros
      // (m = 2, 3), the 4 lanes of a block sharing hh
      s16x4 an[4][2];
      {
        const char* ab = reinterpret_cast<const char*>(gb + 384) + 128 * min(lane & 3, 2) + 16 * hh;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int j = 0; j < 2; ++j) an[ks][j] = *reinterpret_cast<const s16x4*>(ab + 32 * ks + 8 * j);
      }
      if (!STATES_ONLY) {
        // Transposed product C^T Q^T per 32-column tile vt: lane (hh, l32) gets
        // columns 32 vt + 8i + 4hh + j of token 32 tt + l32.  The split of k-step
        // q+1 (VALU) is interleaved with the four MFMAs of k-step q, and the
        // partials of column tile 0 are stored one k-step into tile 1.
        constexpr int NQ = 2 * QKS;
        V8 bsp[2][2];
        f32x16 P[2][2];
        auto split_q = [&](int qi, V8 (&o)[2]) {
          const int vt = qi / QKS, s = qi % QKS;
          const f32x16& x = acc[s >> 1][vt];
          const int e0 = 8 * (s & 1);
          split8_t<E>(f32x4{x[e0], x[e0 + 1], x[e0 + 2], x[e0 + 3]}, f32x4{x[e0 + 4], x[e0 + 5], x[e0 + 6], x[e0 + 7]},
                 o[0], o[1]);
        };
        auto store_p = [&](int vt) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              *reinterpret_cast<f32x4*>(hp + (ws * 64 + 32 * tt + l32) * HP_PITCH + hp_col(8 * vt + 2 * i + hh)) =
                  f32x4{P[vt][tt][4 * i], P[vt][tt][4 * i + 1], P[vt][tt][4 * i + 2], P[vt][tt][4 * i + 3]};
        };
        split_q(0, bsp[0]);
#pragma unroll
        for (int qi = 0; qi < NQ; ++qi) {
          const int cur = qi & 1, vt = qi / QKS, s = qi % QKS;
          if (qi + 1 < NQ) split_q(qi + 1, bsp[cur ^ 1]);
          if (s == 0) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) P[vt][tt] = f32x16{};
          }
#pragma unroll
          for (int hl = 0; hl < 2; ++hl)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
              P[vt][tt] = E::mma32(bsp[cur][hl], __builtin_bit_cast(V8, Qs[tt][s]), P[vt][tt]);
          if (vt == 1 && s == 1) {
            store_p(0);
            __builtin_amdgcn_sched_barrier(0);  // keep these stores here, behind the MFMAs of tile 1
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
          }
        }
        store_p(1);
        load_qs(kc + 1);
      }
      __syncthreads();  // B2: partials and alpha' V of the chunk are complete

      // ---------------- phase B: the chunk update of C and n
      V8 avh[2][2], avl[2][2];
      auto load_av = [&](int ks, int buf) {
#pragma unroll
        for (int vt = 0; vt < 2; ++vt) {
          const char* base = av + (16 * ks + 8 * hh + kk) * AV_PITCH + 2 * (32 * vt + 16 * (g & 1) + 4 * ka);
          avh[buf][vt] = __builtin_bit_cast(V8, tr8(base, base + 4 * AV_PITCH));
          avl[buf][vt] = __builtin_bit_cast(V8, tr8(base + 128, base + 128 + 4 * AV_PITCH));
        }
      };
      load_av(0, 0);
      if (gb[323] != 0.f) {  // renormalise the stored state (wave-uniform)
        const float sc = gb[320];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          nacc[dt] *= sc;
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) acc[dt][vt] *= sc;
        }
      }
      // C += K^T (alpha' V), B = alpha' V hi / lo (column 32 vt + l32, the same token
      // order as K^T), one k-step of operands ahead; and n += K^T alpha' on 4 x 4 x 4
      // MFMA blocks: B = 4 tokens of the lane's own K^T row (column n of block b is lane
      // 4b + n), A = alpha' hi / lo rows, so element m of the lane's result is
      // sum_t alpha'_{hi,lo}(t) K(t, row): products exact in float32, float32 sums
      f32x4 nd[NDT];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) nd[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) load_av(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int vt = 0; vt < 2; ++vt)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            acc[dt][vt] = E::mma32(Kt[dt][ks], avh[ks & 1][vt], acc[dt][vt]);
            acc[dt][vt] = E::mma32(Kt[dt][ks], avl[ks & 1][vt], acc[dt][vt]);
          }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const u32x4 kt = __builtin_bit_cast(u32x4, Kt[dt][ks]);
#pragma unroll
          for (int j = 0; j < 2; ++j)
            nd[dt] = E::mma4(an[ks][j], __builtin_bit_cast(s16x4, u32x2{kt[2 * j], kt[2 * j + 1]}), nd[dt]);
        }
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) nacc[dt] += nd[dt][0] + nd[dt][1];
      if (!STATES_ONLY && kc + 1 < kc1) store_nparts((kc + 1) & 1);
      __syncthreads();  // B1: the next chunk's tiles, gate rows and n parts are staged
    }
    // ---- final states (undo the deferred rescale)
    if (ce) {
      const float* gl = gbuf + ((kc1 - 1) & 1) * GROWS * 64;
      const float sc = exp_(gl[322]);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int vt = 0; vt < 2; ++vt)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            ce[((size_t)bh * dq + srow(dt, e)) * DV + v0 + 32 * vt + l32] = acc[dt][vt][e] * sc;
      if (v0 == 0) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const float x = nacc[dt] + __shfl_xor(nacc[dt], 32);
          if (hh == 0) ne[(size_t)bh * dq + state_row(dw0, dt, l32)] = x * sc;
        }
        if (tid == 0) me[bh] = gl[321];
      }
    }
  } else {
    // =====================================================================
    // output waves: rows [16o, 16o + 16) of every chunk, the staging of K and V,
    // alpha' V one chunk ahead, and (wave 0 of the group) the gate rows
    // =====================================================================
    __builtin_amdgcn_s_setprio(2);
    const int t = tid - 64 * NSW;  // 0 .. NOT-1
    // ---- gate rows (output wave 0, one chunk ahead): row terms of the
    // intra-chunk exponent (log2 of the score scale included), column terms,
    // output row scales, the combined
    // stabiliser mc and alpha' = exp(a_t - m') e^{-G} of chunk c go to buffer
    // c & 1 with the chunk's renormalisation factor of the stored state, m',
    // the deferred log rescale G, the renormalise flag, and alpha' as bf16
    // hi (64) | lo (64) in token order (the n update's operand).
    const float* preph = a.prep + (size_t)bh * NC * PREP_STRIDE;
    float gm = m_init, gG = 0.f;  // running m and G (every output wave runs the recurrence)
    auto prep_load = [&](int c, float (&pv)[5]) {
      const float* pc = preph + (size_t)c * PREP_STRIDE;
      pv[0] = pc[lane];
      pv[1] = pc[64 + lane];
      pv[2] = pc[128 + lane];
      pv[3] = pc[192 + lane];
      pv[4] = pc[256 + (lane & 1)];
    };
    // every output wave steps the recurrence and returns alpha' of its lane's token; only
    // the writer (output wave 0) forms and stores the rows
    auto gate_rows = [&](int c, const float (&pv)[5], bool writer) {
      float* gb = gbuf + (c & 1) * GROWS * 64;
      const float pg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv[4]), 0));
      const float pamax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv[4]), 1));
      const float b = pv[0], av_ = pv[1], cmu = pv[2];
      const float m_next = fmaxf(pg + gm, pamax);
      const float lg = pg + gm - m_next;  // log of this chunk's rescale of the state (<= 0)
      float Gn = gG + lg;
      const bool renorm = Gn < E::RENORM;   // wave-uniform
      if (renorm) Gn = 0.f;
      const float al = exp_(av_ - m_next - Gn);  // alpha' = exp(a_t - m') e^{-G}
      if (writer) {
        const float mb = b + gm;
        const float mc = fmaxf(mb, b + cmu);
        // row term of the intra-chunk exponent, with log2 of the score scale folded in
        gb[lane] = (b - mc) * LOG2E + __builtin_amdgcn_logf(a.qk_scale);
        gb[64 + lane] = pv[3];                             // column term
        gb[128 + lane] = exp_(mb - mc + gG) * a.qk_scale;  // output row scale (deferred state rescale folded in)
        gb[192 + lane] = mc;
        const uint32_t ahi = E::pack(al, 0.f);
        uint16_t* ar = reinterpret_cast<uint16_t*>(gb + 384);
        ar[lane] = (uint16_t)ahi;
        ar[64 + lane] = (uint16_t)E::pack(al - E::lo(ahi), 0.f);
        ar[128 + lane] = 0;  // the zero rows of the n update's A operand
        if (lane == 0) {
          gb[320] = exp_(gG + lg);  // may underflow to 0: the old state is then negligible
          gb[321] = m_next;
          gb[322] = Gn;
          gb[323] = renorm ? 1.f : 0.f;
        }
      }
      gm = m_next;
      gG = Gn;
      return al;
    };
    // ---- K and V staging of the next chunk: piece u of thread t
    u32x4 Kst[NKO], Vst[2];
    // piece u * NOT + t: K row (piece / (DQK / 8)), 16-byte column piece % (DQK / 8) of the
    // tile (NOT / (DQK / 8) rows further per u); in memory rows of dq, so a column past dq
    // gets an offset beyond the buffer's records and reads as zero; V row piece >> 3, 8 columns
    const uint32_t k_off = (t % (DQK / 8)) < dq / 8 ? (uint32_t)((t / (DQK / 8)) * dq * 2 + 16 * (t % (DQK / 8)))
                                                     : 0x80000000u;
    const uint32_t v_off = (uint32_t)(((t >> 3) * DV + v0 + 8 * (t & 7)) * 2);
    auto load_kv = [&](int kc) {
      const auto r = chunk_rsrc(kh + (size_t)kc * L * dq, rows_of(kc), dq * 2);
#pragma unroll
      for (int u = 0; u < NKO; ++u) Kst[u] = ld16s(r, k_off, (uint32_t)(u * (NOT / (DQK / 8)) * dq * 2));
      const auto rv = chunk_rsrc(vh + (size_t)kc * L * DV, rows_of(kc), DV * 2);
#pragma unroll
      for (int u = 0; u < 2; ++u) Vst[u] = ld16s(rv, v_off, (uint32_t)(u * (NOT / 8) * DV * 2));  // NOT / 8 rows per u
    };
    auto store_kv = [&]() {
#pragma unroll
      for (int u = 0; u < NKO; ++u) {
        const int piece = u * NOT + t;
        *reinterpret_cast<u32x4*>(kn + (piece / (DQK / 8)) * SM::KN_PITCH + 16 * (piece % (DQK / 8))) = Kst[u];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int piece = u * NOT + t;
        *reinterpret_cast<u32x4*>(vn + (piece >> 3) * VN_PITCH + 16 * (piece & 7)) = Vst[u];
      }
    };
    // ---- alpha' V of a chunk as bf16 hi | lo rows (B operand of the update), formed from
    // the V pieces this thread stages (Vst, the same piece -> row map) while they are still
    // in registers, one phase before they are written: alpha' of row r is lane r's value
    u32x4 avh_r[2], avl_r[2];
    auto alpha_v_regs = [&](float al) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = (u * NOT + t) >> 3;
        const float ar = __shfl(al, row);
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          const float x0 = ar * E::lo(Vst[u][c2]), x1 = ar * E::hi(Vst[u][c2]);
          avh_r[u][c2] = E::pack(x0, x1);
          avl_r[u][c2] = pack_lo_t<E>(avh_r[u][c2], x0, x1);
        }
      }
    };
    auto alpha_v_store = [&]() {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int piece = u * NOT + t, row = piece >> 3, cg = piece & 7;
        *reinterpret_cast<u32x4*>(av + row * AV_PITCH + 16 * cg) = avh_r[u];
        *reinterpret_cast<u32x4*>(av + row * AV_PITCH + 128 + 16 * cg) = avl_r[u];
      }
    };

    // one specialisation per output row tile O: the causal bounds of the S and
    // M V products are compile-time constants
    auto out_wave = [&](auto otag) {
      constexpr int o = decltype(otag)::value;
      u32x4 Qf[KPD];
      const uint32_t qf_off = (uint32_t)(((16 * o + r16) * dq + 8 * g) * 2);
      float pv[5];  // gate prep of the next chunk
      // q fragments of rows 16o + r16 for S: k-slice 32p + 8g .. 32p + 8g + 7 (one
      // 16-byte load; the K operand below uses the same contiguous k order)
      auto load_q = [&](int kc) {
        const auto rq = q_rsrc(kc);
#pragma unroll
        for (int p = 0; p < KPD; ++p)  // k-steps past dq: an offset beyond the records reads zeros
          Qf[p] = ld16s(rq, qf_off, 32 * p < dq ? (uint32_t)(64 * p) : 0x80000000u);
      };
      // prologue: the first chunk's tiles and gate rows, the second chunk's loads in flight
      load_kv(kc0);
      if (!STATES_ONLY) load_q(kc0);
      prep_load(kc0, pv);
      alpha_v_regs(gate_rows(kc0, pv, o == 0));
      store_kv();
      load_kv(kc0 + 1);
      prep_load(min(kc0 + 1, kc1 - 1), pv);
      __syncthreads();  // B0

      for (int kc = kc0; kc < kc1; ++kc) {
        const float* gb = gbuf + (kc & 1) * GROWS * 64;
        const bf16_t* nbk = nbuf + (kc & 1) * 4 * SM::NB_PITCH;
        // ---------------- phase A: alpha' V of the chunk (formed in the previous phase B) to
        // LDS, S, M [V | 1]
        alpha_v_store();
        f32x4 Hmv[NVX];
        float qn = 0.f;
        if (!STATES_ONLY) {
          // S^T tiles over the whole DQK: A = K rows 16jt + r16, B = q rows; only the
          // causal j-tiles jt <= o (the rest are masked).  A fifth A tile holds n as
          // bf16 hi / lo rows (rows 2, 3 zero), so the same MFMAs give q.n.
          f32x4 Sacc[5];
          constexpr int KD = 2;  // K operands one k-step ahead
          u32x4 kf[KD][5];
          auto load_kf = [&](int p, u32x4 (&dst)[5]) {
#pragma unroll
            for (int jt = 0; jt <= o; ++jt)
              dst[jt] = *reinterpret_cast<const u32x4*>(kn + (16 * jt + r16) * SM::KN_PITCH + 16 * g + 64 * p);
            dst[4] = *reinterpret_cast<const u32x4*>(nbk + (r16 & 3) * SM::NB_PITCH + 32 * p + 8 * g);
          };
#pragma unroll
          for (int p = 0; p < KD - 1; ++p) load_kf(p, kf[p]);
#pragma unroll
          for (int jt = 0; jt < 5; ++jt) Sacc[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < KPD; ++p) {
            if (p + KD - 1 < KPD) load_kf(p + KD - 1, kf[(p + KD - 1) % KD]);
#pragma unroll
            for (int jt = 0; jt < 5; ++jt)
              if (jt == 4 || jt <= o)
                Sacc[jt] = E::mma16(__builtin_bit_cast(V8, kf[p % KD][jt]), __builtin_bit_cast(V8, Qf[p]), Sacc[jt]);
          }
          load_q(kc + 1);  // q fragments are dead: prefetch
          qn = (Sacc[4][0] + Sacc[4][1]) + (Sacc[4][2] + Sacc[4][3]);  // q . n (stored state)
          // gate the scores of row i = 16o + r16, then M [V | 1] with M split hi + lo
          const int i = 16 * o + r16;
          const float bli = gb[i];
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) {
            const f32x4 ul = *reinterpret_cast<const f32x4*>(gb + 64 + 16 * jt + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int j = 16 * jt + 4 * g + e;
              Sacc[jt][e] = (j <= i) ? Sacc[jt][e] * exp2_(bli + ul[e]) : 0.f;
            }
          }
#pragma unroll
          for (int vq = 0; vq < NVX; ++vq) Hmv[vq] = f32x4{0.f, 0.f, 0.f, 0.f};
          // the V operands of both token halves first (their LDS latency then overlaps the splits)
          constexpr int NPJ = (16 * o + 15) / 32 + 1;  // token halves with unmasked M (compile-time)
          V8 vbs[NPJ][NVT];
#pragma unroll
          for (int pj = 0; pj < NPJ; ++pj)
#pragma unroll
            for (int vq = 0; vq < NVT; ++vq) {
              const char* base = vn + (32 * pj + 4 * g + (r16 >> 2)) * VN_PITCH + 2 * vcol_of(vq, 4 * (r16 & 3));
              vbs[pj][vq] = __builtin_bit_cast(V8, tr8(base, base + 16 * VN_PITCH));
            }
          // [.. | 1]: rows 0, 4, 8, 12 of the fifth tile are all ones
          const uint32_t one = ((r16 & 3) == 0) ? E::ONE2 : 0u;
          const V8 ones = __builtin_bit_cast(V8, u32x4{one, one, one, one});
#pragma unroll
          for (int pj = 0; pj < NPJ; ++pj) {
            V8 mh, ml;
            split8_t<E>(Sacc[2 * pj], Sacc[2 * pj + 1], mh, ml);
#pragma unroll
            for (int vq = 0; vq < NVX; ++vq) {
              const V8 vb = vq < NVT ? vbs[pj][vq] : ones;
              // transposed product [V | 1]^T M^T: lane (g, r16) gets columns 4g+e of row r16
              Hmv[vq] = E::mma16(vb, mh, Hmv[vq]);
              Hmv[vq] = E::mma16(vb, ml, Hmv[vq]);
            }
          }
        }
        __syncthreads();  // B2: the state waves' partial Q C of this chunk are complete

        // ---------------- phase B: finish h of the chunk, stage the next chunk's K, V and
        // gate rows.  The partials are read first, the K / V tiles written while they arrive.
        // Q C of row 16o + r16, columns vcol_of(vq, 4g + e): sum of the four state waves'
        // partials (two 16-byte runs of 4 columns per tile pair)
        f32x4 Hqc[NVT];
        if (!STATES_ONLY) {
          const float* pr = hp + (16 * o + r16) * HP_PITCH;
#pragma unroll
          for (int vq = 0; vq < NVT; ++vq) Hqc[vq] = *reinterpret_cast<const f32x4*>(pr + hp_col(8 * (vq >> 1) + 2 * g + (vq & 1)));
#pragma unroll
          for (int sw = 1; sw < NSW; ++sw)
#pragma unroll
            for (int vq = 0; vq < NVT; ++vq)
              Hqc[vq] += *reinterpret_cast<const f32x4*>(pr + sw * 64 * HP_PITCH + hp_col(8 * (vq >> 1) + 2 * g + (vq & 1)));
        }
        if (kc + 1 < kc1) store_kv();
        if (!STATES_ONLY) {
          // this lane holds columns vcol_of(vq, 4g + e), i.e. the 8 consecutive
          // columns 32h + 8g .. +7 of tiles (2h, 2h+1); the row sum of M is element 0
          // of the fifth tile
          const float qb = gb[128 + 16 * o + r16];
          const float mcr = gb[192 + 16 * o + r16];
          const float den = qb * qn + Hmv[NVT][0];
          const float inv = __builtin_amdgcn_rcpf(fmaxf(fabsf(den), exp_(-mcr)) + a.eps);
          // rows past S (ragged last chunk) are dropped by the range check
          const auto rh = chunk_rsrc(hh + (size_t)kc * L * DV, rows_of(kc), DV * 2);
          const uint32_t hoff = (uint32_t)(((16 * o + r16) * DV + v0 + 8 * g) * 2);
#pragma unroll
          for (int h2 = 0; h2 < NVT / 2; ++h2) {
            u32x4 out;
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              const int vq = 2 * h2 + b;
              out[2 * b] = E::pack((qb * Hqc[vq][0] + Hmv[vq][0]) * inv, (qb * Hqc[vq][1] + Hmv[vq][1]) * inv);
              out[2 * b + 1] = E::pack((qb * Hqc[vq][2] + Hmv[vq][2]) * inv, (qb * Hqc[vq][3] + Hmv[vq][3]) * inv);
            }
            st16(rh, hoff + 64 * h2, out);
          }
        }
        if (kc + 1 < kc1) alpha_v_regs(gate_rows(kc + 1, pv, o == 0));  // before Vst is reloaded
        load_kv(kc + 2);
        prep_load(min(kc + 2, kc1 - 1), pv);
        __syncthreads();  // B1
      }
    };
    switch (__builtin_amdgcn_readfirstlane(ws)) {
      case 0: out_wave(std::integral_constant<int, 0>{}); break;
      case 1: out_wave(std::integral_constant<int, 1>{}); break;
      case 2: out_wave(std::integral_constant<int, 2>{}); break;
      default: out_wave(std::integral_constant<int, 3>{}); break;
    }
  }
}

template <typename T, int DQK, bool STATES_ONLY>
static int launch_one(unsigned nwg, hipStream_t st, const MainArgs& a) {
  const size_t smem = Smem<DQK>::BYTES;
  auto kern = chunkwise_pipe_kernel<T, DQK, STATES_ONLY>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess)
    return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd: LDS attribute failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(kern, dim3(nwg), dim3(NTHREADS), smem, st, a);
  return XL_OK;
}

}  // namespace pipe

template <typename T>
static int pipe_launch_t(int DQK, bool states_only, unsigned nwg, hipStream_t st, const MainArgs& a) {
  if (DQK == 256)
    return states_only ? pipe::launch_one<T, 256, true>(nwg, st, a) : pipe::launch_one<T, 256, false>(nwg, st, a);
  return states_only ? pipe::launch_one<T, 128, true>(nwg, st, a) : pipe::launch_one<T, 128, false>(nwg, st, a);
}

int pipe_launch(bool f16, int DQK, bool states_only, unsigned nwg, hipStream_t st, const MainArgs& a) {
  return f16 ? pipe_launch_t<f16_t>(DQK, states_only, nwg, st, a) : pipe_launch_t<bf16_t>(DQK, states_only, nwg, st, a);
}

}  // namespace fused
}  // namespace xl
