// Fused single-pass chunkwise mLSTM forward for bf16 q/k/v on gfx950.
//
// One workgroup = one (b, h) pair x one 64-column tile of DV, marching over
// the NC = ceil(S / 64) chunks of L = 64 tokens (in a ragged last chunk the
// tokens past S are given no weight and their outputs are not stored).  The C tile (DQK x 64, float32) and the
// normaliser n stay on chip for the whole sequence, so the only HBM traffic is
// q, k, v, the gates, h and the final states.  The math is the reference's
// chunkwise forward (kernel_development/xlstm/mlstm_block/mlstm_chunkwise/
// vendored/torch/native/fw.py:98-143 for the inter-chunk recurrence,
// :193-245 for the outputs), per chunk:
//
//   b = cumsum logsig f, g = b_L, a_t = g - b_t + i_t, m' = max(g + m, max a)
//   m_i = max(b_i + m, max_{j<=i} (b_i - b_j + i_j))
//   M_ij = (q_i.k_j) s exp(b_i - b_j + i_j - m_i)         (j <= i)
//   H_i  = exp(b_i + m - m_i) s (q_i C) + sum_j M_ij v_j
//   den_i = exp(b_i + m - m_i) s (q_i.n) + sum_j M_ij
//   h_i = H_i / (max(|den_i|, exp(-m_i)) + eps)
//   C' = exp(g + m - m') C + sum_t exp(a_t - m') k_t v_t^T,  n' likewise
//
// Producer / consumer split (8 waves, two per SIMD):
//  * state waves 0..3: wave s owns rows [s*DW, (s+1)*DW) of C (DW = DQK/4,
//    float32 accumulators of v_mfma_f32_32x32x16_bf16).  Per chunk it first
//    forms the partial product Q[:, rows] C[rows, :] for all 64 tokens, with
//    the A operand built straight from its accumulators as bf16 hi + lo (two
//    MFMAs, so q C keeps float32 accuracy), and leaves it in LDS.  It then
//    applies the chunk update C += K^T (alpha V) with alpha V split into bf16
//    hi + lo, so the state keeps float32 accuracy too.
//  * output waves 4..7: wave o owns output rows [16o, 16o+16) of every chunk:
//    exact S^T = K Q^T over the whole DQK, gating and M [V | 1] (M split
//    hi + lo); after the chunk's second barrier it adds the four partial
//    Q C rows and writes h.  Wave o also carries rows [o*DQK/4, (o+1)*DQK/4)
//    of the normaliser n (16 x 16 accumulators, alpha' hi and lo in
//    alternate columns) and applies n += K^T alpha'; q.n comes out of a fifth
//    A tile of the S product that holds n as four bf16 rows (hi and lo of
//    both column sums), staged in LDS once per chunk.
// The state never leaves the state waves' registers; the only cross-wave
// traffic besides the staged q/k/v tiles is the 16-byte-per-lane partials.
// K^T, V and alpha V operands are read with ds_read_b64_tr_b16 from the
// natural row-major tiles (within 16 lanes, output lane 4a+c receives element
// c of source lanes 4k+a, k = 0..3).  Row pitches follow measured LDS rates
// on gfx950: 16-byte reads of 16 consecutive rows at one column (the S
// operand, the n rows) run at full rate when the pitch is 32 mod 64 bytes,
// and the transposed reads of 4 consecutive rows stay conflict free there.
//
// The forget rescale exp(g + m - m') of C is deferred: the state is stored as
// C e^{-G} (G = accumulated log rescale), the factor e^{-G} is folded into
// alpha V and e^{G} into the output row scale, and C is renormalised only
// when G drops below -30 (the eager path).
//
// Grid mapping is XCD aware: the DV tiles of one head land on the same XCD so
// the head's q/k chunks are fetched from HBM once and then hit that XCD's L2.
#include "fused_common.h"

#include <type_traits>

namespace xl {
namespace fused {


// Chunk-local gate prep, one wave per (head, chunk), lane = token t
// (fw.py:308-316 and :98, :204-213 before the running stabiliser enters):
//   b_t = sum_{s<=t} logsig f_s,  g = b_63,  a_t = g - b_t + i_t,  max_t a_t,
//   u_t = i_t - b_t (stored times log2 e),  cummax_{s<=t} u_s.
// These are the scans of the chunk; the main kernel folds in the running m
// and the deferred state rescale with a handful of scalar operations.  Tokens
// past S (a ragged last chunk) enter as logsig f = 0 and i = -inf: they leave
// b unchanged and contribute nothing to the state, n or max a.
template <typename TG>
__global__ __launch_bounds__(256) void gate_prep_kernel(const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                        float* __restrict__ prep, int total_chunks, int NC, int S) {
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);  // bh * NC + chunk
  if (c >= total_chunks) return;
  const int bh = c / NC, t = (c - bh * NC) * L + lane;  // token t of head bh
  const bool ok = t < S;
  const size_t gi = (size_t)bh * S + (ok ? t : S - 1);
  const float f = to_f32(fg[gi]), i = ok ? to_f32(ig[gi]) : -INFINITY;
  const float b = wave_scan<false>(ok ? logsig_fast(f) : 0.f);
  const float g = lane63(b);
  const float a = g - b + i;
  const float amax = lane63(wave_scan<true>(a));
  const float u = i - b;
  const float cmu = wave_scan<true>(u);
  float* p = prep + (size_t)c * PREP_STRIDE;
  p[lane] = b;
  p[64 + lane] = a;
  p[128 + lane] = cmu;
  p[192 + lane] = u * LOG2E;
  if (lane == 0) {
    p[256] = g;
    p[257] = amax;
  }
}




template <int DQK, bool STATES_ONLY>
__global__ __launch_bounds__(NTHREADS, 1) void chunkwise_fused_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const float* __restrict__ c0,
    const float* __restrict__ n0, const float* __restrict__ m0, bf16_t* __restrict__ h,
    float* __restrict__ c_last, float* __restrict__ n_last, float* __restrict__ m_last,
    const float* __restrict__ prep, int S, int NC, int DV, int BNH, int nvtile, float qk_scale, float eps,
    SegArgs sg) {
  using SM = Smem<DQK>;
  constexpr int KPD = SM::KPD;
  constexpr int DW = DQK / NSW;   // C rows per state wave (64 or 32)
  constexpr int NKU = DQK / 64;   // K staging: 16-byte pieces per thread (64 rows x DQK / 512 threads / 8)
  constexpr int ND = DQK / NOW;   // n rows per output wave
  constexpr int NTO = ND / 16;    // 16-row n tiles per output wave
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int ws = w & 3;  // index within the state or output group

  // ---- XCD-aware workgroup -> (head, column tile): consecutive tiles of a head share an XCD
  const int nwg = BNH * nvtile * sg.nseg;
  int lin = blockIdx.x;
  if ((nwg & 7) == 0) lin = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int bhs = lin / nvtile;  // segment * BNH + head
  const int v0 = (lin - bhs * nvtile) * DVT;
  const int seg = bhs / BNH, bh = bhs - seg * BNH;
  const int kc0 = seg * sg.kc_per_seg, kc1 = min(NC, kc0 + sg.kc_per_seg);  // this segment's chunks
  // initial state of this segment (see SegArgs)
  const size_t cst = (size_t)BNH * DQK * DV, nst = (size_t)BNH * DQK;
  const float* ci = seg == 0 ? c0 : (sg.sc ? sg.sc + (seg - 1) * cst : nullptr);
  const float* ni = seg == 0 ? n0 : (sg.sn ? sg.sn + (seg - 1) * nst : nullptr);
  const float m_init = seg == 0 ? (m0 ? m0[bh] : 0.f) : (sg.sm ? sg.sm[(seg - 1) * BNH + bh] : -INFINITY);
  // where the end state goes: every segment's (ec) or the last segment's (c_last)
  float* ce = sg.ec ? sg.ec + seg * cst : (seg == sg.nseg - 1 ? c_last : nullptr);
  float* ne = sg.ec ? sg.en + seg * nst : n_last;
  float* me = sg.ec ? sg.em + (size_t)seg * BNH : m_last;

  char* kn = smem + SM::KN;
  char* vn = smem + SM::VN;
  char* av = smem + SM::AV;
  float* hp = (float*)(smem + SM::HP);
  bf16_t* nbuf = (bf16_t*)(smem + SM::NB);   // [2][4][NB_PITCH]: n parts of chunk kc live in buffer kc & 1
  float* gbuf = (float*)(smem + SM::GATES);  // [2][GROWS][64]: rows of chunk kc live in buffer kc & 1

  const bf16_t* qh = q + (size_t)bh * S * DQK;
  const bf16_t* kh = k + (size_t)bh * S * DQK;
  const bf16_t* vh = v + (size_t)bh * S * DV;
  bf16_t* hh = h + (size_t)bh * S * DV;
  auto rows_of = [&](int kc) { return min(L, S - kc * L); };  // valid rows of chunk kc
  auto q_rsrc = [&](int kc) { return chunk_rsrc(qh + (size_t)kc * L * DQK, rows_of(kc), DQK * 2); };

  // ---- K staging: piece u of thread tid = u*NTHREADS + tid -> row piece / (DQK/8), 16-byte column group
  // (rows past S read as 0: those tokens carry alpha' = 0 and gate weight
  // exp(-inf) = 0, their S columns are causally masked for real rows, and their
  // own rows of h are not stored)
  auto load_k = [&](int kc, u32x4 (&Kst)[NKU]) {
    const auto r = chunk_rsrc(kh + (size_t)kc * L * DQK, rows_of(kc), DQK * 2);
#pragma unroll
    for (int u = 0; u < NKU; ++u) {
      const int piece = u * NTHREADS + tid;
      Kst[u] = ld16(r, (uint32_t)((piece / (DQK / 8)) * DQK * 2 + 16 * (piece % (DQK / 8))));
    }
  };
  auto store_k = [&](const u32x4 (&Kst)[NKU]) {
#pragma unroll
    for (int u = 0; u < NKU; ++u) {
      const int piece = u * NTHREADS + tid;
      *reinterpret_cast<u32x4*>(kn + (piece / (DQK / 8)) * SM::KN_PITCH + 16 * (piece % (DQK / 8))) = Kst[u];
    }
  };
  // ---- gate rows (computed by the gate wave, output wave 0, one chunk ahead)
  // Row terms of the intra-chunk exponent, column terms, output row scales,
  // the combined stabiliser mc and alpha' = exp(a_t - m') e^{-G} of chunk c go
  // to buffer c & 1 together with the chunk's renormalisation factor of the
  // stored state, m', the deferred log rescale G, the renormalise flag and
  // alpha' as bf16 hi / lo (the B operand of the n update).
  const float* preph = prep + (size_t)bh * NC * PREP_STRIDE;
  float gm = m_init, gG = 0.f;  // running m and G (gate wave only)
  // pv[4] holds g (lane 0) and max a (lane 1): a per-lane load, so it is
  // counted with the vector loads and never stalls the LDS waits
  auto prep_load = [&](int c, float (&pv)[5]) {
    const float* pc = preph + (size_t)c * PREP_STRIDE;
    pv[0] = pc[lane];
    pv[1] = pc[64 + lane];
    pv[2] = pc[128 + lane];
    pv[3] = pc[192 + lane];
    pv[4] = pc[256 + (lane & 1)];
  };
  auto gate_rows = [&](int c, const float (&pv)[5]) {
    float* gb = gbuf + (c & 1) * GROWS * 64;
    const float pg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv[4]), 0));
    const float pamax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv[4]), 1));
    const float b = pv[0], a = pv[1], cmu = pv[2];
    const float m_next = fmaxf(pg + gm, pamax);
    const float lg = pg + gm - m_next;  // log of this chunk's rescale of the state (<= 0)
    float Gn = gG + lg;
    const bool renorm = Gn < RENORM;   // wave-uniform
    if (renorm) Gn = 0.f;
    const float mb = b + gm;
    const float mc = fmaxf(mb, b + cmu);
    gb[lane] = (b - mc) * LOG2E;                       // row term of the intra-chunk exponent
    gb[64 + lane] = pv[3];                             // column term
    gb[128 + lane] = exp_(mb - mc + gG) * qk_scale;    // output row scale (deferred state rescale folded in)
    gb[192 + lane] = mc;
    const float al = exp_(a - m_next - Gn);            // alpha' = exp(a_t - m') e^{-G}
    gb[256 + lane] = al;
    // alpha' hi / lo as bf16; token t of each 8-token group at 4 (t & 1) + (t & 7) / 2, the k
    // order of the transposed K reads of the n update
    const uint32_t ahi = pack_bf16(al, 0.f);
    uint16_t* ar = reinterpret_cast<uint16_t*>(gb + 384);
    const int pos = (lane & ~7) + 4 * (lane & 1) + ((lane & 7) >> 1);
    ar[pos] = (uint16_t)ahi;
    ar[64 + pos] = (uint16_t)pack_bf16(al - bf_lo(ahi), 0.f);
    if (lane == 0) {
      gb[320] = exp_(gG + lg);  // may underflow to 0: the old state is then negligible
      gb[321] = m_next;
      gb[322] = Gn;
      gb[323] = renorm ? 1.f : 0.f;
    }
    gm = m_next;
    gG = Gn;
  };

  // ---- n (output waves): wave o holds rows [o*ND, (o+1)*ND) as NTO 16 x 16 MFMA
  // accumulator tiles; lane (g, r16) holds rows 16 dt + 4g + e of column r16.
  // Even columns accumulate K^T alpha'_hi, odd columns K^T alpha'_lo, so
  // n = (even column) + (odd column) keeps float32 accuracy with one MFMA per
  // k-step.  Before every chunk the four parts (hi, lo of both halves) go to
  // LDS as bf16 rows, the A operand of q.n in the output waves' S product.
  const int nd0 = ND * ws;
  f32x4 nacc[NTO];
  auto store_nparts = [&](int buf) {
    if (r16 < 2) {  // lane 0: even column (parts 0, 1), lane 1: odd column (parts 2, 3)
      bf16_t* nb = nbuf + buf * 4 * SM::NB_PITCH + nd0 + 4 * g;
#pragma unroll
      for (int dt = 0; dt < NTO; ++dt) {
        const f32x4 x = nacc[dt];
        const u32x2 hi = {pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])};
        const u32x2 lo = {pack_lo(hi[0], x[0], x[1]), pack_lo(hi[1], x[2], x[3])};
        *reinterpret_cast<u32x2*>(nb + (2 * r16) * SM::NB_PITCH + 16 * dt) = hi;
        *reinterpret_cast<u32x2*>(nb + (2 * r16 + 1) * SM::NB_PITCH + 16 * dt) = lo;
      }
    }
  };
  if (w >= NSW) {
#pragma unroll
    for (int dt = 0; dt < NTO; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        nacc[dt][e] = (ni && (r16 & 1) == 0) ? ni[(size_t)bh * DQK + nd0 + 16 * dt + 4 * g + e] : 0.f;
    store_nparts(kc0 & 1);
  }
  if (w == NSW) {
    float pv[5];
    prep_load(kc0, pv);
    gate_rows(kc0, pv);
  }
  __syncthreads();  // B0: gate rows and n parts of chunk 0

  if (w < NSW) {
    // =====================================================================
    // state waves: rows [dw0, dw0 + DW) of C, stored as C e^{-G}
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
          acc[dt][vt][e] = ci ? ci[((size_t)bh * DQK + srow(dt, e)) * DV + v0 + 32 * vt + l32] : 0.f;

    // V staging (state threads): rows t0 = 4*(tid>>4) + ((tid>>3)&1) and t0 + 2, columns 8*(tid&7)
    const int vrow = 4 * (tid >> 4) + ((tid >> 3) & 1), vcol = 8 * (tid & 7);
    u32x4 Kst[NKU], Vst[2];
    // q fragments (B operand of the transposed product C^T Q^T): token 32 tt + l32,
    // rows dw0 + 16 s + 8 hh .. +7
    u32x4 Qs[2][QKS];
    auto load_v = [&](int kc) {
      const auto rv = chunk_rsrc(vh + (size_t)kc * L * DV, rows_of(kc), DV * 2);
#pragma unroll
      for (int r = 0; r < 2; ++r) Vst[r] = ld16(rv, (uint32_t)(((vrow + 2 * r) * DV + v0 + vcol) * 2));
    };
    auto load_qs = [&](int kc) {
      const auto rq = q_rsrc(kc);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int s = 0; s < QKS; ++s)
          Qs[tt][s] = ld16(rq, (uint32_t)(((32 * tt + l32) * DQK + dw0 + 8 * hh + 16 * s) * 2));
    };
    load_k(kc0, Kst);
    load_v(kc0);
    if (!STATES_ONLY) load_qs(kc0);
    for (int kc = kc0; kc < kc1; ++kc) {
      const float* gb = gbuf + (kc & 1) * GROWS * 64;
      store_k(Kst);
      // V natural and alpha' V hi / lo (natural layout, 16-byte rows)
      *reinterpret_cast<u32x4*>(vn + vrow * VN_PITCH + 2 * vcol) = Vst[0];
      *reinterpret_cast<u32x4*>(vn + (vrow + 2) * VN_PITCH + 2 * vcol) = Vst[1];
      const float al2[2] = {gb[256 + vrow], gb[256 + vrow + 2]};
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        u32x4 hv, lv;
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          const float x0 = al2[r] * bf_lo(Vst[r][c2]), x1 = al2[r] * bf_hi(Vst[r][c2]);
          hv[c2] = pack_bf16(x0, x1);
          lv[c2] = pack_lo(hv[c2], x0, x1);
        }
        *reinterpret_cast<u32x4*>(av + (vrow + 2 * r) * AV_PITCH + 2 * vcol) = hv;
        *reinterpret_cast<u32x4*>(av + (vrow + 2 * r) * AV_PITCH + 128 + 2 * vcol) = lv;
      }
      __syncthreads();  // B1: the chunk's tiles are visible; the previous chunk's partials have been read
      if (kc + 1 < kc1) {  // staging registers are free: prefetch (q after its last use below)
        load_k(kc + 1, Kst);
        load_v(kc + 1);
      }
      // partial Q C over this wave's rows, with the state before this chunk
      // (bf16 hi + lo of the float32 accumulators, so q C keeps float32
      // accuracy).  Transposed product C^T Q^T per 32-column tile vt: lane
      // (hh, l32) gets columns 32 vt + 8i + 4hh + j of token 32 tt + l32.
      // Software pipelined: the split of k-step q+1 (VALU) is interleaved with
      // the four MFMAs of k-step q, and the partials of column tile 0 are
      // stored one k-step into tile 1, when their MFMAs have retired.
      if (!STATES_ONLY) {
        constexpr int NQ = 2 * QKS;
        bf16x8 bsp[2][2];
        f32x16 P[2][2];
        auto split_q = [&](int qi, bf16x8 (&o)[2]) {
          const int vt = qi / QKS, s = qi % QKS;
          const f32x16& a = acc[s >> 1][vt];
          const int e0 = 8 * (s & 1);
          split8(f32x4{a[e0], a[e0 + 1], a[e0 + 2], a[e0 + 3]}, f32x4{a[e0 + 4], a[e0 + 5], a[e0 + 6], a[e0 + 7]},
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
              P[vt][tt] = mfma32(bsp[cur][hl], __builtin_bit_cast(bf16x8, Qs[tt][s]), P[vt][tt]);
          if (vt == 1 && s == 1) store_p(0);
          // ask the scheduler for 1 MFMA : 6 VALU
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
          }
        }
        store_p(1);
      }
      if (!STATES_ONLY && kc + 1 < kc1) load_qs(kc + 1);
      if (gb[323] != 0.f) {  // renormalise the stored state (wave-uniform)
        const float sc = gb[320];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) acc[dt][vt] *= sc;
      }
      // update C += K^T (alpha' V): A = K^T (row l32 of tile dt is state row
      // srow(dt, .) of that accumulator row), B = alpha' V (column 32 vt + l32),
      // 16-token k-steps, tokens 16 ks + 8 hh + jj in both.  Transposed reads:
      // within 16 lanes, source lane 4kk + a reads token 16 ks + 8 hh + kk (+4
      // for the second read) at 4 consecutive columns.
      {
        const int kk = r16 >> 2, ka = r16 & 3;
        bf16x8 Kt[NDT][4];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const char* base = kn + (16 * ks + 8 * hh + kk) * SM::KN_PITCH +
                               2 * (dw0 + 32 * dt + 16 * (g & 1) + 8 * (ka & 1) + 4 * (ka >> 1));
            Kt[dt][ks] = tr8(base, base + 4 * SM::KN_PITCH);
          }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int vt = 0; vt < 2; ++vt) {
            const char* base = av + (16 * ks + 8 * hh + kk) * AV_PITCH + 2 * (32 * vt + 16 * (g & 1) + 4 * ka);
            const bf16x8 bh = tr8(base, base + 4 * AV_PITCH);
            const bf16x8 bl = tr8(base + 128, base + 128 + 4 * AV_PITCH);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
              acc[dt][vt] = mfma32(Kt[dt][ks], bh, acc[dt][vt]);
              acc[dt][vt] = mfma32(Kt[dt][ks], bl, acc[dt][vt]);
            }
          }
      }
      __syncthreads();  // B2: partials complete; the chunk's tiles may be overwritten
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
            ce[((size_t)bh * DQK + srow(dt, e)) * DV + v0 + 32 * vt + l32] = acc[dt][vt][e] * sc;
      if (v0 == 0 && tid == 0) me[bh] = gl[321];
    }
  } else {
    // =====================================================================
    // output waves: rows [16o, 16o + 16) of every chunk, and n rows [nd0, nd0 + ND)
    // =====================================================================
    // the output waves are the longer dependency chain of a chunk: let their
    // MFMAs and loads win the SIMD's issue arbitration over the state waves'
    __builtin_amdgcn_s_setprio(2);
    // one specialisation per output row tile O: the causal bounds of the S and
    // M V products are compile-time constants
    auto out_wave = [&](auto otag) {
    constexpr int o = decltype(otag)::value;
    u32x4 Kst[NKU], Qf[KPD];
    float pv[5];  // gate prep of the next chunk (gate wave)
    // q fragments of rows 16o + r16 for S: k-slice 32p + 8g .. 32p + 8g + 7 (one
    // 16-byte load; the K operand below uses the same contiguous k order)
    auto load_q = [&](int kc) {
      const auto rq = q_rsrc(kc);
#pragma unroll
      for (int p = 0; p < KPD; ++p) Qf[p] = ld16(rq, (uint32_t)(((16 * o + r16) * DQK + 8 * g + 32 * p) * 2));
    };
    load_k(kc0, Kst);
    if (!STATES_ONLY) load_q(kc0);
    for (int kc = kc0; kc < kc1; ++kc) {
      const float* gb = gbuf + (kc & 1) * GROWS * 64;
      const bf16_t* nbk = nbuf + (kc & 1) * 4 * SM::NB_PITCH;
      store_k(Kst);
      __syncthreads();  // B1
      if (kc + 1 < kc1) {
        load_k(kc + 1, Kst);
        if (o == 0) prep_load(kc + 1, pv);
      }
      if (STATES_ONLY) {  // the n update and the next gate rows only
        if (gb[323] != 0.f) {
          const float sc = gb[320];
#pragma unroll
          for (int dt = 0; dt < NTO; ++dt) nacc[dt] *= sc;
        }
        const uint16_t* ar = reinterpret_cast<const uint16_t*>(gb + 384) + 64 * (r16 & 1);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const bf16x8 ab = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(ar + 32 * p + 8 * g));
#pragma unroll
          for (int dt = 0; dt < NTO; ++dt) {
            const char* base = kn + (32 * p + 8 * g + 2 * (r16 >> 2)) * SM::KN_PITCH + 2 * (nd0 + 16 * dt + 4 * (r16 & 3));
            nacc[dt] = mfma(tr8(base, base + SM::KN_PITCH), ab, nacc[dt]);
          }
        }
        if (o == 0 && kc + 1 < kc1) gate_rows(kc + 1, pv);
        __syncthreads();  // B2
        continue;
      }

      // S^T tiles over the whole DQK: A = K rows 16jt + r16, B = q rows; only the
      // causal j-tiles jt <= o (the rest are masked), the bound a compile-time
      // constant of this specialisation.  A fifth A tile holds the four parts of
      // n (row r16 = part r16 & 3), so the same MFMAs give q.n in every lane.
      f32x4 Sacc[5];
      constexpr int KD = 2;
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
          if (jt == 4 || jt <= o)  // j-tiles above the diagonal are all masked (compile-time)
            Sacc[jt] = mfma(__builtin_bit_cast(bf16x8, kf[p % KD][jt]), __builtin_bit_cast(bf16x8, Qf[p]), Sacc[jt]);
      }
      if (kc + 1 < kc1) load_q(kc + 1);  // q fragments are dead: prefetch
      const float qn = (Sacc[4][0] + Sacc[4][1]) + (Sacc[4][2] + Sacc[4][3]);  // q . n (stored state)
      // gate the scores of row i = 16o + r16, then M [V | 1] with M split hi + lo
      const int i = 16 * o + r16;
      const float bli = gb[i];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const f32x4 ul = *reinterpret_cast<const f32x4*>(gb + 64 + 16 * jt + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 16 * jt + 4 * g + e;
          Sacc[jt][e] = (j <= i) ? Sacc[jt][e] * qk_scale * exp2_(bli + ul[e]) : 0.f;
        }
      }
      f32x4 Hmv[NVX];
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq) Hmv[vq] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pj = 0; pj < 2; ++pj) {
        if (32 * pj > 16 * o + 15) continue;  // all of M is masked for these tokens (compile-time)
        bf16x8 mh, ml;
        split8(Sacc[2 * pj], Sacc[2 * pj + 1], mh, ml);
#pragma unroll
        for (int vq = 0; vq < NVX; ++vq) {
          bf16x8 vb;
          if (vq < NVT) {
            const char* base = vn + (32 * pj + 4 * g + (r16 >> 2)) * VN_PITCH + 2 * vcol_of(vq, 4 * (r16 & 3));
            vb = tr8(base, base + 16 * VN_PITCH);
          } else {  // [.. | 1]: rows 0, 4, 8, 12 of the fifth tile are all ones
            const uint32_t one = ((r16 & 3) == 0) ? 0x3f803f80u : 0u;
            vb = __builtin_bit_cast(bf16x8, u32x4{one, one, one, one});
          }
          // transposed product [V | 1]^T M^T: lane (g, r16) gets columns 4g+e of row r16
          Hmv[vq] = mfma(vb, mh, Hmv[vq]);
          Hmv[vq] = mfma(vb, ml, Hmv[vq]);
        }
      }
      // n update: n += K^T alpha' over rows [nd0, nd0 + ND) (renormalised first
      // when the chunk asks for it).  A = K^T (transposed reads: source lane 4kk + a
      // of group g reads token 32p + 8g + 2kk (+1) at rows nd0 + 16dt + 4a ..),
      // B = alpha' hi (even columns) / lo (odd columns) in the same token order.
      {
        if (gb[323] != 0.f) {
          const float sc = gb[320];
#pragma unroll
          for (int dt = 0; dt < NTO; ++dt) nacc[dt] *= sc;
        }
        const uint16_t* ar = reinterpret_cast<const uint16_t*>(gb + 384) + 64 * (r16 & 1);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const bf16x8 ab = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(ar + 32 * p + 8 * g));
#pragma unroll
          for (int dt = 0; dt < NTO; ++dt) {
            const char* base = kn + (32 * p + 8 * g + 2 * (r16 >> 2)) * SM::KN_PITCH + 2 * (nd0 + 16 * dt + 4 * (r16 & 3));
            nacc[dt] = mfma(tr8(base, base + SM::KN_PITCH), ab, nacc[dt]);
          }
        }
        store_nparts((kc + 1) & 1);
      }
      // the gate wave forms the gate rows of chunk kc + 1 (buffer (kc + 1) & 1,
      // last read before B2 of the previous chunk)
      if (o == 0 && kc + 1 < kc1) gate_rows(kc + 1, pv);
      __syncthreads();  // B2: the state waves' partial Q C of this chunk are complete
      // Q C of row 16o + r16, columns vcol_of(vq, 4g + e): sum of the four state
      // waves' partials (two 16-byte runs of 4 columns per tile pair)
      f32x4 Hqc[NVT];
      const float* pr = hp + (16 * o + r16) * HP_PITCH;
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq) Hqc[vq] = *reinterpret_cast<const f32x4*>(pr + hp_col(8 * (vq >> 1) + 2 * g + (vq & 1)));
#pragma unroll
      for (int sw = 1; sw < NSW; ++sw)
#pragma unroll
        for (int vq = 0; vq < NVT; ++vq)
          Hqc[vq] += *reinterpret_cast<const f32x4*>(pr + sw * 64 * HP_PITCH + hp_col(8 * (vq >> 1) + 2 * g + (vq & 1)));
      // finish row 16o + r16: this lane holds columns vcol_of(vq, 4g + e), i.e. the
      // 8 consecutive columns 32h + 8g .. +7 of tiles (2h, 2h+1); the row sum of M
      // (ones in rows 0, 4, 8, 12 of the fifth tile) is element 0
      const float qb = gb[128 + 16 * o + r16];
      const float mcr = gb[192 + 16 * o + r16];
      const float den = qb * qn + Hmv[NVT][0];
      const float inv = __builtin_amdgcn_rcpf(fmaxf(fabsf(den), exp_(-mcr)) + eps);
      // rows past S (ragged last chunk) are dropped by the range check
      const auto rh = chunk_rsrc(hh + (size_t)kc * L * DV, rows_of(kc), DV * 2);
      const uint32_t hoff = (uint32_t)(((16 * o + r16) * DV + v0 + 8 * g) * 2);
#pragma unroll
      for (int h2 = 0; h2 < NVT / 2; ++h2) {
        u32x4 out;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int vq = 2 * h2 + b;
          out[2 * b] = pack_bf16((qb * Hqc[vq][0] + Hmv[vq][0]) * inv, (qb * Hqc[vq][1] + Hmv[vq][1]) * inv);
          out[2 * b + 1] = pack_bf16((qb * Hqc[vq][2] + Hmv[vq][2]) * inv, (qb * Hqc[vq][3] + Hmv[vq][3]) * inv);
        }
        st16(rh, hoff + 64 * h2, out);
      }
    }
    // ---- final n (undo the deferred rescale): even + odd column, lanes r16 = 0, 1
    if (ce && v0 == 0) {
      const float* gl = gbuf + ((kc1 - 1) & 1) * GROWS * 64;
      const float sc = exp_(gl[322]);
#pragma unroll
      for (int dt = 0; dt < NTO; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float na = nacc[dt][e];
          // quad_perm [1, 0, 3, 2]: lane 4q gets lane 4q + 1
          const float nb = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, na), 0xB1, 0xf, 0xf, false));
          if (r16 == 0) ne[(size_t)bh * DQK + nd0 + 16 * dt + 4 * g + e] = (na + nb) * sc;
        }
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

// Start states of segments 1 .. P-1 from the end states of the first pass:
// start(1) = E_0 (segment 0 ran from the caller's initial state), and
// start(s + 1) = compose(start(s), E_s), E_s being segment s's own
// contribution (run from the empty state) and g_s its total log forget gate
// (the sum of its chunks' g from the gate prep):
//   m' = max(g_s + m, m_s),  X' = e^{g_s + m - m'} X + e^{m_s - m'} X_s  (X = C, n).
// This is the inter-chunk recurrence of fw.py:115-133 applied to whole
// segments.  Block (head, part): lanes 0 .. P-2 sum their segment's g, lane 0
// runs the m recurrence, then one float4 of [C | n] per thread.
__global__ __launch_bounds__(256) void segment_combine_kernel(const float* __restrict__ prep, const float* __restrict__ ec,
                                                              const float* __restrict__ en, const float* __restrict__ em,
                                                              float* __restrict__ sc, float* __restrict__ sn,
                                                              float* __restrict__ sm, int P, int kc_per_seg, int NC,
                                                              int BNH, int DQK, int DV) {
  __shared__ float s_g[kMaxSegmentsDev], s_a[kMaxSegmentsDev], s_b[kMaxSegmentsDev];
  const int bh = blockIdx.y;
  const int t = threadIdx.x;
  if (t < P - 1) {
    float gsum = 0.f;
    const int c1 = min(NC, (t + 1) * kc_per_seg);
    for (int c = t * kc_per_seg; c < c1; ++c) gsum += prep[((size_t)bh * NC + c) * PREP_STRIDE + 256];
    s_g[t] = gsum;
  }
  __syncthreads();
  if (t == 0) {
    float m = em[bh];  // start(1) = E_0
    if (blockIdx.x == 0) sm[bh] = m;
    for (int sgi = 1; sgi + 1 < P; ++sgi) {
      const float ms = em[(size_t)sgi * BNH + bh];
      const float mn = fmaxf(s_g[sgi] + m, ms);
      s_a[sgi] = exp_(s_g[sgi] + m - mn);
      s_b[sgi] = exp_(ms - mn);
      m = mn;
      if (blockIdx.x == 0) sm[(size_t)sgi * BNH + bh] = m;
    }
  }
  __syncthreads();
  const size_t cst = (size_t)BNH * DQK * DV, nst = (size_t)BNH * DQK;
  const int per4 = (DQK * DV + DQK) / 4;  // float4 elements of [C | n] per head
  {
    const int e4 = blockIdx.x * 256 + t;
    if (e4 >= per4) return;
    const bool isc = e4 < DQK * DV / 4;
    const size_t off = isc ? (size_t)bh * DQK * DV + 4 * (size_t)e4 : (size_t)bh * DQK + 4 * (size_t)(e4 - DQK * DV / 4);
    const float* src = isc ? ec : en;
    float* dst = isc ? sc : sn;
    const size_t st = isc ? cst : nst;
    f32x4 x = *reinterpret_cast<const f32x4*>(src + off);
    *reinterpret_cast<f32x4*>(dst + off) = x;
    for (int sgi = 1; sgi + 1 < P; ++sgi) {
      x = s_a[sgi] * x + s_b[sgi] * *reinterpret_cast<const f32x4*>(src + sgi * st + off);
      *reinterpret_cast<f32x4*>(dst + sgi * st + off) = x;
    }
  }
}

// Workgroups the fused kernel needs to occupy an MI355X (256 CUs, one
// workgroup per CU).  With fewer (head, column tile) pairs the sequence is
// split into segments: P = min(256 / pairs, chunks / 4, 16).
constexpr int kTargetWorkgroups = 256;
constexpr int kMaxSegments = kMaxSegmentsDev;

static int segments_for(int B, int NH, int S, int DV, int max_seg) {
  const long long pairs = (long long)B * NH * (DV / DVT);
  const int NC = (S + L - 1) / L;
  if (pairs <= 0 || pairs >= kTargetWorkgroups || max_seg < 2) return 1;
  int P = (int)(kTargetWorkgroups / pairs);
  P = min(P, NC / 4);
  P = min(P, min(kMaxSegments, max_seg));
  return P < 2 ? 1 : P;
}

struct Layout {  // workspace: gate prep, then (split only) the end states and start states
  int P, kc_per_seg;
  size_t prep_bytes, states_bytes, total;
};

static size_t align256(size_t x) { return (x + 255) / 256 * 256; }

static Layout layout_for(int B, int NH, int S, int DQK, int DV, int max_seg) {
  Layout l;
  const int NC = (S + L - 1) / L;
  l.P = segments_for(B, NH, S, DV, max_seg);
  l.kc_per_seg = (NC + l.P - 1) / l.P;
  l.P = (NC + l.kc_per_seg - 1) / l.kc_per_seg;  // no empty segment
  l.prep_bytes = align256((size_t)B * NH * NC * PREP_STRIDE * sizeof(float));
  const size_t per = (size_t)B * NH * ((size_t)DQK * DV + DQK + 1);
  l.states_bytes = l.P > 1 ? align256((size_t)(l.P - 1) * per * sizeof(float)) : 0;
  l.total = l.prep_bytes + 2 * l.states_bytes;
  return l;
}

template <typename TG, int DQK>
static int launch(const ChunkwiseArgs& A) {
  const int BNH = A.B * A.NH;
  const int nvtile = A.DV / DVT;
  const int NC = (A.S + L - 1) / L;  // the last chunk may be ragged
  const Layout lay = layout_for(A.B, A.NH, A.S, A.DQK, A.DV, A.max_segments);
  hipStream_t st = (hipStream_t)A.stream;
  float* prep = (float*)A.workspace;
  const int total = BNH * NC;
  hipLaunchKernelGGL(gate_prep_kernel<TG>, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, st, (const TG*)A.i,
                     (const TG*)A.f, prep, total, NC, A.S);
  const size_t smem = Smem<DQK>::BYTES;
  if (!A.pipelined) {
    for (auto kern : {chunkwise_fused_kernel<DQK, false>, chunkwise_fused_kernel<DQK, true>}) {
      hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      if (e != hipSuccess)
        return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd: LDS attribute failed: %s", hipGetErrorString(e));
    }
  }
  // the main kernel: the pipelined schedule (chunkwise_pipe.hip) or the fused one
  auto main = [&](bool states_only, unsigned nwg, const MainArgs& m) -> int {
    if (A.pipelined) return pipe_launch(A.dtype_qkv == XL_DTYPE_F16, DQK, states_only, nwg, st, m);
    if (states_only)
      hipLaunchKernelGGL((chunkwise_fused_kernel<DQK, true>), dim3(nwg), dim3(NTHREADS), smem, st, m.q, m.k, m.v,
                         m.c0, m.n0, m.m0, m.h, m.c_last, m.n_last, m.m_last, m.prep, m.S, m.NC, m.DV, m.BNH,
                         m.nvtile, m.qk_scale, m.eps, m.sg);
    else
      hipLaunchKernelGGL((chunkwise_fused_kernel<DQK, false>), dim3(nwg), dim3(NTHREADS), smem, st, m.q, m.k, m.v,
                         m.c0, m.n0, m.m0, m.h, m.c_last, m.n_last, m.m_last, m.prep, m.S, m.NC, m.DV, m.BNH,
                         m.nvtile, m.qk_scale, m.eps, m.sg);
    return XL_OK;
  };
  const bf16_t *q = (const bf16_t*)A.q, *k = (const bf16_t*)A.k, *v = (const bf16_t*)A.v;
  SegArgs sg = {1, NC, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  if (lay.P > 1) {
    // pass 1: every segment but the last, states only (segment 0 from the caller's initial
    // state, the others from the empty state), end states into the workspace
    const size_t cst = (size_t)BNH * A.DQK * A.DV, nst = (size_t)BNH * A.DQK;
    char* base = (char*)A.workspace + lay.prep_bytes;
    float* ec = (float*)base;
    float* en = ec + (lay.P - 1) * cst;
    float* em = en + (lay.P - 1) * nst;
    float* scs = (float*)(base + lay.states_bytes);
    float* sns = scs + (lay.P - 1) * cst;
    float* sms = sns + (lay.P - 1) * nst;
    SegArgs s1 = {lay.P - 1, lay.kc_per_seg, nullptr, nullptr, nullptr, ec, en, em};
    const MainArgs m1 = {q, k, v, A.c0, A.n0, A.m0, nullptr, nullptr, nullptr, nullptr, prep,
                         A.S, NC, A.DV, BNH, nvtile, A.qk_scale, A.eps, s1, A.DQK};
    const int rc = main(true, (unsigned)(BNH * nvtile * (lay.P - 1)), m1);
    if (rc) return rc;
    const int per4 = (A.DQK * A.DV + A.DQK) / 4;
    hipLaunchKernelGGL(segment_combine_kernel, dim3((unsigned)((per4 + 255) / 256), (unsigned)BNH), dim3(256), 0,
                       st, prep, ec, en, em, scs, sns, sms, lay.P, lay.kc_per_seg, NC, BNH, A.DQK, A.DV);
    sg = SegArgs{lay.P, lay.kc_per_seg, scs, sns, sms, nullptr, nullptr, nullptr};
  }
  const MainArgs m2 = {q, k, v, A.c0, A.n0, A.m0, (bf16_t*)A.h, A.c_last, A.n_last, A.m_last, prep,
                       A.S, NC, A.DV, BNH, nvtile, A.qk_scale, A.eps, sg, A.DQK};
  const int rc = main(false, (unsigned)(BNH * nvtile * sg.nseg), m2);
  if (rc) return rc;
  return check_launch(A.pipelined ? "xl_mlstm_chunkwise_fwd(pipelined)" : "xl_mlstm_chunkwise_fwd(fused)");
}

template <typename TG>
static int launch_d(const ChunkwiseArgs& A) {  // the tile: 128 rows for DQK <= 128, else 256
  return A.DQK > 128 ? launch<TG, 256>(A) : launch<TG, 128>(A);
}

}  // namespace fused

size_t chunkwise_fused_workspace(int B, int NH, int S, int DQK, int DV, int max_segments) {
  return fused::layout_for(B, NH, S, DQK, DV, max_segments).total;
}

int chunkwise_fused_segments(int B, int NH, int S, int DQK, int DV, int max_segments) {
  return fused::layout_for(B, NH, S, DQK, DV, max_segments).P;
}

bool chunkwise_fused_supported(const ChunkwiseArgs& a, const char** why, bool pipelined) {
  const char* r = nullptr;
  // the pipelined kernel also takes a DQK below its 128 / 256 tile that is a whole number of
  // state-wave row blocks (32 / 64 rows): the rows and columns past it stay zero
  const bool dqk_pipe = a.DQK <= 128 ? (a.DQK >= 32 && a.DQK % 32 == 0) : (a.DQK <= 256 && a.DQK % 64 == 0);
  if (pipelined && a.dtype_qkv != XL_DTYPE_BF16 && a.dtype_qkv != XL_DTYPE_F16) r = "q/k/v must be bfloat16 or float16";
  else if (!pipelined && a.dtype_qkv != XL_DTYPE_BF16) r = "q/k/v must be bfloat16 (float16 runs the pipelined schedule)";
  else if (pipelined && !dqk_pipe) r = "DQK must be 32, 64, 96, 128, 192 or 256";
  else if (!pipelined && a.DQK != 128 && a.DQK != 256) r = "DQK must be 128 or 256 (32, 64, 96 and 192 run the pipelined schedule)";
  else if (a.DV % fused::DVT != 0) r = "DV must be a multiple of 64";
  if (why) *why = r;
  return r == nullptr;
}

int chunkwise_fused(const ChunkwiseArgs& a) {
  switch (a.dtype_gates) {
    case XL_DTYPE_F32: return fused::launch_d<float>(a);
    case XL_DTYPE_BF16: return fused::launch_d<bf16_t>(a);
    default: return fused::launch_d<f16_t>(a);
  }
}

}  // namespace xl
