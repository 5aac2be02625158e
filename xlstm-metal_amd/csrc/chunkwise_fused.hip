// Fused single-pass chunkwise mLSTM forward for bf16 q/k/v on gfx950.
//
// One workgroup = one (b, h) pair x one 64-column tile of DV, marching over
// the NC chunks of L = 64 tokens.  The C tile (DQK x 64, float32) and the
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
// The normaliser rides along as a fifth 16-column tile: C carries n in its
// column 64, V carries a row of ones and alpha V carries alpha_t, so n', q.n
// and the row sums come out of the same MFMAs as C', q C and M V, and den_i
// lands in column 64 of H_i.
//
// Producer / consumer split (8 waves, two per SIMD):
//  * state waves 0..3: wave s owns rows [s*DW, (s+1)*DW) of [C | n]
//    (DW = DQK/4, float32 accumulators).  Per chunk it first forms the
//    partial product Q[:, rows] [C | n][rows, :] for all 64 tokens, with the
//    B operand built straight from its accumulators as bf16 hi + lo (two
//    MFMAs, so q C keeps float32 accuracy), and leaves it in LDS.  It then
//    applies the chunk update [C | n] += K^T (alpha [V | 1]) with alpha V
//    split into bf16 hi + lo, so the state keeps float32 accuracy too.
//  * output waves 4..7: wave o owns output rows [16o, 16o+16) of every chunk:
//    exact S^T = K Q^T over the whole DQK, gating and M [V | 1] (M split
//    hi + lo); after the chunk's second barrier it adds the four partial
//    Q [C | n] rows and writes h.
// The state never leaves the state waves' registers; the only cross-wave
// traffic besides the staged q/k/v tiles is the 16-byte-per-lane partials.
// All products are v_mfma_f32_16x16x32_bf16.  K^T and V operands are read
// with ds_read_b64_tr_b16 from the natural row-major tiles (within 16 lanes,
// output lane 4a+c receives element c of source lanes 4k+a, k = 0..3), with
// the token order inside a k-slice chosen so that every LDS access pattern is
// free of bank conflicts.
//
// The forget rescale exp(g + m - m') of C is deferred: the state is stored as
// C e^{-G} (G = accumulated log rescale), the factor e^{-G} is folded into
// alpha V and e^{G} into the output row scale, and C is renormalised only
// when G drops below -30 (the eager path).
//
// Grid mapping is XCD aware: the DV tiles of one head land on the same XCD so
// the head's q/k chunks are fetched from HBM once and then hit that XCD's L2.
#include "chunkwise.h"

namespace xl {
namespace fused {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int L = 64;           // chunk size (= wavefront size: one lane per token)
constexpr int NSW = 4;          // state waves
constexpr int NOW = 4;          // output waves
constexpr int NTHREADS = 64 * (NSW + NOW);
constexpr int DVT = 64;         // DV columns per workgroup
constexpr int NVT = DVT / 16;   // 16-wide column tiles of v
constexpr int NVX = NVT + 1;    // ... plus the n / ones / den tile
constexpr int VN_PITCH = 160;   // bytes per row of natural V (8 consecutive rows -> distinct 32 B bank groups)
constexpr int AV_PITCH = 160;   // bytes per row of natural alpha' [V | n] (80 columns; 2-row steps hit distinct banks)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float RENORM = -30.f; // renormalise the stored state when the deferred log rescale drops below this
constexpr int PREP_STRIDE = 320;  // floats per chunk of gate prep: b, a, cummax(i - b), (i - b) log2e, [g, max a]
constexpr int GROWS = 6;          // shared gate rows per chunk: bl, ul, qbar, mc, alpha', [renorm scale, m', G]

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// bf16 hi + lo split of 8 floats: hi = bf16(x), lo = bf16(x - hi)
__device__ __forceinline__ void split8(f32x4 a, f32x4 b, bf16x8& hi, bf16x8& lo) {
  const u32x4 h = {pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3])};
  const u32x4 l = {pack_bf16(a[0] - bf_lo(h[0]), a[1] - bf_hi(h[0])), pack_bf16(a[2] - bf_lo(h[1]), a[3] - bf_hi(h[1])),
                   pack_bf16(b[0] - bf_lo(h[2]), b[1] - bf_hi(h[2])), pack_bf16(b[2] - bf_lo(h[3]), b[3] - bf_hi(h[3]))};
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}
__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float exp_(float x) { return __builtin_amdgcn_exp2f(x * LOG2E); }
// log(sigmoid(x)) = min(x, 0) - log(1 + exp(-|x|)) via the hardware exp2/log2 (abs. error < 1e-7)
__device__ __forceinline__ float logsig_fast(float x) {
  return fminf(x, 0.f) - LN2 * __builtin_amdgcn_logf(1.0f + exp2_(-fabsf(x) * LOG2E));
}
// two 64-bit transposed LDS reads -> one 8 x bf16 MFMA operand
__device__ __forceinline__ bf16x8 tr8(const char* p0, const char* p1) {
  const i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p0);
  const i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p1);
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  const u32x4 r = {ua[0], ua[1], ub[0], ub[1]};
  return __builtin_bit_cast(bf16x8, r);
}

// Inclusive wave64 scans with DPP (row shifts, then row broadcasts).
template <bool MAX>
__device__ __forceinline__ float wave_scan(float x) {
  const int iid = __float_as_int(MAX ? -INFINITY : 0.f);
#define XL_SCAN_STEP(CTRL, ROWMASK)                                                                                 \
  {                                                                                                                 \
    const float y = __int_as_float(__builtin_amdgcn_update_dpp(iid, __float_as_int(x), CTRL, ROWMASK, 0xf, false)); \
    x = MAX ? fmaxf(x, y) : x + y;                                                                                  \
  }
  XL_SCAN_STEP(0x111, 0xf)  // row_shr:1
  XL_SCAN_STEP(0x112, 0xf)  // row_shr:2
  XL_SCAN_STEP(0x114, 0xf)  // row_shr:4
  XL_SCAN_STEP(0x118, 0xf)  // row_shr:8
  XL_SCAN_STEP(0x142, 0xa)  // row_bcast:15 into rows 1, 3
  XL_SCAN_STEP(0x143, 0xc)  // row_bcast:31 into rows 2, 3
#undef XL_SCAN_STEP
  return x;
}

__device__ __forceinline__ float lane63(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// Chunk-local gate prep, one wave per (head, chunk), lane = token t
// (fw.py:308-316 and :98, :204-213 before the running stabiliser enters):
//   b_t = sum_{s<=t} logsig f_s,  g = b_63,  a_t = g - b_t + i_t,  max_t a_t,
//   u_t = i_t - b_t (stored times log2 e),  cummax_{s<=t} u_s.
// These are the scans of the chunk; the main kernel folds in the running m
// and the deferred state rescale with a handful of scalar operations.
template <typename TG>
__global__ __launch_bounds__(256) void gate_prep_kernel(const TG* __restrict__ ig, const TG* __restrict__ fg,
                                                        float* __restrict__ prep, int total_chunks) {
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);  // bh * NC + chunk: the tokens of chunk c are 64c .. 64c + 63
  if (c >= total_chunks) return;
  const float f = to_f32(fg[(size_t)c * L + lane]), i = to_f32(ig[(size_t)c * L + lane]);
  const float b = wave_scan<false>(logsig_fast(f));
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

// Column of the 64-wide DV tile held by column n of 16-wide tile vq (vq < 4):
// runs of 4 consecutive columns, and the tile pair (2h, 2h+1) covers columns
// 32h .. 32h+31 so that a lane of the transposed output holds 8 consecutive
// columns (one 16-byte store).
__device__ __forceinline__ int vcol_of(int vq, int n) { return 32 * (vq >> 1) + 8 * (n >> 2) + 4 * (vq & 1) + (n & 3); }
// First of the 4 consecutive natural columns of alpha' [V | n] that source
// lane 4k + a of a transposed read of column tile vq fetches: the V columns of
// tile vq (vq < 4), or the n tile's columns 64 + 4a .. 64 + 4a + 3.
__device__ __forceinline__ int avcol(int vq, int a) { return vq < NVT ? vcol_of(vq, 4 * a) : 64 + 4 * a; }

template <int DQK>
struct Smem {
  static constexpr int KPD = DQK / 32;                   // 32-deep k-steps over DQK
  static constexpr int KN_PITCH = DQK * 2 + 16;          // bytes per K row: 16 consecutive rows -> distinct 16 B groups
  static constexpr int KN = 0;                           // [64 t][KN_PITCH]: K natural
  static constexpr int VN = KN + 64 * KN_PITCH;          // [64 t][VN_PITCH]: V natural
  static constexpr int AVH = VN + 64 * VN_PITCH;         // [64 t][AV_PITCH]: alpha' [V | n] hi, natural
  static constexpr int AVL = AVH + 64 * AV_PITCH;        // ... lo
  static constexpr int HP = AVL + 64 * AV_PITCH;         // [4 state waves][4 row tiles][NVX][64] f32x4: partial Q [C | n]
  static constexpr int GATES = HP + 4 * 4 * NVX * 64 * 16;  // [2 chunks][GROWS][64] float: gate rows + scalars
  static constexpr int BYTES = GATES + 2 * GROWS * 64 * 4;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

template <int DQK>
__global__ __launch_bounds__(NTHREADS, 1) void chunkwise_fused_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const float* __restrict__ c0,
    const float* __restrict__ n0, const float* __restrict__ m0, bf16_t* __restrict__ h,
    float* __restrict__ c_last, float* __restrict__ n_last, float* __restrict__ m_last,
    const float* __restrict__ prep, int NC, int DV, int BNH, int nvtile, float qk_scale, float eps) {
  using SM = Smem<DQK>;
  constexpr int KPD = SM::KPD;
  constexpr int DW = DQK / NSW;   // C rows per state wave (64 or 32)
  constexpr int NDT = DW / 16;    // C row tiles per state wave
  constexpr int NKU = DQK / 64;   // K staging: 16-byte pieces per thread (64 rows x DQK / 512 threads / 8)
  constexpr int KS = DW / 32;     // 32-deep k-steps over a state wave's rows
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int ws = w & 3;  // index within the state or output group

  // ---- XCD-aware workgroup -> (head, column tile): consecutive tiles of a head share an XCD
  const int nwg = BNH * nvtile;
  int lin = blockIdx.x;
  if ((nwg & 7) == 0) lin = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int bh = lin / nvtile;
  const int v0 = (lin - bh * nvtile) * DVT;
  const int S = NC * L;

  char* kn = smem + SM::KN;
  char* vn = smem + SM::VN;
  char* avh = smem + SM::AVH;
  char* avl = smem + SM::AVL;
  f32x4* hp = (f32x4*)(smem + SM::HP);
  float* gbuf = (float*)(smem + SM::GATES);  // [2][GROWS][64]: rows of chunk kc live in buffer kc & 1

  // n-tile columns 64..79 of alpha' [V | n]: zeros, except columns 64, 68, 72,
  // 76, which carry alpha' itself and are rewritten every chunk
  for (int e = tid; e < 64 * 8; e += NTHREADS) {
    reinterpret_cast<uint32_t*>(avh + (e >> 3) * AV_PITCH + 128)[e & 7] = 0u;
    reinterpret_cast<uint32_t*>(avl + (e >> 3) * AV_PITCH + 128)[e & 7] = 0u;
  }

  const bf16_t* qh = q + (size_t)bh * S * DQK;
  const bf16_t* kh = k + (size_t)bh * S * DQK;
  const bf16_t* vh = v + (size_t)bh * S * DV;
  bf16_t* hh = h + (size_t)bh * S * DV;
  const float m_init = m0 ? m0[bh] : 0.f;

  // ---- K staging: piece u of thread tid = u*NTHREADS + tid -> row piece / (DQK/8), 16-byte column group
  auto load_k = [&](int kc, u32x4 (&Kst)[NKU]) {
    const bf16_t* kb = kh + (size_t)kc * L * DQK;
#pragma unroll
    for (int u = 0; u < NKU; ++u) {
      const int piece = u * NTHREADS + tid;
      Kst[u] = *reinterpret_cast<const u32x4*>(kb + (size_t)(piece / (DQK / 8)) * DQK + 8 * (piece % (DQK / 8)));
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
  // stored state, m', the deferred log rescale G and the renormalise flag.
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
    gb[256 + lane] = exp_(a - m_next - Gn);            // alpha' = exp(a_t - m') e^{-G}
    if (lane == 0) {
      gb[320] = exp_(gG + lg);  // may underflow to 0: the old state is then negligible
      gb[321] = m_next;
      gb[322] = Gn;
      gb[323] = renorm ? 1.f : 0.f;
    }
    gm = m_next;
    gG = Gn;
  };
  if (w == NSW) {
    float pv[5];
    prep_load(0, pv);
    gate_rows(0, pv);
  }
  __syncthreads();  // B0: gate rows of chunk 0

  if (w < NSW) {
    // =====================================================================
    // state waves: rows [dw0, dw0 + DW) of [C | n], stored as C e^{-G}
    // =====================================================================
    // Row 4a + c of accumulator tile dt holds state row d = dw0 + 32 (dt >> 1) +
    // 8a + 4 (dt & 1) + c: each tile's rows come in runs of 4 consecutive d (what
    // a transposed K read delivers), and the tile pair (2p, 2p+1) covers the 32
    // consecutive d = dw0 + 32p .. +31 in k order, so q fragments are one
    // 16-byte load.
    const int dw0 = ws * DW;
    auto crow = [&](int dt, int a, int c) { return dw0 + 32 * (dt >> 1) + 8 * a + 4 * (dt & 1) + c; };
    f32x4 Cacc[NDT][NVX];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = crow(dt, g, e);  // accumulator row 4g+e of tile dt
#pragma unroll
        for (int vq = 0; vq < NVT; ++vq)
          Cacc[dt][vq][e] = c0 ? c0[((size_t)bh * DQK + d) * DV + v0 + vcol_of(vq, r16)] : 0.f;
        // n is replicated in columns 0, 4, 8, 12 of the fifth tile
        Cacc[dt][NVT][e] = (n0 && (r16 & 3) == 0) ? n0[(size_t)bh * DQK + d] : 0.f;
      }

    // V staging (state threads): rows t0 = 4*(tid>>4) + ((tid>>3)&1) and t0 + 2, columns 8*(tid&7)
    const int vrow = 4 * (tid >> 4) + ((tid >> 3) & 1), vcol = 8 * (tid & 7);
    u32x4 Kst[NKU], Vst[2];
    // q fragments of this wave's k range for every row: rows 16rt + r16, columns
    // dw0 + 32p + 8g .. +7 -- the k order of the B fragments that
    // split8(Cacc[2p], Cacc[2p+1]) yields
    u32x4 Qs[4][KS];
    auto load_v = [&](int kc) {
      const bf16_t* vb = vh + (size_t)kc * L * DV + v0 + vcol;
      Vst[0] = *reinterpret_cast<const u32x4*>(vb + (size_t)vrow * DV);
      Vst[1] = *reinterpret_cast<const u32x4*>(vb + (size_t)(vrow + 2) * DV);
    };
    auto load_qs = [&](int kc) {
      const bf16_t* qb = qh + ((size_t)kc * L + r16) * DQK + dw0 + 8 * g;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int p = 0; p < KS; ++p) Qs[rt][p] = *reinterpret_cast<const u32x4*>(qb + (size_t)16 * rt * DQK + 32 * p);
    };
    load_k(0, Kst);
    load_v(0);
    load_qs(0);
    for (int kc = 0; kc < NC; ++kc) {
      const float* gb = gbuf + (kc & 1) * GROWS * 64;
      store_k(Kst);
      // V natural and alpha' V hi / lo (natural layout, 16-byte rows)
      *reinterpret_cast<u32x4*>(vn + vrow * VN_PITCH + 2 * vcol) = Vst[0];
      *reinterpret_cast<u32x4*>(vn + (vrow + 2) * VN_PITCH + 2 * vcol) = Vst[1];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const float al = gb[256 + vrow + 2 * r];
        u32x4 hv, lv;
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          const float x0 = al * bf_lo(Vst[r][c2]), x1 = al * bf_hi(Vst[r][c2]);
          hv[c2] = pack_bf16(x0, x1);
          lv[c2] = pack_bf16(x0 - bf_lo(hv[c2]), x1 - bf_hi(hv[c2]));
        }
        *reinterpret_cast<u32x4*>(avh + (vrow + 2 * r) * AV_PITCH + 2 * vcol) = hv;
        *reinterpret_cast<u32x4*>(avl + (vrow + 2 * r) * AV_PITCH + 2 * vcol) = lv;
      }
      __syncthreads();  // B1: the chunk's tiles are visible; the previous chunk's partials have been read
      if (kc + 1 < NC) {  // staging registers are free: prefetch (q after its last use below)
        load_k(kc + 1, Kst);
        load_v(kc + 1);
      }
      // partial Q [C | n] over this wave's rows, with the state before this chunk
      // (bf16 hi + lo of the float32 accumulators, so q C keeps float32 accuracy).
      // Transposed product [C | n]^T Q^T: lane (g, r16) gets columns 4g+e of
      // token 16rt + r16.  Software pipelined: the split of tile vq+1 (VALU) is
      // interleaved with the MFMAs of tile vq, and tile vq's partials are stored
      // one tile later, when its MFMAs have retired.
      {
        bf16x8 bsp[2][KS][2];
        f32x4 Hp[2][4];
#pragma unroll
        for (int p = 0; p < KS; ++p) split8(Cacc[2 * p][0], Cacc[2 * p + 1][0], bsp[0][p][0], bsp[0][p][1]);
#pragma unroll
        for (int vq = 0; vq < NVX; ++vq) {
          const int cur = vq & 1;
          if (vq + 1 < NVX) {
#pragma unroll
            for (int p = 0; p < KS; ++p)
              split8(Cacc[2 * p][vq + 1], Cacc[2 * p + 1][vq + 1], bsp[cur ^ 1][p][0], bsp[cur ^ 1][p][1]);
          }
#pragma unroll
          for (int rt = 0; rt < 4; ++rt) Hp[cur][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < KS; ++p)
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
              Hp[cur][rt] = mfma(bsp[cur][p][0], __builtin_bit_cast(bf16x8, Qs[rt][p]), Hp[cur][rt]);
              Hp[cur][rt] = mfma(bsp[cur][p][1], __builtin_bit_cast(bf16x8, Qs[rt][p]), Hp[cur][rt]);
            }
          if (vq > 0) {
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) hp[((ws * 4 + rt) * NVX + vq - 1) * 64 + lane] = Hp[cur ^ 1][rt];
          }
          // ask the scheduler for 1 MFMA : 3 VALU, then the stores
#pragma unroll
          for (int u = 0; u < 8 * KS; ++u) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x200, 4, 0);
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) hp[((ws * 4 + rt) * NVX + NVX - 1) * 64 + lane] = Hp[(NVX - 1) & 1][rt];
      }
      if (kc + 1 < NC) load_qs(kc + 1);
      if (gb[323] != 0.f) {  // renormalise the stored state (wave-uniform)
        const float sc = gb[320];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int vq = 0; vq < NVX; ++vq) Cacc[dt][vq] *= sc;
      }
      // K^T fragments of all this wave's row tiles stay in registers, so every
      // alpha' [V | n] fragment is read from LDS once per wave
      bf16x8 Ka[NDT][2];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          // source lane 4k+a of group g: token 32p + 8g + 2k (+1), state rows crow(dt, a, 0 .. 3)
          const char* base = kn + (32 * p + 8 * g + 2 * (r16 >> 2)) * SM::KN_PITCH + 2 * crow(dt, r16 & 3, 0);
          Ka[dt][p] = tr8(base, base + SM::KN_PITCH);
        }
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          // source lane 4k+a of group g: token 32p + 8g + 2k (+1) -- the token order
          // of the K^T operand -- and 4 consecutive columns from avcol(vq, a)
          const int off = (32 * p + 8 * g + 2 * (r16 >> 2)) * AV_PITCH + 2 * avcol(vq, r16 & 3);
          const bf16x8 bh = tr8(avh + off, avh + off + AV_PITCH);
          const bf16x8 bl = tr8(avl + off, avl + off + AV_PITCH);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            Cacc[dt][vq] = mfma(Ka[dt][p], bh, Cacc[dt][vq]);
            Cacc[dt][vq] = mfma(Ka[dt][p], bl, Cacc[dt][vq]);
          }
        }
      __syncthreads();  // B2: partials complete; the chunk's tiles may be overwritten
    }
    // ---- final states (undo the deferred rescale)
    if (c_last) {
      const float* gl = gbuf + ((NC - 1) & 1) * GROWS * 64;
      const float sc = exp_(gl[322]);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = crow(dt, g, e);
#pragma unroll
          for (int vq = 0; vq < NVT; ++vq)
            c_last[((size_t)bh * DQK + d) * DV + v0 + vcol_of(vq, r16)] = Cacc[dt][vq][e] * sc;
          if (v0 == 0 && r16 == 0) n_last[(size_t)bh * DQK + d] = Cacc[dt][NVT][e] * sc;
        }
      if (v0 == 0 && tid == 0) m_last[bh] = gl[321];
    }
  } else {
    // =====================================================================
    // output waves: rows [16o, 16o + 16) of every chunk
    // =====================================================================
    const int o = ws;
    u32x4 Kst[NKU], Qf[KPD];
    float pv[5];  // gate prep of the next chunk (gate wave)
    // q fragments of rows 16o + r16 for S: k-slice 32p + 8g .. 32p + 8g + 7 (one
    // 16-byte load; the K operand below uses the same contiguous k order)
    auto load_q = [&](int kc) {
      const bf16_t* qb = qh + ((size_t)kc * L + 16 * o + r16) * DQK + 8 * g;
#pragma unroll
      for (int p = 0; p < KPD; ++p) Qf[p] = *reinterpret_cast<const u32x4*>(qb + 32 * p);
    };
    load_k(0, Kst);
    load_q(0);
    for (int kc = 0; kc < NC; ++kc) {
      const float* gb = gbuf + (kc & 1) * GROWS * 64;
      store_k(Kst);
      if (o == 0) {  // columns 64, 68, 72, 76 of alpha' [V | n], token `lane`: alpha' itself (n replicated 4x)
        const float al = gb[256 + lane];
        const uint32_t hv = pack_bf16(al, 0.f);
        const uint16_t lo = (uint16_t)pack_bf16(al - bf_lo(hv), 0.f);
#pragma unroll
        for (int c = 64; c < 80; c += 4) {
          reinterpret_cast<uint16_t*>(avh + lane * AV_PITCH)[c] = (uint16_t)hv;
          reinterpret_cast<uint16_t*>(avl + lane * AV_PITCH)[c] = lo;
        }
      }
      __syncthreads();  // B1
      if (kc + 1 < NC) {
        load_k(kc + 1, Kst);
        if (o == 0) prep_load(kc + 1, pv);
      }

      // S^T tiles of all four j-tiles over the whole DQK: A = K rows 16jt + r16,
      // B = q rows.  Every output wave computes all four (tiles above the
      // diagonal are masked in the gating), so the code is branch-free; the
      // busiest SIMD (the wave of the last row tile) does the same work as
      // before.  All K fragments are requested up front: LDS latency is many
      // times the four MFMAs of one k-step.
      f32x4 Sacc[4];
      constexpr int KD = 2;
      u32x4 kf[KD][4];
#pragma unroll
      for (int p = 0; p < KD - 1; ++p)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          kf[p][jt] = *reinterpret_cast<const u32x4*>(kn + (16 * jt + r16) * SM::KN_PITCH + 16 * g + 64 * p);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) Sacc[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < KPD; ++p) {
        if (p + KD - 1 < KPD) {
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
            kf[(p + KD - 1) % KD][jt] = *reinterpret_cast<const u32x4*>(kn + (16 * jt + r16) * SM::KN_PITCH + 16 * g + 64 * (p + KD - 1));
        }
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          Sacc[jt] = mfma(__builtin_bit_cast(bf16x8, kf[p % KD][jt]), __builtin_bit_cast(bf16x8, Qf[p]), Sacc[jt]);
      }
      if (kc + 1 < NC) load_q(kc + 1);  // q fragments are dead: prefetch
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
      // the gate wave forms the gate rows of chunk kc + 1 (buffer (kc + 1) & 1,
      // last read before B1 of this chunk)
      if (o == 0 && kc + 1 < NC) gate_rows(kc + 1, pv);
      __syncthreads();  // B2: the state waves' partial Q [C | n] of this chunk are complete
      // Q [C | n] of rows 16o + 4g + e: sum of the four state waves' partials
      f32x4 Hqc[NVX];
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq) {
        Hqc[vq] = hp[((0 * 4 + o) * NVX + vq) * 64 + lane];
#pragma unroll
        for (int sw = 1; sw < NSW; ++sw) Hqc[vq] += hp[((sw * 4 + o) * NVX + vq) * 64 + lane];
      }
      // finish row 16o + r16: this lane holds columns vcol_of(vq, 4g + e), i.e. the
      // 8 consecutive columns 32h + 8g .. +7 of tiles (2h, 2h+1); the denominator
      // (n / ones replicated in rows 0, 4, 8, 12 of the fifth tile) is element 0
      const float qb = gb[128 + 16 * o + r16];
      const float mcr = gb[192 + 16 * o + r16];
      const float den = qb * Hqc[NVT][0] + Hmv[NVT][0];
      const float inv = __builtin_amdgcn_rcpf(fmaxf(fabsf(den), exp_(-mcr)) + eps);
      bf16_t* hb = hh + ((size_t)kc * L + 16 * o + r16) * DV + v0 + 8 * g;
#pragma unroll
      for (int h2 = 0; h2 < NVT / 2; ++h2) {
        u32x4 out;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int vq = 2 * h2 + b;
          out[2 * b] = pack_bf16((qb * Hqc[vq][0] + Hmv[vq][0]) * inv, (qb * Hqc[vq][1] + Hmv[vq][1]) * inv);
          out[2 * b + 1] = pack_bf16((qb * Hqc[vq][2] + Hmv[vq][2]) * inv, (qb * Hqc[vq][3] + Hmv[vq][3]) * inv);
        }
        *reinterpret_cast<u32x4*>(hb + 32 * h2) = out;
      }
    }
  }
}

template <typename TG, int DQK>
static int launch(const ChunkwiseArgs& A) {
  const int BNH = A.B * A.NH;
  const int nvtile = A.DV / DVT;
  const int NC = A.S / L;
  float* prep = (float*)A.workspace;
  const int total = BNH * NC;
  hipLaunchKernelGGL(gate_prep_kernel<TG>, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, (hipStream_t)A.stream,
                     (const TG*)A.i, (const TG*)A.f, prep, total);
  auto kern = chunkwise_fused_kernel<DQK>;
  const size_t smem = Smem<DQK>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess)
    return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd: LDS attribute failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(kern, dim3((unsigned)(BNH * nvtile)), dim3(NTHREADS), smem, (hipStream_t)A.stream,
                     (const bf16_t*)A.q, (const bf16_t*)A.k, (const bf16_t*)A.v, A.c0, A.n0, A.m0, (bf16_t*)A.h,
                     A.c_last, A.n_last, A.m_last, prep, NC, A.DV, BNH, nvtile, A.qk_scale, A.eps);
  return check_launch("xl_mlstm_chunkwise_fwd(fused)");
}

template <typename TG>
static int launch_d(const ChunkwiseArgs& A) {
  return A.DQK == 256 ? launch<TG, 256>(A) : launch<TG, 128>(A);
}

}  // namespace fused

size_t chunkwise_fused_workspace(int B, int NH, int S) {
  return ((size_t)B * NH * (S / fused::L) * fused::PREP_STRIDE * sizeof(float) + 255) / 256 * 256;
}

bool chunkwise_fused_supported(const ChunkwiseArgs& a, const char** why) {
  const char* r = nullptr;
  if (a.dtype_qkv != XL_DTYPE_BF16) r = "q/k/v must be bfloat16";
  else if (a.S % fused::L != 0) r = "sequence length must be a multiple of 64";
  else if (a.DQK != 128 && a.DQK != 256) r = "DQK must be 128 or 256";
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
