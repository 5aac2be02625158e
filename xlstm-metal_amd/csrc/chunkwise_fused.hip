// Fused single-pass chunkwise mLSTM forward for bf16 q/k/v on gfx950.
//
// One workgroup = one (b, h) pair x one 64-column tile of DV; it marches over
// the NC chunks of L = 64 tokens keeping its C tile (DQK x 64, float32) and
// the normaliser n (DQK) in registers, so the only HBM traffic is q, k, v, the
// gates, h and the final states (no per-chunk state round trip).  The math is
// the reference's chunkwise forward (kernel_development/xlstm/mlstm_block/
// mlstm_chunkwise/vendored/torch/native/fw.py:98-143 for the inter-chunk
// recurrence, :193-245 for the outputs), fused per chunk:
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
// column 64, V carries a row of ones (for sum_j M_ij) and alpha V carries
// alpha_t (for sum_t alpha_t k_t), so n', q.n and the row sums are produced by
// the same MFMAs as C', q C and M V, and den_i lands in column 64 of H_i.
//
// Work split (4 waves, 256 threads): wave w owns rows [w*DW, (w+1)*DW) of C
// (DW = DQK/4).  Per chunk each wave computes, over its slice of the DQK
// contraction, a partial S^T = K Q^T and a partial Q [C | n]; the S partials
// are summed through LDS so that wave w gates the exact scores of its own 16
// output rows and multiplies them with V; the Q [C | n] partials are summed
// through LDS the same way before the output rows are finished.  All dense
// products are v_mfma_f32_16x16x32_bf16 with float32 accumulation:
//   S^T  (j x i, over d)   A = K rows (LDS),        B = q rows (registers)
//   QC   (i x v, over d)   A = q rows (registers),  B = [C | n] (accumulators -> bf16)
//   MV   (i x v, over j)   A = M hi + lo,           B = [V | 1]^T (LDS)
//   KV   (d x v, over t)   A = K^T (LDS),           B = (alpha [V | 1])^T hi + lo (LDS)
// Operands coming from accumulators use a row permutation: the 16 rows of an
// MFMA tile are mapped to physical indices so that the 4 rows a lane holds in
// two adjacent tiles are 8 consecutive indices, i.e. exactly the 8-element
// k-slice that lane must supply when the accumulator is reused as an operand.
// alpha_t v_t and the gated scores are split into bf16 hi + lo parts (two
// MFMAs) so the float32 state and the outputs do not inherit bf16 rounding of
// those products; [C | n] is rounded to bf16 only as the operand of Q [C | n].
//
// Grid mapping is XCD aware: the DV tiles of one head land on the same XCD so
// the head's q/k chunks are fetched from HBM once and then hit that XCD's L2.
#include "chunkwise.h"

namespace xl {
namespace fused {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int L = 64;          // chunk size (= wavefront size: one lane per token)
constexpr int NW = 4;          // waves per workgroup
constexpr int NTHREADS = NW * 64;
constexpr int DVT = 64;        // DV columns per workgroup
constexpr int NVT = DVT / 16;  // 16-wide column tiles of v
constexpr int NVX = NVT + 1;   // ... plus the n / ones / den tile
constexpr int PITCH = 72;      // bf16 per LDS row (144 B): 16 consecutive rows hit distinct banks
constexpr int NST = 12;        // causal S^T tiles (jt, it) with jt/2 <= it/2
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ bf16x8 pack8(f32x4 a, f32x4 b) {
  u32x4 r = {pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3])};
  return __builtin_bit_cast(bf16x8, r);
}
// bf16 hi + lo split of 8 floats: hi = bf16(x), lo = bf16(x - hi)
__device__ __forceinline__ void split8(f32x4 a, f32x4 b, bf16x8& hi, bf16x8& lo) {
  const u32x4 h = {pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3])};
  const u32x4 l = {pack_bf16(a[0] - bf_lo(h[0]), a[1] - bf_hi(h[0])), pack_bf16(a[2] - bf_lo(h[1]), a[3] - bf_hi(h[1])),
                   pack_bf16(b[0] - bf_lo(h[2]), b[1] - bf_hi(h[2])), pack_bf16(b[2] - bf_lo(h[3]), b[3] - bf_hi(h[3]))};
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}
__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }
// log(sigmoid(x)) = min(x, 0) - log(1 + exp(-|x|)) via the hardware exp2/log2;
// absolute error < 1e-7.
__device__ __forceinline__ float logsig_fast(float x) {
  return fminf(x, 0.f) - LN2 * __builtin_amdgcn_logf(1.0f + exp2_(-fabsf(x) * LOG2E));
}

// Inclusive wave64 scans with DPP (row shifts, then row broadcasts).
template <bool MAX>
__device__ __forceinline__ float wave_scan(float x) {
  const float ident = MAX ? -INFINITY : 0.f;
  const int iid = __float_as_int(ident);
#define XL_SCAN_STEP(CTRL, ROWMASK)                                                                     \
  {                                                                                                     \
    const float y = __int_as_float(__builtin_amdgcn_update_dpp(iid, __float_as_int(x), CTRL, ROWMASK, 0xf, false)); \
    x = MAX ? fmaxf(x, y) : x + y;                                                                      \
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

// LDS row of physical index x within a 64-row block: tiles of 16 rows, each
// tile pair (32 indices) interleaved so that lane group g of a tile pair
// covers indices 8g..8g+7 (4 in each tile).
__device__ __forceinline__ int lds_row(int x) {
  return 32 * (x >> 5) + 16 * ((x >> 2) & 1) + 4 * ((x >> 3) & 3) + (x & 3);
}
// physical index held by accumulator element e of lane group g in tile `tile`
__device__ __forceinline__ int phys(int tile, int g, int e) { return 32 * (tile >> 1) + 8 * g + 4 * (tile & 1) + e; }
// slot of causal S^T tile (jt, it), jt/2 <= it/2
__device__ __forceinline__ constexpr int st_slot(int it, int jt) { return it < 2 ? 2 * it + jt : 4 + 4 * (it - 2) + jt; }

template <int DQK>
struct Smem {
  static constexpr int DW = DQK / NW;                          // C rows per wave
  static constexpr int KN_SLOT = NST * 64 * 16;                 // per wave: K natural tile, then its S^T partials
  static_assert(64 * PITCH * 2 <= KN_SLOT, "K tile must fit its slot");
  static constexpr int KT_SLOT = DW * PITCH * 2;                // per wave: K^T tile
  static constexpr int VTILE = 80 * PITCH * 2;                  // [80][PITCH] bf16
  static constexpr int HRED_BYTES = NW * 3 * NVX * 64 * 16;     // [NW][3][NVX][64] f32x4
  static constexpr int KN = 0;                                  // [NW][KN_SLOT]
  static constexpr int KT = KN + NW * KN_SLOT;                  // [NW][KT_SLOT]
  static constexpr int VBH = KT + NW * KT_SLOT;                 // (alpha [V | 1])^T hi
  static constexpr int VBL = VBH + VTILE;                       // ... lo
  // Q [C | n] partials alias K^T and alpha V (dead once the state update is done)
  static constexpr int HRED = KT;
  static constexpr int VT = (VBL + VTILE > HRED + HRED_BYTES) ? VBL + VTILE : HRED + HRED_BYTES;  // [V | 1]^T
  static constexpr int GATES = VT + VTILE;                      // [NW][5][64] float: per-wave gate rows
  static constexpr int BYTES = GATES + NW * 5 * 64 * 4;
};

template <typename TG, int DQK>
__global__ __launch_bounds__(NTHREADS, 1) void chunkwise_fused_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const TG* __restrict__ ig, const TG* __restrict__ fg, const float* __restrict__ c0,
    const float* __restrict__ n0, const float* __restrict__ m0, bf16_t* __restrict__ h,
    float* __restrict__ c_last, float* __restrict__ n_last, float* __restrict__ m_last, int NC, int DV, int BNH,
    int nvtile, float qk_scale, float eps) {
  using SM = Smem<DQK>;
  constexpr int DW = SM::DW;    // 64 or 32
  constexpr int KP = DW / 32;   // 32-deep k-steps of this wave's d-slice
  constexpr int NDT = DW / 16;  // C row tiles per wave
  constexpr int KU = DW / 32;   // K staging units per lane (4 rows x 8 d each)
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;

  // ---- XCD-aware workgroup -> (head, column tile): consecutive tiles of a head share an XCD
  const int nwg = BNH * nvtile;
  int lin = blockIdx.x;
  if ((nwg & 7) == 0) lin = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int bh = lin / nvtile;
  const int v0 = (lin - bh * nvtile) * DVT;
  const int S = NC * L;
  const int dw0 = w * DW;  // first C row of this wave

  char* kn = smem + SM::KN + w * SM::KN_SLOT;  // K natural tile, then this wave's S^T partials
  f32x4* sred = (f32x4*)(smem + SM::KN);       // [src][NST][64]
  __bf16* kt = (__bf16*)(smem + SM::KT + w * SM::KT_SLOT);
  __bf16* vt = (__bf16*)(smem + SM::VT);
  __bf16* vbh = (__bf16*)(smem + SM::VBH);
  __bf16* vbl = (__bf16*)(smem + SM::VBL);
  float* gw = (float*)(smem + SM::GATES) + w * 5 * 64;  // bl, ul, qbar, mc, alpha
  f32x4* hred = (f32x4*)(smem + SM::HRED);     // [src][slot][NVX][64]

  // ---- constant rows 64..79 of the V^T tiles: ones (row 64 of [V | 1]^T) and zeros
  for (int e = tid; e < 16 * PITCH; e += NTHREADS) {
    const int row = 64 + e / PITCH, col = e % PITCH;
    const __bf16 one = (__bf16)1.0f, zero = (__bf16)0.0f;
    vt[row * PITCH + col] = (row == 64) ? one : zero;
    vbh[row * PITCH + col] = zero;
    vbl[row * PITCH + col] = zero;
  }

  // ---- state in registers: C tiles and the n tile (n in column 0 of tile NVT)
  f32x4 Cacc[NDT][NVX];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = dw0 + phys(dt, g, e);
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq)
        Cacc[dt][vq][e] = c0 ? c0[((size_t)bh * DQK + d) * DV + v0 + 16 * vq + r16] : 0.f;
      Cacc[dt][NVT][e] = (n0 && r16 == 0) ? n0[(size_t)bh * DQK + d] : 0.f;
    }
  float m_prev = m0 ? m0[bh] : 0.f;

  // ---- loop-invariant global offsets (elements); per-chunk bases advance uniformly
  const int tq = lane & 15;                    // K staging: rows 4tq..4tq+3
  const int vtp = tid & 31, vg = tid >> 5;     // V staging: rows 2vtp, 2vtp+1, columns 8vg..8vg+7
  uint32_t offq[4][KP], offk[KU][4], offv[2];
#pragma unroll
  for (int it = 0; it < 4; ++it)
#pragma unroll
    for (int p = 0; p < KP; ++p) offq[it][p] = (uint32_t)((16 * it + r16) * DQK + dw0 + 32 * p + 8 * g);
#pragma unroll
  for (int u = 0; u < KU; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) offk[u][r] = (uint32_t)((4 * tq + r) * DQK + dw0 + 8 * (g + 4 * u));
#pragma unroll
  for (int r = 0; r < 2; ++r) offv[r] = (uint32_t)((2 * vtp + r) * DV + v0 + 8 * vg);
  const bf16_t* qh = q + (size_t)bh * S * DQK;
  const bf16_t* kh = k + (size_t)bh * S * DQK;
  const bf16_t* vh = v + (size_t)bh * S * DV;
  const TG* fh = fg + (size_t)bh * S;
  const TG* ih = ig + (size_t)bh * S;
  bf16_t* hh = h + (size_t)bh * S * DV;

  u32x4 Qc[4][KP], Kc[KU][4], Vc[2];
  float fc, ic;
  auto load_q = [&](int kc) {
    const bf16_t* base = qh + (size_t)kc * L * DQK;
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int p = 0; p < KP; ++p) Qc[it][p] = *reinterpret_cast<const u32x4*>(base + offq[it][p]);
  };
  auto load_kv = [&](int kc) {
    const bf16_t* kb = kh + (size_t)kc * L * DQK;
    const bf16_t* vb = vh + (size_t)kc * L * DV;
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) Kc[u][r] = *reinterpret_cast<const u32x4*>(kb + offk[u][r]);
#pragma unroll
    for (int r = 0; r < 2; ++r) Vc[r] = *reinterpret_cast<const u32x4*>(vb + offv[r]);
    fc = to_f32(fh[(size_t)kc * L + lane]);
    ic = to_f32(ih[(size_t)kc * L + lane]);
  };
  load_q(0);
  load_kv(0);

  for (int kc = 0; kc < NC; ++kc) {
    // ================= gates (every wave, lane = token of the chunk) -> this wave's gate rows
    const float b = wave_scan<false>(logsig_fast(fc));
    const float gsum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, b), 63));
    const float a = gsum - b + ic;
    const float m_next = fmaxf(gsum + m_prev, wave_max(a));
    const float alpha = exp2_((a - m_next) * LOG2E);      // exp(a_t - m')
    const float gbar = exp2_((gsum + m_prev - m_next) * LOG2E);
    const float u = ic - b;                              // i_j - b_j
    const float mb = b + m_prev;
    const float mc = fmaxf(mb, b + wave_scan<true>(u));  // combined stabiliser of row `lane`
    gw[lane] = (b - mc) * LOG2E;                         // bl: row term of the intra-chunk exponent
    gw[64 + lane] = u * LOG2E;                           // ul: column term
    gw[128 + lane] = exp2_((mb - mc) * LOG2E) * qk_scale;  // qbar
    gw[192 + lane] = mc;
    gw[256 + lane] = alpha;

    // ================= stage K (natural and transposed, raw) and V ([V | 1]^T and alpha-scaled hi/lo)
#pragma unroll
    for (int uu = 0; uu < KU; ++uu) {
      const int dgl = g + 4 * uu;  // 8-column group of this wave's d-slice
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<u32x4*>(kn + (lds_row(4 * tq + r) * PITCH + 8 * dgl) * 2) = Kc[uu][r];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint32_t sel = (s & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t p01 = __builtin_amdgcn_perm(Kc[uu][1][s >> 1], Kc[uu][0][s >> 1], sel);
        const uint32_t p23 = __builtin_amdgcn_perm(Kc[uu][3][s >> 1], Kc[uu][2][s >> 1], sel);
        const u32x2 pr = {p01, p23};
        *reinterpret_cast<u32x2*>(kt + lds_row(8 * dgl + s) * PITCH + 4 * tq) = pr;
      }
    }
    {
      const f32x2 al = *reinterpret_cast<const f32x2*>(gw + 256 + 2 * vtp);  // alpha of rows 2vtp, 2vtp+1
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint32_t sel = (s & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t pr = __builtin_amdgcn_perm(Vc[1][s >> 1], Vc[0][s >> 1], sel);
        const int off = (8 * vg + s) * PITCH + 2 * vtp;
        *reinterpret_cast<uint32_t*>(vt + off) = pr;
        const float x0 = al[0] * bf_lo(pr), x1 = al[1] * bf_hi(pr);
        const uint32_t hi = pack_bf16(x0, x1);
        *reinterpret_cast<uint32_t*>(vbh + off) = hi;
        *reinterpret_cast<uint32_t*>(vbl + off) = pack_bf16(x0 - bf_lo(hi), x1 - bf_hi(hi));
      }
      // rows 65..79 of the alpha-V tiles are zero (the previous chunk's H partials overwrote them)
      constexpr int ZCH = 15 * PITCH / 8;  // 16-byte pieces
      if (tid < ZCH) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(vbh + 65 * PITCH + 8 * tid) = z;
        *reinterpret_cast<u32x4*>(vbl + 65 * PITCH + 8 * tid) = z;
      }
      if (tid < 32) {  // row 64 of (alpha [V | 1])^T: alpha itself
        const uint32_t hi = pack_bf16(al[0], al[1]);
        *reinterpret_cast<uint32_t*>(vbh + 64 * PITCH + 2 * vtp) = hi;
        *reinterpret_cast<uint32_t*>(vbl + 64 * PITCH + 2 * vtp) = pack_bf16(al[0] - bf_lo(hi), al[1] - bf_hi(hi));
      }
    }

    __syncthreads();  // B1: V tiles visible to every wave, K tiles to their wave
    if (kc + 1 < NC) load_kv(kc + 1);  // staging registers are free: prefetch the next chunk's k, v, gates

    // ================= Q [C | n] (partial over this wave's d-slice)
    f32x4 Hacc[4][NVX];
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq) Hacc[it][vq] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int vq = 0; vq < NVX; ++vq) {
      bf16x8 Cb[KP];
#pragma unroll
      for (int p = 0; p < KP; ++p) Cb[p] = pack8(Cacc[2 * p][vq], Cacc[2 * p + 1][vq]);
#pragma unroll
      for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int p = 0; p < KP; ++p) Hacc[it][vq] = mfma(__builtin_bit_cast(bf16x8, Qc[it][p]), Cb[p], Hacc[it][vq]);
    }

    // ================= S^T = K Q^T (partial over the d-slice), causal tiles only
    f32x4 Sacc[4][4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      bf16x8 Ka[KP];
#pragma unroll
      for (int p = 0; p < KP; ++p)
        Ka[p] = *reinterpret_cast<const bf16x8*>(kn + ((16 * jt + r16) * PITCH + 32 * p + 8 * g) * 2);
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        if ((jt >> 1) > (it >> 1)) continue;
        Sacc[jt][it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < KP; ++p) Sacc[jt][it] = mfma(Ka[p], __builtin_bit_cast(bf16x8, Qc[it][p]), Sacc[jt][it]);
      }
    }
    if (kc + 1 < NC) load_q(kc + 1);  // q fragments are dead: prefetch the next chunk's

    // S^T partials -> this wave's slot (its K tile is dead)
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        if ((jt >> 1) > (it >> 1)) continue;
        sred[(w * NST + st_slot(it, jt)) * 64 + lane] = Sacc[jt][it];
      }

    // ================= state update [C | n]' = gbar [C | n] + K^T (alpha [V | 1]) (hi + lo)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      bf16x8 Ka[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) Ka[p] = *reinterpret_cast<const bf16x8*>(kt + (16 * dt + r16) * PITCH + 32 * p + 8 * g);
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq) {
        f32x4 c = Cacc[dt][vq] * gbar;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int off = (16 * vq + r16) * PITCH + 32 * p + 8 * g;
          c = mfma(Ka[p], *reinterpret_cast<const bf16x8*>(vbh + off), c);
          c = mfma(Ka[p], *reinterpret_cast<const bf16x8*>(vbl + off), c);
        }
        Cacc[dt][vq] = c;
      }
    }

    __syncthreads();  // B2: S^T partials visible

    // ================= own rows i = 16w + r16: exact scores, gating, M [V | 1] with M split hi + lo
    f32x4 Hmv[NVX];
#pragma unroll
    for (int vq = 0; vq < NVX; ++vq) Hmv[vq] = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      const int i = 16 * w + r16;
      const float bli = gw[i];
      const int npj = (w >> 1) + 1;  // tile pairs with j-range starting at or before the own rows
#pragma unroll
      for (int pj = 0; pj < 2; ++pj) {
        if (pj >= npj) break;
        f32x4 Ms[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int jt = 2 * pj + hf;
          const int slot = w < 2 ? 2 * w + jt : 4 + 4 * (w - 2) + jt;
          f32x4 sv = sred[slot * 64 + lane];
#pragma unroll
          for (int src = 1; src < NW; ++src) sv += sred[(src * NST + slot) * 64 + lane];
          const f32x4 ul = *reinterpret_cast<const f32x4*>(gw + 64 + 32 * pj + 8 * g + 4 * hf);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = 32 * pj + 8 * g + 4 * hf + e;
            sv[e] = (j <= i) ? sv[e] * qk_scale * exp2_(bli + ul[e]) : 0.f;
          }
          Ms[hf] = sv;
        }
        bf16x8 mh, ml;
        split8(Ms[0], Ms[1], mh, ml);
#pragma unroll
        for (int vq = 0; vq < NVX; ++vq) {
          const bf16x8 vb = *reinterpret_cast<const bf16x8*>(vt + (16 * vq + r16) * PITCH + 32 * pj + 8 * g);
          Hmv[vq] = mfma(mh, vb, Hmv[vq]);
          Hmv[vq] = mfma(ml, vb, Hmv[vq]);
        }
      }
    }

    // ================= sum Q [C | n] over the waves; wave w finishes rows 16w..16w+15
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      if (it == w) continue;
      const int slot = it < w ? it : it - 1;
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq) hred[((w * 3 + slot) * NVX + vq) * 64 + lane] = Hacc[it][vq];
    }
    __syncthreads();  // B3: Q [C | n] partials visible (the K / S regions are dead)
    {
      const f32x4 qb = *reinterpret_cast<const f32x4*>(gw + 128 + 16 * w + 4 * g);  // rows 16w + 4g + e
      const f32x4 mcr = *reinterpret_cast<const f32x4*>(gw + 192 + 16 * w + 4 * g);
      f32x4 H[NVX];
#pragma unroll
      for (int vq = 0; vq < NVX; ++vq) {
        f32x4 acc = (w == 0) ? Hacc[0][vq] : (w == 1) ? Hacc[1][vq] : (w == 2) ? Hacc[2][vq] : Hacc[3][vq];
#pragma unroll
        for (int src = 0; src < NW; ++src) {
          if (src == w) continue;
          const int slot = w < src ? w : w - 1;
          acc += hred[((src * 3 + slot) * NVX + vq) * 64 + lane];
        }
        H[vq] = qb * acc + Hmv[vq];
      }
      bf16_t* hb = hh + (size_t)kc * L * DV + v0 + 16 * 0 + r16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float den = __shfl(H[NVT][e], lane & 48, 64);  // column 64 lives in lane r16 == 0
        const float inv = 1.0f / (fmaxf(fabsf(den), exp2_(-mcr[e] * LOG2E)) + eps);
        const int i = 16 * w + 4 * g + e;
#pragma unroll
        for (int vq = 0; vq < NVT; ++vq) hb[(size_t)i * DV + 16 * vq] = from_f32<bf16_t>(H[vq][e] * inv);
      }
    }
    __syncthreads();  // B4: H partial slots (aliasing the K regions) consumed
    m_prev = m_next;
  }

  // ---- final states
  if (c_last) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = dw0 + phys(dt, g, e);
#pragma unroll
        for (int vq = 0; vq < NVT; ++vq)
          c_last[((size_t)bh * DQK + d) * DV + v0 + 16 * vq + r16] = Cacc[dt][vq][e];
        if (v0 == 0 && r16 == 0) n_last[(size_t)bh * DQK + d] = Cacc[dt][NVT][e];
      }
    if (v0 == 0 && tid == 0) m_last[bh] = m_prev;
  }
}

template <typename TG, int DQK>
static int launch(const ChunkwiseArgs& A) {
  const int BNH = A.B * A.NH;
  const int nvtile = A.DV / DVT;
  const int NC = A.S / L;
  auto kern = chunkwise_fused_kernel<TG, DQK>;
  const size_t smem = Smem<DQK>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess)
    return set_error(XL_ERR_LAUNCH, "xl_mlstm_chunkwise_fwd: LDS attribute failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(kern, dim3((unsigned)(BNH * nvtile)), dim3(NTHREADS), smem, (hipStream_t)A.stream,
                     (const bf16_t*)A.q, (const bf16_t*)A.k, (const bf16_t*)A.v, (const TG*)A.i, (const TG*)A.f,
                     A.c0, A.n0, A.m0, (bf16_t*)A.h, A.c_last, A.n_last, A.m_last, NC, A.DV, BNH, nvtile,
                     A.qk_scale, A.eps);
  return check_launch("xl_mlstm_chunkwise_fwd(fused)");
}

template <typename TG>
static int launch_d(const ChunkwiseArgs& A) {
  return A.DQK == 256 ? launch<TG, 256>(A) : launch<TG, 128>(A);
}

}  // namespace fused

bool chunkwise_fused_supported(const ChunkwiseArgs& a, const char** why) {
  const char* r = nullptr;
  if (a.dtype_qkv != XL_DTYPE_BF16) r = "q/k/v must be bfloat16";
  else if (a.L != fused::L) r = "chunk size must be 64";
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
