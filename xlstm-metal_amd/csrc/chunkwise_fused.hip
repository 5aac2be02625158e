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
// Work split (4 waves, 256 threads): wave w owns rows [w*DW, (w+1)*DW) of C
// (DW = DQK/4) and computes, for its slice of the DQK contraction, partial
// S^T = K Q^T, partial QC, the gated partial M and M V, and its slice of the
// state update.  The partial H's of the four waves are summed through LDS
// once per chunk (each wave owns 16 output rows).  All dense products are
// v_mfma_f32_16x16x32_bf16 with float32 accumulation:
//   S^T  (j x i, over d)   A = K rows  (LDS),      B = q rows (registers)
//   QC   (i x v, over d)   A = q rows  (registers), B = C (accumulators -> bf16)
//   MV   (i x v, over j)   A = M hi + lo (S^T accumulators -> bf16), B = V^T (LDS)
//   KV   (d x v, over t)   A = Kbar^T hi + lo (LDS), B = V^T (LDS)
// Operands coming from accumulators use a row permutation: the 16 rows of an
// MFMA tile are mapped to physical indices so that the 4 rows a lane holds in
// two adjacent tiles are 8 consecutive indices, i.e. exactly the 8-element
// k-slice that lane must supply when the accumulator is reused as an operand.
// Kbar = alpha_t k_t is split into bf16 hi + lo parts (two MFMAs) so the
// float32 state does not inherit bf16 rounding of the gated keys.  The gated
// scores are split the same way: each wave holds only a partial M (its slice
// of the q.k contraction), and partials can be much larger than their sum, so
// rounding them to bf16 alone would lose the sum.  C is rounded to bf16 only
// as the operand of the q C product.
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
constexpr int NVT = DVT / 16;  // 16-wide column tiles
constexpr int PITCH = 72;      // bf16 per LDS row (144 B): 16 consecutive rows hit distinct banks
constexpr float LOG2E = 1.4426950408889634f;

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
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * LOG2E); }

// LDS row of physical index x within a 64-row block: tiles of 16 rows, each
// tile pair (32 indices) interleaved so that lane group g of a tile pair
// covers indices 8g..8g+7 (4 in each tile).
__device__ __forceinline__ int lds_row(int x) {
  return 32 * (x >> 5) + 16 * ((x >> 2) & 1) + 4 * ((x >> 3) & 3) + (x & 3);
}
// physical index held by accumulator element e of lane group g in tile `tile`
__device__ __forceinline__ int phys(int tile, int g, int e) { return 32 * (tile >> 1) + 8 * g + 4 * (tile & 1) + e; }

template <int DQK>
struct Smem {
  static constexpr int DW = DQK / NW;              // C rows per wave
  static constexpr int KN_SLOT = NVT * (NW - 1) * 64 * 16;  // per-wave region: max(K natural, H partials)
  static_assert(64 * PITCH * 2 <= KN_SLOT, "K tile must fit the per-wave slot");
  static constexpr int R1 = 0;                                 // [NW][KN_SLOT]: K natural / H partials
  static constexpr int KTH = R1 + NW * KN_SLOT;               // [NW][DW][PITCH] bf16: (alpha k)^T hi
  static constexpr int KTL = KTH + NW * DW * PITCH * 2;        // lo
  static constexpr int VT = KTL + NW * DW * PITCH * 2;         // [64 v][PITCH] bf16: V^T
  static constexpr int QN = VT + DVT * PITCH * 2;              // [NW][64] float: partial q.n
  static constexpr int RS = QN + NW * 64 * 4;                  // [NW][64] float: partial row sums of M
  static constexpr int BYTES = RS + NW * 64 * 4;
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

  char* kn = smem + SM::R1 + w * SM::KN_SLOT;                      // this wave's K natural tile
  __bf16* kth = (__bf16*)(smem + SM::KTH) + w * DW * PITCH;
  __bf16* ktl = (__bf16*)(smem + SM::KTL) + w * DW * PITCH;
  __bf16* vt = (__bf16*)(smem + SM::VT);
  float* qn_red = (float*)(smem + SM::QN);
  float* rs_red = (float*)(smem + SM::RS);
  f32x4* h_red = (f32x4*)(smem + SM::R1);  // [src][slot][vt][lane]

  // ---- state in registers
  f32x4 Cacc[NDT][NVT];
  float nv[KP][8];  // n for d_local = 32p + 8g + s (same in all r16 lanes)
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int vq = 0; vq < NVT; ++vq)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = dw0 + phys(dt, g, e);
        Cacc[dt][vq][e] = c0 ? c0[((size_t)bh * DQK + d) * DV + v0 + 16 * vq + r16] : 0.f;
      }
#pragma unroll
  for (int p = 0; p < KP; ++p)
#pragma unroll
    for (int s = 0; s < 8; ++s) nv[p][s] = n0 ? n0[(size_t)bh * DQK + dw0 + 32 * p + 8 * g + s] : 0.f;
  float m_prev = m0 ? m0[bh] : 0.f;

  // ---- global prefetch registers (chunk kc and kc + 1)
  const bf16_t* qh = q + (size_t)bh * S * DQK;
  const bf16_t* kh = k + (size_t)bh * S * DQK;
  const bf16_t* vh = v + (size_t)bh * S * DV;
  const size_t gh = (size_t)bh * S;
  const int tq = lane & 15;        // K staging: rows 4tq..4tq+3
  const int vtp = tid & 31, vg = tid >> 5;  // V staging: rows 2vtp, 2vtp+1, columns 8vg..8vg+7

  u32x4 Qc[4][KP], Kc[KU][4], Vc[2];
  float fc, ic;
  auto load_chunk = [&](int kc, u32x4 (&Qr)[4][KP], u32x4 (&Kr)[KU][4], u32x4 (&Vr)[2], float& fr, float& ir) {
    const size_t row0 = (size_t)kc * L;
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int p = 0; p < KP; ++p)
        Qr[it][p] = *reinterpret_cast<const u32x4*>(qh + (row0 + 16 * it + r16) * DQK + dw0 + 32 * p + 8 * g);
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        Kr[u][r] = *reinterpret_cast<const u32x4*>(kh + (row0 + 4 * tq + r) * DQK + dw0 + 8 * (g + 4 * u));
#pragma unroll
    for (int r = 0; r < 2; ++r)
      Vr[r] = *reinterpret_cast<const u32x4*>(vh + (row0 + 2 * vtp + r) * DV + v0 + 8 * vg);
    fr = to_f32(fg[gh + row0 + lane]);
    ir = to_f32(ig[gh + row0 + lane]);
  };
  load_chunk(0, Qc, Kc, Vc, fc, ic);

  for (int kc = 0; kc < NC; ++kc) {
    // ================= gates (every wave, lane = token of the chunk)
    const float lsf = logsigmoid(fc);
    float b = lsf;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(b, o, 64);
      if (lane >= o) b += y;
    }
    const float gsum = __shfl(b, 63, 64);
    const float a = gsum - b + ic;
    const float m_next = fmaxf(gsum + m_prev, wave_max(a));
    const float alpha = fast_exp(a - m_next);           // Kbar scale of token `lane`
    const float gbar = fast_exp(gsum + m_prev - m_next);
    const float u = ic - b;                             // i_j - b_j
    float pm = u;                                       // prefix max of u
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(pm, o, 64);
      if (lane >= o) pm = fmaxf(pm, y);
    }
    const float mb = b + m_prev;
    const float mc = fmaxf(mb, b + pm);                 // combined stabiliser of row `lane`
    const float qbar = fast_exp(mb - mc) * qk_scale;
    const float bl = (b - mc) * LOG2E;                  // row term of the intra-chunk exponent
    const float ul = u * LOG2E;                         // column term

    // ================= stage K (natural, and alpha-scaled transposed hi/lo) and V^T into LDS
#pragma unroll
    for (int uu = 0; uu < KU; ++uu) {
      const int dgl = g + 4 * uu;  // 8-column group of this wave's d-slice
      float al[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * tq + r, 64);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<u32x4*>(kn + (lds_row(4 * tq + r) * PITCH + 8 * dgl) * 2) = Kc[uu][r];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t wd = Kc[uu][r][s >> 1];
          x[r] = al[r] * ((s & 1) ? bf_hi(wd) : bf_lo(wd));
        }
        const uint32_t h01 = pack_bf16(x[0], x[1]), h23 = pack_bf16(x[2], x[3]);
        const float l0 = x[0] - bf_lo(h01), l1 = x[1] - bf_hi(h01), l2 = x[2] - bf_lo(h23), l3 = x[3] - bf_hi(h23);
        const int row = lds_row(8 * dgl + s);
        u32x2 hv = {h01, h23}, lv = {pack_bf16(l0, l1), pack_bf16(l2, l3)};
        *reinterpret_cast<u32x2*>(kth + row * PITCH + 4 * tq) = hv;
        *reinterpret_cast<u32x2*>(ktl + row * PITCH + 4 * tq) = lv;
      }
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint32_t w0 = Vc[0][s >> 1], w1 = Vc[1][s >> 1];
      const uint32_t pr = (s & 1) ? ((w0 >> 16) | (w1 & 0xffff0000u)) : ((w0 & 0xffffu) | (w1 << 16));
      *reinterpret_cast<uint32_t*>(vt + (8 * vg + s) * PITCH + 2 * vtp) = pr;
    }

    // ================= q.n with the state entering the chunk, then n' (from the staging registers)
    float qn_part[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      float acc = 0.f;
#pragma unroll
      for (int p = 0; p < KP; ++p)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const uint32_t wd = Qc[it][p][s >> 1];
          acc += ((s & 1) ? bf_hi(wd) : bf_lo(wd)) * nv[p][s];
        }
      acc += __shfl_xor(acc, 16, 64);
      acc += __shfl_xor(acc, 32, 64);
      qn_part[it] = acc;
    }
#pragma unroll
    for (int uu = 0; uu < KU; ++uu) {
      float al[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * tq + r, 64);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        float x = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t wd = Kc[uu][r][s >> 1];
          x += al[r] * ((s & 1) ? bf_hi(wd) : bf_lo(wd));
        }
        // sum over the 16 lanes of a row (all 64 tokens), n' = gbar n + sum_t alpha_t k_t
        x += __shfl_xor(x, 1, 64);
        x += __shfl_xor(x, 2, 64);
        x += __shfl_xor(x, 4, 64);
        x += __shfl_xor(x, 8, 64);
        nv[uu][s] = gbar * nv[uu][s] + x;
      }
    }

    __syncthreads();  // B1: V^T visible to every wave, K tiles to their wave

    // ================= QC (partial over this wave's d-slice), rows scaled by qbar afterwards
    f32x4 Hacc[4][NVT];
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq) Hacc[it][vq] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int vq = 0; vq < NVT; ++vq) {
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
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) Sacc[jt][it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      bf16x8 Ka[KP];
#pragma unroll
      for (int p = 0; p < KP; ++p)
        Ka[p] = *reinterpret_cast<const bf16x8*>(kn + ((16 * jt + r16) * PITCH + 32 * p + 8 * g) * 2);
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        if ((jt >> 1) > (it >> 1)) continue;
#pragma unroll
        for (int p = 0; p < KP; ++p) Sacc[jt][it] = mfma(Ka[p], __builtin_bit_cast(bf16x8, Qc[it][p]), Sacc[jt][it]);
      }
    }

    // ================= prefetch the next chunk (the current q fragments are dead now)
    float fn = 0.f, in_ = 0.f;
    if (kc + 1 < NC) load_chunk(kc + 1, Qc, Kc, Vc, fn, in_);

#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float qb = __shfl(qbar, 16 * it + 4 * g + e, 64);
#pragma unroll
        for (int vq = 0; vq < NVT; ++vq) Hacc[it][vq][e] *= qb;
      }

    // ================= gate S^T into M (j <= i), row sums, M V with M split into bf16 hi + lo
    float rs_part[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int i = 16 * it + r16;
      const float bli = __shfl(bl, i, 64);
      float acc = 0.f;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        if ((jt >> 1) > (it >> 1)) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = phys(jt, g, e);
          const float ulj = __shfl(ul, j, 64);
          const float mval = (j <= i) ? Sacc[jt][it][e] * qk_scale * __builtin_amdgcn_exp2f(bli + ulj) : 0.f;
          Sacc[jt][it][e] = mval;
          acc += mval;
        }
      }
      acc += __shfl_xor(acc, 16, 64);
      acc += __shfl_xor(acc, 32, 64);
      rs_part[it] = acc;
#pragma unroll
      for (int pj = 0; pj < 2; ++pj) {
        if (pj > (it >> 1)) continue;
        const f32x4 x0 = Sacc[2 * pj][it], x1 = Sacc[2 * pj + 1][it];
        const bf16x8 mh = pack8(x0, x1);
        const u32x4 mw = __builtin_bit_cast(u32x4, mh);
        const f32x4 l0 = {x0[0] - bf_lo(mw[0]), x0[1] - bf_hi(mw[0]), x0[2] - bf_lo(mw[1]), x0[3] - bf_hi(mw[1])};
        const f32x4 l1 = {x1[0] - bf_lo(mw[2]), x1[1] - bf_hi(mw[2]), x1[2] - bf_lo(mw[3]), x1[3] - bf_hi(mw[3])};
        const bf16x8 ml = pack8(l0, l1);
#pragma unroll
        for (int vq = 0; vq < NVT; ++vq) {
          const bf16x8 vb = *reinterpret_cast<const bf16x8*>(vt + (16 * vq + r16) * PITCH + 32 * pj + 8 * g);
          Hacc[it][vq] = mfma(mh, vb, Hacc[it][vq]);
          Hacc[it][vq] = mfma(ml, vb, Hacc[it][vq]);
        }
      }
    }

    // ================= state update C' = gbar C + (Kbar hi + lo)^T V
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      bf16x8 Kh[2], Kl[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        Kh[p] = *reinterpret_cast<const bf16x8*>(kth + (16 * dt + r16) * PITCH + 32 * p + 8 * g);
        Kl[p] = *reinterpret_cast<const bf16x8*>(ktl + (16 * dt + r16) * PITCH + 32 * p + 8 * g);
      }
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq) {
        f32x4 c = Cacc[dt][vq] * gbar;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const bf16x8 vb = *reinterpret_cast<const bf16x8*>(vt + (16 * vq + r16) * PITCH + 32 * p + 8 * g);
          c = mfma(Kh[p], vb, c);
          c = mfma(Kl[p], vb, c);
        }
        Cacc[dt][vq] = c;
      }
    }

    // ================= reduce H over the waves; wave w finishes rows 16w..16w+15
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      if (it == w) continue;
      const int slot = it < w ? it : it - 1;
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq) h_red[((w * (NW - 1) + slot) * NVT + vq) * 64 + lane] = Hacc[it][vq];
    }
    if (g == 0) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        qn_red[w * 64 + 16 * it + r16] = qn_part[it];
        rs_red[w * 64 + 16 * it + r16] = rs_part[it];
      }
    }
    __syncthreads();  // B2: partials visible
    f32x4 Hown[NVT];
#pragma unroll
    for (int vq = 0; vq < NVT; ++vq) {
      // runtime-indexed own tile (it == w): select without dynamic register indexing
      f32x4 acc = (w == 0) ? Hacc[0][vq] : (w == 1) ? Hacc[1][vq] : (w == 2) ? Hacc[2][vq] : Hacc[3][vq];
#pragma unroll
      for (int src = 0; src < NW; ++src) {
        if (src == w) continue;
        const int slot = w < src ? w : w - 1;
        acc += h_red[((src * (NW - 1) + slot) * NVT + vq) * 64 + lane];
      }
      Hown[vq] = acc;
    }
    const size_t tok0 = gh + (size_t)kc * L;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * w + 4 * g + e;
      float qn = 0.f, rs = 0.f;
#pragma unroll
      for (int src = 0; src < NW; ++src) {
        qn += qn_red[src * 64 + i];
        rs += rs_red[src * 64 + i];
      }
      const float mci = __shfl(mc, i, 64);
      const float den = __shfl(qbar, i, 64) * qn + rs;
      const float inv = 1.0f / (fmaxf(fabsf(den), fast_exp(-mci)) + eps);
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq)
        h[(tok0 + i) * DV + v0 + 16 * vq + r16] = from_f32<bf16_t>(Hown[vq][e] * inv);
    }
    __syncthreads();  // B3: H partial slots may be overwritten by the next chunk's K tiles

    m_prev = m_next;
    fc = fn;
    ic = in_;
  }

  // ---- final states
  if (c_last) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int vq = 0; vq < NVT; ++vq)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = dw0 + phys(dt, g, e);
          c_last[((size_t)bh * DQK + d) * DV + v0 + 16 * vq + r16] = Cacc[dt][vq][e];
        }
    if (v0 == 0) {
      if (r16 == 0) {
#pragma unroll
        for (int p = 0; p < KP; ++p)
#pragma unroll
          for (int s = 0; s < 8; ++s) n_last[(size_t)bh * DQK + dw0 + 32 * p + 8 * g + s] = nv[p][s];
      }
      if (tid == 0) m_last[bh] = m_prev;
    }
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
