// Device helpers shared by the fused chunkwise kernels (chunkwise_fused.hip and
// chunkwise_pipe.hip): MFMA wrappers, bf16 hi + lo splits, chunk-relative buffer
// access, transposed LDS reads, DPP scans, and the layout constants both kernels use.
#pragma once

#include "chunkwise.h"

namespace xl {
namespace fused {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int L = 64;           // chunk size (= wavefront size: one lane per token)
constexpr int NSW = 4;          // state waves
constexpr int NOW = 4;          // output waves
constexpr int NTHREADS = 64 * (NSW + NOW);
constexpr int DVT = 64;         // DV columns per workgroup
constexpr int NVT = DVT / 16;   // 16-wide column tiles of v
constexpr int NVX = NVT + 1;    // ... plus the ones tile (row sums of M)
constexpr int VN_PITCH = 160;   // bytes per row of natural V (8 consecutive rows -> distinct 32 B bank groups)
constexpr int AV_PITCH = 304;   // bytes per row of natural alpha' V: hi (64 bf16) | lo (64 bf16) | pad
// Partial Q C tiles: 72 floats per token row (2 mod 16 slots of 16 bytes) with the row's
// 4-column groups G stored in the order (G >> 1) + 8 (G & 1).  The output waves read groups
// 2g + b of rows r16, which then fall on slots 2 r16 + g + const: a b128 read without bank
// conflicts (the natural order at any padded pitch is served at half that rate).
constexpr int HP_PITCH = 72;    // floats per token row of the partial Q C tiles
__device__ __forceinline__ constexpr int hp_col(int G) { return 4 * ((G >> 1) + 8 * (G & 1)); }
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float RENORM = -30.f; // renormalise the stored state when the deferred log rescale drops below this
constexpr int PREP_STRIDE = 320;  // floats per chunk of gate prep: b, a, cummax(i - b), (i - b) log2e, [g, max a]
constexpr int kMaxSegmentsDev = 16;  // most sequence segments of one call (few heads)
constexpr int GROWS = 8;          // shared gate rows per chunk: bl, ul, qbar, mc, alpha', [renorm scale, m', G], alpha' bf16 hi | lo, bf16 zeros

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// 32 x 32 x 16: lane l holds A row l % 32 / B column l % 32 at k = 8 (l / 32) .. +7;
// D column l % 32, rows 8i + 4 (l / 32) + j in element 4i + j
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// The low part of a pair packed as hi = {bf16(x0), bf16(x1)}: bf16(x_e - hi_e), the
// subtraction exact (x - bf16(x) is representable).  hi_e is unpacked with a shift
// (element 0) or a mask (element 1); on gfx950 this runs faster than a v_dot2c_f32_bf16
// against {-1, 0}, which also needs a copy of x for its accumulator.
__device__ __forceinline__ uint32_t pack_lo(uint32_t hi, float x0, float x1) {
  return pack_bf16(x0 - bf_lo(hi), x1 - bf_hi(hi));
}
// bf16 hi + lo split of 8 floats: hi = bf16(x), lo = bf16(x - hi)
__device__ __forceinline__ void split8(f32x4 a, f32x4 b, bf16x8& hi, bf16x8& lo) {
  const u32x4 h = {pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3])};
  const u32x4 l = {pack_lo(h[0], a[0], a[1]), pack_lo(h[1], a[2], a[3]), pack_lo(h[2], b[0], b[1]),
                   pack_lo(h[3], b[2], b[3])};
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}
__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }
// Chunk-relative global access: a raw buffer resource per 64-token chunk
// (wave-uniform base, num_records = the chunk's valid rows) and a per-thread
// byte offset that stays the same for every chunk.  Rows past S (a ragged last
// chunk) read as 0 and their stores are dropped by the buffer range check, so
// no address needs clamping.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const bf16_t* base, int rows, int row_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, rows * row_bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Same with a wave-uniform byte offset (the instruction's scalar offset): loads of
// one thread that differ by a constant keep a single offset register.
__device__ __forceinline__ u32x4 ld16s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ void st16(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 x) {
  typedef unsigned int b128 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(b128, x), r, off, 0, 0);
}
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

// Column of the 64-wide DV tile held by column n of 16-wide tile vq of the
// output waves: runs of 4 consecutive columns, and the tile pair (2h, 2h+1)
// covers columns 32h .. 32h+31 so that a lane of the transposed output holds 8
// consecutive columns (one 16-byte store).
__device__ __forceinline__ int vcol_of(int vq, int n) { return 32 * (vq >> 1) + 8 * (n >> 2) + 4 * (vq & 1) + (n & 3); }

// Sequence segments (for few heads: B * NH * DV / 64 workgroups leave CUs idle).
// The grid covers nseg segments of kc_per_seg chunks per (head, column tile).
// Segment 0 starts from (c0, n0, m0) (zeros and m = 0 when absent, the
// reference's zero state); segment s >= 1 starts from the s-1'th entry of
// (sc, sn, sm) or, when sc is null, from the empty state (C = n = 0, m = -inf,
// so its end state is the segment's own contribution).  With ec set, every
// segment writes its end state to entry s of (ec, en, em); otherwise the last
// segment writes (c_last, n_last, m_last).  STATES_ONLY launches skip q C and
// the outputs (h is not written).
struct SegArgs {
  int nseg, kc_per_seg;
  const float *sc, *sn, *sm;
  float *ec, *en, *em;
};

// LDS layout of one workgroup of the fused kernels (DQK 128 or 256, 64 DV columns).
template <int DQK>
struct Smem {
  static constexpr int KPD = DQK / 32;                   // 32-deep k-steps over DQK
  static constexpr int KN_PITCH = DQK * 2 + 32;          // bytes per K row (= 32 mod 64, see the header)
  static constexpr int KN = 0;                           // [64 t][KN_PITCH]: K natural
  static constexpr int VN = KN + 64 * KN_PITCH;          // [64 t][VN_PITCH]: V natural
  static constexpr int AV = VN + 64 * VN_PITCH;          // [64 t][AV_PITCH]: alpha' V hi (64 bf16) | lo (64 bf16)
  static constexpr int HP = AV + 64 * AV_PITCH;          // [4 state waves][64 t][HP_PITCH] float: partial Q C
  static constexpr int NB = HP + NSW * 64 * HP_PITCH * 4;  // [2 chunks][4 parts][NB_PITCH] bf16: n (hi, lo of both halves)
  static constexpr int NB_PITCH = DQK + 16;              // bf16 per n part row (= 32 mod 64 bytes)
  static constexpr int GATES = NB + 2 * 4 * NB_PITCH * 2;     // [2 chunks][GROWS][64] float: gate rows + scalars
  static constexpr int BYTES = GATES + 2 * GROWS * 64 * 4;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// Everything the main chunkwise kernels take (one (head, column tile, segment) per workgroup).
struct MainArgs {
  const bf16_t *q, *k, *v;
  const float *c0, *n0, *m0;
  bf16_t* h;
  float *c_last, *n_last, *m_last;
  const float* prep;
  int S, NC, DV, BNH, nvtile;
  float qk_scale, eps;
  SegArgs sg;
  int dq;  // q / k width in memory (DQK of the launch, or less: a multiple of DQK / 4)
};

// The pipelined main kernel (chunkwise_pipe.hip): nwg workgroups of NTHREADS on stream st.
// XL_OK or a negative XL_ERR_* code.
int pipe_launch(bool f16, int DQK, bool states_only, unsigned nwg, hipStream_t st, const MainArgs& a);

}  // namespace fused
}  // namespace xl
