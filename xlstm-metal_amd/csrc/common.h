// Shared device helpers and host-side error plumbing for libxlstm_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xlstm_hip.h"

namespace xl {

// ---------------------------------------------------------------- host errors
// Records the message for xl_last_error() (thread local) and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Maps a HIP launch status to XL_OK / XL_ERR_LAUNCH (recording the message).
int check_launch(const char* what);

inline bool dtype_ok(int dt) { return dt == XL_DTYPE_F32 || dt == XL_DTYPE_BF16 || dt == XL_DTYPE_F16; }
inline int dtype_size(int dt) { return dt == XL_DTYPE_F32 ? 4 : 2; }

// ------------------------------------------------------------- element types
// Storage types: float, bf16 (raw uint16 bits) and f16 (_Float16).
struct bf16_t { uint16_t bits; };
typedef _Float16 f16_t;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(((uint32_t)x.bits) << 16); }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }

// float -> bf16 bits, round to nearest even (quiet NaN preserved).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { bf16_t r; r.bits = f32_to_bf16_bits(x); return r; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return (f16_t)x; }

// Rounds a float to the precision of T (identity for float).
template <typename T> __device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// Rounds a pair of floats to T in place with one packed hardware conversion
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: round to nearest even, NaN kept).
typedef __bf16 xl_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 xl_f16x2 __attribute__((ext_vector_type(2)));
typedef float xl_f32x2 __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ void round2_to(float& a, float& b);
template <> __device__ __forceinline__ void round2_to<float>(float&, float&) {}
template <> __device__ __forceinline__ void round2_to<bf16_t>(float& a, float& b) {
  const xl_f32x2 v = {a, b};
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, xl_bf16x2));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}
template <> __device__ __forceinline__ void round2_to<f16_t>(float& a, float& b) {
  const xl_f32x2 v = {a, b};
  const xl_f16x2 h = __builtin_convertvector(v, xl_f16x2);
  a = (float)h[0];
  b = (float)h[1];
}

template <typename T> struct is_f32 { static constexpr bool value = false; };
template <> struct is_f32<float> { static constexpr bool value = true; };

// ----------------------------------------------------------------- gate math
// log(sigmoid(x)) = min(x, 0) - log1p(exp(-|x|)), accurate for all x.
__device__ __forceinline__ float logsigmoid(float x) {
  return fminf(x, 0.0f) - log1pf(expf(-fabsf(x)));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// tanh from its Taylor series near 0 and (1 - e)/(1 + e), e = exp(-2|x|),
// elsewhere.  |x| < 0.3: terms through x^11 (next term < 3e-10 relative);
// otherwise 1 - e >= 0.45 so the quotient has no cancellation.
__device__ __forceinline__ float tanh_f32(float x) {
  float ax = fabsf(x);
  if (ax < 0.3f) {
    float x2 = x * x;
    // x - x^3/3 + 2x^5/15 - 17x^7/315 + 62x^9/2835 - 1382x^11/155925
    float p = -1382.0f / 155925.0f;
    p = fmaf(p, x2, 62.0f / 2835.0f);
    p = fmaf(p, x2, -17.0f / 315.0f);
    p = fmaf(p, x2, 2.0f / 15.0f);
    p = fmaf(p, x2, -1.0f / 3.0f);
    return fmaf(x * x2, p, x);
  }
  float e = __expf(-2.0f * ax);
  float t = (1.0f - e) / (1.0f + e);
  return copysignf(t, x);
}

// cap * tanh(x / cap) for a 16-bit output: tanh(z) = 1 - 2 / (1 + e^{2z}) from
// the hardware exp2 and reciprocal (absolute error < 5e-7, far under half an
// ulp), and z itself below |z| = 2^-6, where the subtraction cancels (relative
// error z^2 / 3 < 1e-4).
__device__ __forceinline__ float soft_cap16(float x, float cap, float inv_cap) {
  const float z = x * inv_cap;
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * 2.8853900817779268f));
  return cap * (fabsf(z) < 0.015625f ? z : t);
}

// ------------------------------------------------------- wavefront reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the 64 lanes with DPP row shifts and row broadcasts (no LDS
// round trips); the total lands in lane 63.
__device__ __forceinline__ float wave_sum_dpp(float x) {
#define XL_DPP_ADD(CTRL, ROWMASK) \
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWMASK, 0xf, false));
  XL_DPP_ADD(0x111, 0xf)  // row_shr:1
  XL_DPP_ADD(0x112, 0xf)  // row_shr:2
  XL_DPP_ADD(0x114, 0xf)  // row_shr:4
  XL_DPP_ADD(0x118, 0xf)  // row_shr:8
  XL_DPP_ADD(0x142, 0xa)  // row_bcast:15 into rows 1, 3
  XL_DPP_ADD(0x143, 0xc)  // row_bcast:31 into rows 2, 3
#undef XL_DPP_ADD
  return x;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ------------------------------------------------- stabiliser scans over time
// The stabiliser recurrence m_t = max(m_{t-1} + a_t, b_t) (a = logsig f, b = i)
// is the composition of the max-plus maps m -> max(m + a, b):
// (a, b) o (a', b') = (a + a', max(b + a', b')).  A span's map carries sums
// of a over sub-spans only, so m has the rounding of the step-by-step
// recurrence (exact wherever b_t resets it).
// inclusive scan over the lanes (lane order = time) of the maps m -> max(m + a, b)
__device__ __forceinline__ void maxplus_scan(float& a, float& b) {
  const int ida = __float_as_int(0.f), idb = __float_as_int(-INFINITY);
#define XL_MP_STEP(CTRL, ROWMASK)                                                                                 \
  {                                                                                                               \
    const float ae = __int_as_float(__builtin_amdgcn_update_dpp(ida, __float_as_int(a), CTRL, ROWMASK, 0xf, false)); \
    const float be = __int_as_float(__builtin_amdgcn_update_dpp(idb, __float_as_int(b), CTRL, ROWMASK, 0xf, false)); \
    b = fmaxf(be + a, b);                                                                                         \
    a = ae + a;                                                                                                   \
  }
  XL_MP_STEP(0x111, 0xf)  // row_shr:1
  XL_MP_STEP(0x112, 0xf)  // row_shr:2
  XL_MP_STEP(0x114, 0xf)  // row_shr:4
  XL_MP_STEP(0x118, 0xf)  // row_shr:8
  XL_MP_STEP(0x142, 0xa)  // row_bcast:15 into rows 1, 3
  XL_MP_STEP(0x143, 0xc)  // row_bcast:31 into rows 2, 3
#undef XL_MP_STEP
}

__device__ __forceinline__ float lane_of(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

}  // namespace xl
