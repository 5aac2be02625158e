// bf16 matrix-core building blocks shared by the chunkwise kernels (gfx950).
#pragma once
#include "common.h"

#include <type_traits>

namespace xl {
namespace mfma {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// v_mfma_f32_16x16x32_bf16: A[i][k] in lane i + 16 (k / 8), element k % 8; B[k][j] in lane
// j + 16 (k / 8); D as for 16x16x4f32 (D[i][j] in lane j + 16 (i / 4), element i % 4).
// Operands exact in bf16 (q, k, v, dH) enter once; a float32 operand x enters as the pair
// hi = bf16(x), lo = bf16(x - hi) (two products, 16 significant bits of x), accumulated in
// float32.
typedef __bf16 bfx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bfx2 __attribute__((ext_vector_type(2)));
typedef short sx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) sx4 lds_sx4;

__device__ __forceinline__ f32x4 mfma_bf(bfx8 a, bfx8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// {bf16(x0), bf16(x1)} (round to nearest even), x0 in the low half
__device__ __forceinline__ uint32_t pk_bf(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x0, x1}), bfx2));
}
__device__ __forceinline__ float bf_l(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_h(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// hi / lo pair of 8 floats (x - hi is exact in float32)
__device__ __forceinline__ void split_bf(const float (&x)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = pk_bf(x[2 * e], x[2 * e + 1]);
    lo[e] = pk_bf(x[2 * e] - bf_l(hi[e]), x[2 * e + 1] - bf_h(hi[e]));
  }
}
// Two ds_read_b64_tr_b16 -> one 8 x bf16 operand.  Within each 16 lanes, lane s passes the
// address of 4 consecutive 16-bit columns at 4 (s % 4) of row s / 4 (of a 4-row block) and
// receives column s of the 4 rows: with p0 / p1 the addresses in two 4-row blocks, lane s ends
// with column c0 + s of rows R0 .. R0 + 3 (elements 0..3) and R1 .. R1 + 3 (elements 4..7).
__device__ __forceinline__ bfx8 tr_pair(const void* p0, const void* p1) {
  const sx4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sx4*)p0);
  const sx4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sx4*)p1);
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return __builtin_bit_cast(bfx8, (u32x4{ua[0], ua[1], ub[0], ub[1]}));
}
__device__ __forceinline__ bfx8 ld_bf8(const void* p) { return __builtin_bit_cast(bfx8, *(const u32x4*)p); }
// Workgroup b of a grid of G runs on XCD b % 8 (round-robin dispatch over the 8 XCDs, each with
// its own L2).  The logical index returned gives every XCD one contiguous range, so logical
// neighbours (the column tiles of one head and chunk, which read the same q / k / v / dH rows)
// share an L2.  A bijection on [0, G).
__device__ __forceinline__ int xcd_contiguous(int b, int G) {
  const int x = b & 7, i = b >> 3, per = G >> 3, rem = G & 7;
  return x * per + (x < rem ? x : rem) + i;
}

// f(integral_constant<int, I>) for I = I0 .. N - 1, unrolled at compile time
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

}  // namespace mfma
}  // namespace xl
