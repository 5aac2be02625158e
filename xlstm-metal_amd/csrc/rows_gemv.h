// Row-streaming GEMV on the matrix cores, shared by the lm_head and the gate
// projection: dot products of every row of a long streamed matrix S [R, D] with
// each of a few small rows X [M, D], bound by reading S once.
//
// Each wave streams whole S rows, every load one contiguous 1 KB piece of a row
// (lane l holds elements 8l .. 8l + 7 of it), and keeps each small row's
// matching slices in registers.  The loads are the A operand of
// v_mfma_f32_16x16x32 as they stand: row i of the 16 x 32 operand is lanes i,
// 16 + i, 32 + i, 48 + i's slices, and the small row's slices in the same lane
// layout are B, so D[i][j] pairs the S slices of lanes {16g + i} with the X
// slices of lanes {16g + j}: the diagonal D[i][i] is the dot product over lane
// i's quarter of the piece, and the trace (a select and 6 DPP adds over the 16
// lanes that hold it) is the row's dot product.  One MFMA per small row and
// piece uses a sixteenth of its products: the pass is bound by the stream, not
// the matrix cores.  Reading S as 1 KB runs of one row streams it at 6.1-6.7
// TB/s on MI355X where 16 rows x 64 bytes per load (the operand layout of a
// tiled GEMM) reaches 4.0-5.2 TB/s.
//
// Waves stride over the rows (wave gw of nw takes rows gw, gw + nw, ...), two
// rows' pieces in flight: the next row requested before this one's MFMAs.  MT:
// the small rows rounded up to a power of two (rows past M are zero); NPC: 1 KB
// pieces per row (D = 512 NPC).
#pragma once

#include "common.h"

#include <mutex>
#include <type_traits>
#include <vector>

namespace xl {
namespace rowgemv {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int WAVES = 4;          // waves per workgroup
constexpr int MAX_XREGS = 128;    // registers of small-row slices per lane (MT * NPC * 4)

template <typename T>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same<T, bf16_t>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

// The whole wave calls epi(r, lane, dot) after each streamed row r; lane m < MT
// holds dot(S[r], X[m]) (0 for m >= M).
template <typename T, int MT, int NPC, typename Epi>
__device__ __forceinline__ void stream_rows(const T* __restrict__ x, int M, const T* __restrict__ s, int R, int D,
                                            Epi&& epi) {
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * WAVES;
  const int gw = blockIdx.x * WAVES + (threadIdx.x >> 6);
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 xr[MT][NPC];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int p = 0; p < NPC; ++p)
      xr[m][p] = m < M ? *reinterpret_cast<const u32x4*>(x + (size_t)m * D + 512 * p + 8 * lane) : zero;
  // lane (g, r16) holds D[4g + e][r16], e = 0..3: the diagonal element D[i][i] sits in lane
  // 16 (i >> 2) + i at e = i & 3
  const bool on_diag = (lane >> 4) == ((lane & 15) >> 2);
  const int de = lane & 3;
  u32x4 sa[2][NPC];
  auto load = [&](int r, auto buf_tag) {
    constexpr int b = decltype(buf_tag)::value;
    const T* sr = s + (size_t)r * D + 8 * lane;
#pragma unroll
    for (int p = 0; p < NPC; ++p) sa[b][p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(sr + 512 * p));
  };
  auto run = [&](int r, auto buf_tag) {
    constexpr int b = decltype(buf_tag)::value;
    f32x4 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NPC; ++p)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[m] = mfma16<T>(sa[b][p], xr[m][p], acc[m]);
    float dot = 0.f;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float d = de == 0 ? acc[m][0] : de == 1 ? acc[m][1] : de == 2 ? acc[m][2] : acc[m][3];
      const float tr = wave_sum_dpp(on_diag ? d : 0.f);  // the trace, in lane 63
      const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tr), 63));
      dot = lane == m ? t : dot;
    }
    epi(r, lane, dot);
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // two rows per trip keep the buffer indices compile-time constants
  int r = gw;
  if (r < R) load(r, B0{});
  for (; r < R; r += 2 * nw) {
    if (r + nw < R) load(r + nw, B1{});
    run(r, B0{});
    if (r + 2 * nw < R) load(r + 2 * nw, B0{});
    if (r + nw < R) run(r + nw, B1{});
  }
}

// MT for M small rows, 0 when the row form does not take the shape (D = 512 NPC with NPC in
// {1, 2, 4, 8}, M <= 16, the slices within MAX_XREGS registers).
inline int small_rows(int M, int D) {
  if (M < 1 || M > 16 || D % 512 != 0) return 0;
  const int npc = D / 512;
  if (npc != 1 && npc != 2 && npc != 4 && npc != 8) return 0;
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
  return mt * npc * 4 <= MAX_XREGS ? mt : 0;
}

// Resident workgroups of kern on the current device (CUs x workgroups per CU), queried once per
// (device, kernel) and kept: the launch path then makes no runtime query.
inline hipError_t resident_blocks(const void* kern, int* out) {
  struct Entry {
    int dev;
    const void* kern;
    int blocks;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& c : cache)
      if (c.dev == dev && c.kern == kern) {
        *out = c.blocks;
        return hipSuccess;
      }
  }
  int cus = 0, per_cu = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * WAVES, 0);
  if (e != hipSuccess) return e;
  const int blocks = cus * (per_cu > 0 ? per_cu : 1);
  std::lock_guard<std::mutex> lock(mu);
  cache.push_back(Entry{dev, kern, blocks});
  *out = blocks;
  return hipSuccess;
}

// One full set of resident workgroups of kern (each wave strides over the rows), at most one
// wave per row; launches with args.
inline int launch_streaming(const void* kern, void** args, int R, hipStream_t st, const char* who) {
  int resident = 0;
  hipError_t e = resident_blocks(kern, &resident);
  if (e != hipSuccess) return set_error(XL_ERR_LAUNCH, "%s: occupancy query failed: %s", who, hipGetErrorString(e));
  const int64_t need = ((int64_t)R + WAVES - 1) / WAVES;
  int64_t blocks = resident;
  if (blocks > need) blocks = need;
  if (blocks < 1) blocks = 1;
  e = hipLaunchKernel(kern, dim3((unsigned)blocks), dim3(64 * WAVES), args, 0, st);
  if (e != hipSuccess) return set_error(XL_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return check_launch(who);
}

}  // namespace rowgemv
}  // namespace xl

// The instance of KERN<T, MT, NPC> for mt = rowgemv::small_rows(M, D) and npc = D / 512 (a
// statement: returns the kernel pointer from the enclosing function).
#define XL_ROWGEMV_PICK(KERN, T, mt, npc)                                                              \
  do {                                                                                                 \
    if ((mt) == 1 && (npc) == 1) return (const void*)KERN<T, 1, 1>;                                    \
    if ((mt) == 1 && (npc) == 2) return (const void*)KERN<T, 1, 2>;                                    \
    if ((mt) == 1 && (npc) == 4) return (const void*)KERN<T, 1, 4>;                                    \
    if ((mt) == 1 && (npc) == 8) return (const void*)KERN<T, 1, 8>;                                    \
    if ((mt) == 2 && (npc) == 1) return (const void*)KERN<T, 2, 1>;                                    \
    if ((mt) == 2 && (npc) == 2) return (const void*)KERN<T, 2, 2>;                                    \
    if ((mt) == 2 && (npc) == 4) return (const void*)KERN<T, 2, 4>;                                    \
    if ((mt) == 2 && (npc) == 8) return (const void*)KERN<T, 2, 8>;                                    \
    if ((mt) == 4 && (npc) == 1) return (const void*)KERN<T, 4, 1>;                                    \
    if ((mt) == 4 && (npc) == 2) return (const void*)KERN<T, 4, 2>;                                    \
    if ((mt) == 4 && (npc) == 4) return (const void*)KERN<T, 4, 4>;                                    \
    if ((mt) == 4 && (npc) == 8) return (const void*)KERN<T, 4, 8>;                                    \
    if ((mt) == 8 && (npc) == 1) return (const void*)KERN<T, 8, 1>;                                    \
    if ((mt) == 8 && (npc) == 2) return (const void*)KERN<T, 8, 2>;                                    \
    if ((mt) == 8 && (npc) == 4) return (const void*)KERN<T, 8, 4>;                                    \
    if ((mt) == 16 && (npc) == 1) return (const void*)KERN<T, 16, 1>;                                  \
    if ((mt) == 16 && (npc) == 2) return (const void*)KERN<T, 16, 2>;                                  \
    return nullptr;                                                                                    \
  } while (0)
