// Logit projection with the soft-cap epilogue: y[m, v] = cap * tanh(z / cap),
// z = sum_d x[m, d] W[v, d] rounded to the dtype, for the few token rows a
// decoder needs logits of (M <= 16: a decode step's tokens, a prompt's last
// positions) against a vocabulary-sized W [V, D].
//
// The launch is bound by streaming W (V * D * 2 bytes, 412 MB for the 7B
// model) from HBM once; the arithmetic runs on v_mfma_f32_16x16x32 (bf16 /
// f16).  The epilogue rounds the logits to the dtype (the Linear's output),
// applies the soft-cap in float32 and rounds once more, as
// soft_cap(lm_head(x), cap) does.  Three forms (measured on MI355X with the
// weights cold in the caches):
//
// * D a multiple of 512 and the token rows' slices within 128 registers
//   (lm_head_rows_kernel): the row-streaming loop of rows_gemv.h with W as the
//   streamed matrix and the token rows as the small ones (each W row as 1 KB
//   contiguous loads, the logit as the trace of an MFMA diagonal); 64 us for
//   412 MB at the 7B shape against 83 for the split form below.
// * Otherwise the tile forms: 16 vocabulary rows as the A operand straight from
//   nontemporal 16-byte loads (lane (g, r16) holds row r16's k-slice 8g .. 8g + 7
//   of each 32-wide k-step), the token rows as B; lane (g, r16) ends with the
//   logits of token r16 at vocabulary rows 4g .. 4g + 3 of the tile.
// * M <= 4 (lm_head_split_kernel): a workgroup of 4 waves per vocabulary tile,
//   each wave over a quarter of D with the token rows loaded alongside W (a few
//   distinct cache lines per load, served by L1), partial tiles summed through
//   LDS.  3144 short workgroups at the 7B shape keep every CU busy to the end:
//   79 us for 412 MB at M = 1 (5.2 TB/s, 84 % of a plain read's 6.2 TB/s).
// * M > 4 (lm_head_staged_kernel): the token rows staged once per workgroup in
//   LDS (16 bytes of padding per row keep the 16 rows of a k-slice in distinct
//   banks) and each of 8 waves over a whole tile and all of D, two register
//   blocks of 8 k-steps in flight; loading up to 16 distinct token rows
//   alongside W slows the split form by a third at M = 16.
#include "common.h"
#include "rows_gemv.h"

#include <type_traits>

namespace xl {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename T>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same<T, bf16_t>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

constexpr int LS_WAVES = 4;  // split form: waves per vocabulary tile, each over a quarter of D
constexpr int LS_KB = 8;     // split form: k-steps per load block
constexpr int LS_MAX_ROWS = 4;
constexpr int LH_WAVES = 8;  // staged form: vocabulary tiles per workgroup
constexpr int LH_BLOCK = 64 * LH_WAVES;
constexpr int LH_KB = 8;  // k-steps per register block
constexpr int LH_MAX_ROWS = 16;
constexpr size_t LH_MAX_LDS = 160 * 1024;

// LDS bytes of the staged token rows: M rows of D + 8 elements
inline size_t lds_bytes(int M, int D) { return (size_t)M * (D + 8) * 2; }

// Row form: the logits of W's rows against the token rows, soft-capped.
template <typename T, int MT, int NPC>
__global__ __launch_bounds__(64 * rowgemv::WAVES) void lm_head_rows_kernel(const T* __restrict__ x,
                                                                           const T* __restrict__ w,
                                                                           T* __restrict__ y, int M, int D, int V,
                                                                           float cap, float inv_cap) {
  rowgemv::stream_rows<T, MT, NPC>(x, M, w, V, D, [&](int r, int lane, float logit) {
    if (lane < M) {
      float z = round_to<T>(logit);  // the Linear's output in its dtype
      if (cap > 0.0f) z = soft_cap16(z, cap, inv_cap);
      y[(size_t)lane * V + r] = from_f32<T>(z);
    }
  });
}

// Split form: one vocabulary tile per workgroup, wave wv over k-steps
// [wv nkw, (wv + 1) nkw); the k-steps of a block are loaded together, then run.
template <typename T>
__global__ __launch_bounds__(64 * LS_WAVES) void lm_head_split_kernel(const T* __restrict__ x,
                                                                      const T* __restrict__ w, T* __restrict__ y,
                                                                      int M, int D, int V, float cap,
                                                                      float inv_cap) {
  __shared__ f32x4 s_part[LS_WAVES - 1][64];
  const int lane = threadIdx.x & 63, g = lane >> 4, r16 = lane & 15, wv = threadIdx.x >> 6;
  const int v0 = blockIdx.x * 16;
  const int nk = (D + 31) / 32;
  const int nkw = (nk + LS_WAVES - 1) / LS_WAVES;
  const int kbeg = wv * nkw, kend = min(nk, kbeg + nkw);
  // vocabulary rows past V re-read row V - 1, token rows past M re-read row M - 1
  // (neither is stored)
  const T* wr = w + (size_t)min(v0 + r16, V - 1) * D + 8 * g;
  const T* xr = x + (size_t)min(r16, M - 1) * D + 8 * g;
  // k-slice [32 ks + 8 g, +8) lies wholly inside or outside D; past D (or past the
  // wave's range) the address is clamped in bounds and both operands are zeroed
  auto koff = [&](int ks) { return min(32 * ks, D - 8 - 8 * g); };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int k0 = kbeg; k0 < kend; k0 += LS_KB) {
    u32x4 a[LS_KB], b[LS_KB];
#pragma unroll
    for (int p = 0; p < LS_KB; ++p) {
      const int ko = koff(min(k0 + p, nk - 1));
      a[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + ko));
      b[p] = *reinterpret_cast<const u32x4*>(xr + ko);
    }
#pragma unroll
    for (int p = 0; p < LS_KB; ++p) {
      const int ks = k0 + p;
      const bool in_d = ks < kend && 32 * ks + 8 * g < D;
      acc = mfma16<T>(in_d ? a[p] : zero, in_d ? b[p] : zero, acc);
    }
  }
  if (wv > 0) s_part[wv - 1][lane] = acc;
  __syncthreads();
  if (wv > 0 || r16 >= M) return;
#pragma unroll
  for (int q = 0; q < LS_WAVES - 1; ++q) acc += s_part[q][lane];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = v0 + 4 * g + e;
    if (v >= V) continue;
    float z = round_to<T>(acc[e]);  // the Linear's output in its dtype
    if (cap > 0.0f) z = soft_cap16(z, cap, inv_cap);
    y[(size_t)r16 * V + v] = from_f32<T>(z);
  }
}

// Staged form: the token rows in LDS, one whole vocabulary tile per wave.
template <typename T>
__global__ __launch_bounds__(LH_BLOCK) void lm_head_staged_kernel(const T* __restrict__ x,
                                                                  const T* __restrict__ w, T* __restrict__ y, int M,
                                                                  int D, int V, float cap, float inv_cap) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  T* xs = reinterpret_cast<T*>(lds_raw);
  const int ld = D + 8;
  const int pieces = D / 8;  // 16-byte pieces per row (D % 8 == 0)
  for (int p = threadIdx.x; p < M * pieces; p += LH_BLOCK) {
    const int r = p / pieces, c = p - r * pieces;
    *reinterpret_cast<u32x4*>(xs + r * ld + 8 * c) = *reinterpret_cast<const u32x4*>(x + (size_t)r * D + 8 * c);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, g = lane >> 4, r16 = lane & 15, wv = threadIdx.x >> 6;
  const int v0 = (blockIdx.x * LH_WAVES + wv) * 16;
  if (v0 >= V) return;  // no barrier follows
  const int nk = (D + 31) / 32;
  // vocabulary rows past V re-read row V - 1, token rows past M re-read row M - 1
  // (neither is stored)
  const T* wr = w + (size_t)min(v0 + r16, V - 1) * D + 8 * g;
  const T* xr = xs + min(r16, M - 1) * ld + 8 * g;
  // k-slice [32 ks + 8 g, +8) lies wholly inside or outside D; past D the address
  // is clamped in bounds and both operands are zeroed
  auto koff = [&](int ks) { return min(32 * ks, D - 8 - 8 * g); };
  u32x4 wa[2][LH_KB];
  auto load_block = [&](int blk, auto buf_tag) {
    constexpr int b = decltype(buf_tag)::value;
#pragma unroll
    for (int p = 0; p < LH_KB; ++p)
      wa[b][p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + koff(min(blk * LH_KB + p, nk - 1))));
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto run_block = [&](int blk, auto buf_tag) {
    constexpr int b = decltype(buf_tag)::value;
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < LH_KB; ++p) {
      const int ks = blk * LH_KB + p;
      const bool in_d = ks < nk && 32 * ks + 8 * g < D;
      const u32x4 xb = *reinterpret_cast<const u32x4*>(xr + koff(min(ks, nk - 1)));
      acc = mfma16<T>(in_d ? wa[b][p] : zero, in_d ? xb : zero, acc);
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // two blocks per trip keep the buffer indices compile-time constants; the
  // prefetches in the loop need no branch, the last one or two blocks run after it
  const int nblk = (nk + LH_KB - 1) / LH_KB;
  load_block(0, B0{});
  int blk = 0;
  for (; blk + 2 < nblk; blk += 2) {
    load_block(blk + 1, B1{});
    run_block(blk, B0{});
    load_block(blk + 2, B0{});
    run_block(blk + 1, B1{});
  }
  if (blk + 1 < nblk) {
    load_block(blk + 1, B1{});
    run_block(blk, B0{});
    run_block(blk + 1, B1{});
  } else {
    run_block(blk, B0{});
  }
  if (r16 >= M) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = v0 + 4 * g + e;
    if (v >= V) continue;
    float z = round_to<T>(acc[e]);  // the Linear's output in its dtype
    if (cap > 0.0f) z = soft_cap16(z, cap, inv_cap);
    y[(size_t)r16 * V + v] = from_f32<T>(z);
  }
}

template <typename T>
const void* rows_kernel(int M, int D) {
  const int mt = rowgemv::small_rows(M, D);
  if (!mt) return nullptr;
  XL_ROWGEMV_PICK(lm_head_rows_kernel, T, mt, D / 512);
}

template <typename T>
int launch(const void* x, const void* w, void* y, int M, int D, int V, float cap, hipStream_t st) {
  const int64_t tiles = ((int64_t)V + 15) / 16;
  const float inv_cap = cap > 0.0f ? 1.0f / cap : 0.0f;
  if (const void* rk = rows_kernel<T>(M, D)) {
    void* args[] = {(void*)&x, (void*)&w, (void*)&y, (void*)&M, (void*)&D, (void*)&V, (void*)&cap, (void*)&inv_cap};
    return rowgemv::launch_streaming(rk, args, V, st, "xl_lm_head_softcap_fwd");
  }
  if (M <= LS_MAX_ROWS) {
    hipLaunchKernelGGL(lm_head_split_kernel<T>, dim3((unsigned)tiles), dim3(64 * LS_WAVES), 0, st, (const T*)x,
                       (const T*)w, (T*)y, M, D, V, cap, inv_cap);
    return check_launch("xl_lm_head_softcap_fwd");
  }
  const int64_t blocks = (tiles + LH_WAVES - 1) / LH_WAVES;
  const size_t smem = lds_bytes(M, D);
  hipError_t e = hipFuncSetAttribute((const void*)lm_head_staged_kernel<T>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess)
    return set_error(XL_ERR_LAUNCH, "xl_lm_head_softcap_fwd: LDS attribute failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(lm_head_staged_kernel<T>, dim3((unsigned)blocks), dim3(LH_BLOCK), smem, st, (const T*)x,
                     (const T*)w, (T*)y, M, D, V, cap, inv_cap);
  return check_launch("xl_lm_head_softcap_fwd");
}

}  // namespace
}  // namespace xl

extern "C" int xl_lm_head_softcap_fwd(const void* x, const void* weight, void* y, int M, int D, int V, float cap,
                                      int dtype, void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_lm_head_softcap_fwd";
  if (M < 0 || D < 0 || V < 0) return set_error(XL_ERR_INVALID_ARG, "%s: negative size (M=%d D=%d V=%d)", who, M, D, V);
  if (!dtype_ok(dtype)) return set_error(XL_ERR_INVALID_ARG, "%s: unknown dtype %d", who, dtype);
  if (dtype == XL_DTYPE_F32) return set_error(XL_ERR_UNSUPPORTED, "%s: float32 (bf16 / f16 MFMA kernel only)", who);
  if (M > LH_MAX_ROWS)
    return set_error(XL_ERR_UNSUPPORTED,
                     "%s: M=%d token rows (at most %d; more rows are a GEMM for the Linear, then soft_cap)", who, M,
                     LH_MAX_ROWS);
  if (D % 8 != 0 || (D == 0 && M > 0 && V > 0))
    return set_error(XL_ERR_UNSUPPORTED, "%s: D=%d (a positive multiple of 8)", who, D);
  if (lds_bytes(M, D) > LH_MAX_LDS)
    return set_error(XL_ERR_UNSUPPORTED, "%s: M=%d rows of D=%d do not fit the %zu-byte LDS staging", who, M, D,
                     LH_MAX_LDS);
  if (!(cap == cap) || cap == INFINITY) return set_error(XL_ERR_INVALID_ARG, "%s: cap must be finite", who);
  if ((int64_t)M * V == 0) return XL_OK;
  if (V > 0x7fffffff - 16) return set_error(XL_ERR_UNSUPPORTED, "%s: V=%d too large", who, V);
  if (!x || !weight || !y) return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if ((((uintptr_t)x) | ((uintptr_t)weight)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "%s: x and weight must be 16-byte aligned", who);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == XL_DTYPE_BF16) return launch<bf16_t>(x, weight, y, M, D, V, cap, st);
  return launch<f16_t>(x, weight, y, M, D, V, cap, st);
}
