// Gate projection with the soft-cap epilogue: Y[m, n] = softcap(b[n] + sum_d
// X[m, d] W[n, d]) for the few gate outputs of an mLSTM / sLSTM projection cell
// (G = NH or 2 NH columns), replacing nn.Linear(D, NH) launches that each read
// the whole activation plus a separate soft-cap pass.
//
// A skinny GEMM (M = B * S rows, D up to a few thousand, G <= 64) is bound by
// reading X once.  Where D is a multiple of 512 and the G weight rows' slices
// fit 128 registers (config 4's sLSTM gates: D 2048, G 8 or 4), the
// row-streaming loop of rows_gemv.h reads each X row as 1 KB contiguous loads
// with the weight rows held in registers (gate_rows_kernel).  Otherwise a
// workgroup per 16 rows, its 4 waves over 4 ranges of k,
// runs v_mfma_f32_16x16x32 (bf16 / f16) straight from the streamed rows (the
// partial products summed through LDS): lane (g, r16) holds row r16's k-slice
// 8g .. 8g + 7 of every 32-wide k-step (one 16-byte load, the next k-step
// continues the row), the weights come from the caches (W is a few KB to a few
// tens of KB and every wave re-reads it), one block of k-steps ahead.  The
// epilogue adds the bias, rounds to the Linear's output dtype and applies
// cap * tanh(x / cap), either in float32 with one more rounding (cap_rounding 0:
// SoftCapCell, which computes in float32 and casts once) or with every
// operation rounded to the dtype (cap_rounding 1: cap * torch.tanh(x / cap) on
// 16-bit tensors, as sLSTMProjectionCell.soft_cap evaluates it,
// xlstm_metal/torch_native/blocks/slstm/slstm_layers/slstm_projection_cell.py:84-89).
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

// The bias, the Linear's rounding and the soft-cap of one output (both forms).
template <typename T>
__device__ __forceinline__ float gate_epilogue(float acc, float bn, float cap, float inv_cap, int cap_rounding) {
  float v = round_to<T>(acc + bn);  // the Linear's output in its dtype
  if (cap > 0.0f) {
    if (cap_rounding) {  // cap, x / cap, tanh and the product each in the dtype
      const float capr = round_to<T>(cap);
      v = capr * round_to<T>(tanh_f32(round_to<T>(v / capr)));
    } else {
      v = soft_cap16(v, cap, inv_cap);
    }
  }
  return v;
}

constexpr int GP_WAVES = 4;  // waves per 16-row tile, each over a quarter of the k-steps
constexpr int GP_BLOCK = 64 * GP_WAVES;

// A workgroup = one 16-row tile; its 4 waves split the k-steps into 4
// contiguous ranges (4x the loads in flight of one wave per tile) and their
// partial 16 x 16 accumulators are summed through LDS by wave 0.
template <typename T, int NT>
__global__ __launch_bounds__(GP_BLOCK) void gate_proj_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                             const T* __restrict__ bias, T* __restrict__ y, int M,
                                                             int D, int G, float cap, float inv_cap,
                                                             int cap_rounding) {
  __shared__ f32x4 s_part[GP_WAVES - 1][NT][64];
  const int lane = threadIdx.x & 63, g = lane >> 4, r16 = lane & 15, wv = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16;
  const int nk = (D + 31) / 32;
  const int nkw = (nk + GP_WAVES - 1) / GP_WAVES;  // k-steps per wave
  const int kbeg = wv * nkw, kend = min(nk, kbeg + nkw);
  // rows past M re-read row M - 1 (their results are not stored)
  const T* xr = x + (size_t)min(m0 + r16, M - 1) * D + 8 * g;
  // weight rows past G re-read row G - 1 (their columns are not stored)
  const T* wr[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) wr[nt] = w + (size_t)min(nt * 16 + r16, G - 1) * D + 8 * g;

  // k-slice [32 ks + 8 g, +8) of a row lies wholly inside or outside D (D % 8 == 0);
  // past D (or past this wave's range) the address is clamped in bounds and both
  // operands are zeroed
  auto koff = [&](int ks) { return min(32 * ks, D - 8 - 8 * g); };
  // Blocks of KB k-steps, X and W of block j + 1 loaded (double-buffered
  // registers) while block j's MFMAs run: loads retire in issue order, so a
  // weight load issued between X prefetches would make each MFMA wait for the
  // prefetches issued before it.
  constexpr int KB = NT <= 2 ? 8 : 4;
  u32x4 xa[2][KB], wa[2][KB][NT];
  auto load_block = [&](int blk, auto buf_tag) {
    constexpr int b = decltype(buf_tag)::value;
#pragma unroll
    for (int p = 0; p < KB; ++p) {
      const int ko = koff(min(kbeg + blk * KB + p, nk - 1));
      xa[b][p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + ko));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wa[b][p][nt] = *reinterpret_cast<const u32x4*>(wr[nt] + ko);
    }
  };
  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto run_block = [&](int blk, auto buf_tag) {
    constexpr int b = decltype(buf_tag)::value;
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < KB; ++p) {
      const int ks = kbeg + blk * KB + p;
      const bool in_d = ks < kend && 32 * ks + 8 * g < D;
      const u32x4 a = in_d ? xa[b][p] : zero;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma16<T>(a, in_d ? wa[b][p][nt] : zero, acc[nt]);
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // Two blocks per trip keep the buffer indices compile-time constants.  In the
  // loop both blocks ahead exist, so the prefetches need no branch (a load under
  // a branch makes the compiler wait for every load at the join); the last one
  // or two blocks run after it, each branch consuming what it loads.
  const int nblk = (max(kend - kbeg, 0) + KB - 1) / KB;
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
    run_block(blk, B0{});  // no k-steps left for this wave when nblk == 0: the block is all zeros
  }
  if (wv > 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) s_part[wv - 1][nt][lane] = acc[nt];
  }
  __syncthreads();
  if (wv > 0 || m0 >= M) return;
#pragma unroll
  for (int q = 0; q < GP_WAVES - 1; ++q)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] += s_part[q][nt][lane];
  // lane (g, r16) holds Y[m0 + 4 g + e][16 nt + r16]
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = nt * 16 + r16;
    if (n >= G) continue;
    const float bn = bias ? to_f32(bias[n]) : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 4 * g + e;
      if (m >= M) continue;
      y[(size_t)m * G + n] = from_f32<T>(gate_epilogue<T>(acc[nt][e], bn, cap, inv_cap, cap_rounding));
    }
  }
}

// Row form: X streamed row by row, the G weight rows as the small rows; lane n < G of the wave
// ends each row with output n, stored as one contiguous row of y.
template <typename T, int MT, int NPC>
__global__ __launch_bounds__(64 * rowgemv::WAVES) void gate_rows_kernel(const T* __restrict__ x,
                                                                        const T* __restrict__ w,
                                                                        const T* __restrict__ bias,
                                                                        T* __restrict__ y, int M, int D, int G,
                                                                        float cap, float inv_cap, int cap_rounding) {
  const int lane = threadIdx.x & 63;
  const float bn = (bias && lane < G) ? to_f32(bias[lane]) : 0.0f;
  rowgemv::stream_rows<T, MT, NPC>(w, G, x, M, D, [&](int r, int ln, float dot) {
    if (ln < G) y[(size_t)r * G + ln] = from_f32<T>(gate_epilogue<T>(dot, bn, cap, inv_cap, cap_rounding));
  });
}

template <typename T>
const void* gate_rows(int G, int D) {
  const int mt = rowgemv::small_rows(G, D);
  if (!mt) return nullptr;
  XL_ROWGEMV_PICK(gate_rows_kernel, T, mt, D / 512);
}

template <typename T>
int launch(const void* x, const void* w, const void* b, void* y, int M, int D, int G, float cap, int cap_rounding,
           hipStream_t st) {
  if (const void* rk = gate_rows<T>(G, D)) {
    const float inv = cap > 0.0f ? 1.0f / cap : 0.0f;
    void* args[] = {(void*)&x, (void*)&w,   (void*)&b,   (void*)&y,   (void*)&M,
                    (void*)&D, (void*)&G,   (void*)&cap, (void*)&inv, (void*)&cap_rounding};
    return rowgemv::launch_streaming(rk, args, M, st, "xl_gate_proj_softcap_fwd");
  }
  const int64_t blocks = ((int64_t)M + 15) / 16;
  if (blocks > 0x7fffffff) return set_error(XL_ERR_UNSUPPORTED, "xl_gate_proj_softcap_fwd: M=%d too large", M);
  const float inv_cap = cap > 0.0f ? 1.0f / cap : 0.0f;
  const T *xp = (const T*)x, *wp = (const T*)w, *bp = (const T*)b;
  T* yp = (T*)y;
  const dim3 grid((unsigned)blocks), blk(GP_BLOCK);
  switch ((G + 15) / 16) {
    case 1: hipLaunchKernelGGL((gate_proj_kernel<T, 1>), grid, blk, 0, st, xp, wp, bp, yp, M, D, G, cap, inv_cap, cap_rounding); break;
    case 2: hipLaunchKernelGGL((gate_proj_kernel<T, 2>), grid, blk, 0, st, xp, wp, bp, yp, M, D, G, cap, inv_cap, cap_rounding); break;
    case 3: hipLaunchKernelGGL((gate_proj_kernel<T, 3>), grid, blk, 0, st, xp, wp, bp, yp, M, D, G, cap, inv_cap, cap_rounding); break;
    default: hipLaunchKernelGGL((gate_proj_kernel<T, 4>), grid, blk, 0, st, xp, wp, bp, yp, M, D, G, cap, inv_cap, cap_rounding); break;
  }
  return check_launch("xl_gate_proj_softcap_fwd");
}

}  // namespace
}  // namespace xl

extern "C" int xl_gate_proj_softcap_fwd(const void* x, const void* weight, const void* bias, void* y, int M, int D,
                                        int G, float cap, int cap_rounding, int dtype, void* stream) {
  using namespace xl;
  clear_error();
  if (M < 0 || D < 0 || G < 0)
    return set_error(XL_ERR_INVALID_ARG, "xl_gate_proj_softcap_fwd: negative size (M=%d D=%d G=%d)", M, D, G);
  if (!dtype_ok(dtype)) return set_error(XL_ERR_INVALID_ARG, "xl_gate_proj_softcap_fwd: unknown dtype %d", dtype);
  if (dtype == XL_DTYPE_F32)
    return set_error(XL_ERR_UNSUPPORTED, "xl_gate_proj_softcap_fwd: float32 (bf16 / f16 MFMA kernel only)");
  if (G > 64) return set_error(XL_ERR_UNSUPPORTED, "xl_gate_proj_softcap_fwd: G=%d outputs (at most 64)", G);
  if (D % 8 != 0 || (D == 0 && M > 0 && G > 0))
    return set_error(XL_ERR_UNSUPPORTED, "xl_gate_proj_softcap_fwd: D=%d (a positive multiple of 8)", D);
  if (!(cap == cap) || cap == INFINITY) return set_error(XL_ERR_INVALID_ARG, "xl_gate_proj_softcap_fwd: cap must be finite");
  if (cap_rounding != 0 && cap_rounding != 1)
    return set_error(XL_ERR_INVALID_ARG, "xl_gate_proj_softcap_fwd: cap_rounding must be 0 or 1");
  if ((int64_t)M * G == 0) return XL_OK;
  if (!x || !weight || !y) return set_error(XL_ERR_INVALID_ARG, "xl_gate_proj_softcap_fwd: null pointer");
  if ((((uintptr_t)x) | ((uintptr_t)weight)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "xl_gate_proj_softcap_fwd: x and weight must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == XL_DTYPE_BF16) return launch<bf16_t>(x, weight, bias, y, M, D, G, cap, cap_rounding, st);
  return launch<f16_t>(x, weight, bias, y, M, D, G, cap, cap_rounding, st);
}
