// The element-wise stages of the sLSTM layer around its time loop:
//
//  * causal_conv1d_kernel — the projection cell's depthwise causal conv1d over
//    time with the SiLU after it (channels last, x [B, S, D]).  Each thread owns
//    one 16-byte vector of channels (8 bf16/f16 or 4 f32) over TS consecutive
//    time steps: it requests the TS + K - 1 input rows of its tile first (all
//    loads in flight at once), then slides a K-row window over them, K fused
//    multiply-adds per element.  The K - 1 halo rows a tile shares with the tile
//    before it come from L2, so HBM sees x once and y once.
//  * group_norm_kernel — the output cell's GroupNorm with one group per head:
//    rows of G groups of CG channels, each group normalised over its CG values.
//    A team of TL lanes (a power of two, at most one wave) holds one group in
//    registers, reduces the sum and then the centred sum of squares with lane
//    shuffles, and writes the affine result; groups too large for registers are
//    streamed three times (sum, centred squares, output) by a whole wave.
//
// Both are HBM streams (bytes per element: one read and one write of the
// element type); arithmetic is float32.
#include "common.h"

namespace xl {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// VW consecutive elements of T: one 16-byte access when VW * sizeof(T) == 16,
// else VW scalar accesses.
template <typename T, int VW>
union Row {
  static constexpr bool VEC = VW * sizeof(T) == 16;
  u32x4 raw;
  T e[VW];
};

template <typename T, int VW>
__device__ __forceinline__ Row<T, VW> load_row(const T* p) {
  Row<T, VW> r;
  if constexpr (Row<T, VW>::VEC) {
    r.raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) r.e[j] = p[j];
  }
  return r;
}

template <typename T, int VW>
__device__ __forceinline__ void store_row(T* p, const Row<T, VW>& r) {
  if constexpr (Row<T, VW>::VEC) {
    __builtin_nontemporal_store(r.raw, reinterpret_cast<u32x4*>(p));
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) p[j] = r.e[j];
  }
}

// x * sigmoid(x) = x / (1 + e^{-x}) with the hardware exp2 and reciprocal
// (e^{-x} overflows to +inf for x < -88, giving -0: the true value is below
// 1e-36 there).
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// ------------------------------------------------------------ causal conv1d
constexpr int CONV_TS = 16;     // time steps per thread
constexpr int CONV_BLOCK = 256;

// y[b, s, c] = act(bias[c] + sum_j w[c, j] x[b, s - K + 1 + j, c]), x = 0 before s = 0.
// With a 16-bit T the convolution is rounded to T before the activation (the
// convolution's own output dtype) and the activation's result once more.
template <typename T, int VW, int K>
__global__ __launch_bounds__(CONV_BLOCK) void causal_conv1d_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                   const T* __restrict__ bias, T* __restrict__ y,
                                                                   int S, int D, int nt, int64_t nitems, int act) {
  const int64_t item = (int64_t)blockIdx.x * CONV_BLOCK + threadIdx.x;
  if (item >= nitems) return;
  const int nvr = D / VW;
  const int cv = (int)(item % nvr);
  const int64_t rest = item / nvr;
  const int st = (int)(rest % nt);
  const int64_t b = rest / nt;
  const int c0 = cv * VW, s0 = st * CONV_TS;
  const T* xb = x + (size_t)b * S * D + c0;
  T* yb = y + (size_t)b * S * D + c0;

  // the tile's input rows s0 - K + 1 .. s0 + TS - 1, all requested before any use
  constexpr int NR = CONV_TS + K - 1;
  Row<T, VW> rows[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int s = s0 - (K - 1) + r;
    if (s >= 0 && s < S) {
      rows[r] = load_row<T, VW>(xb + (size_t)s * D);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) rows[r].e[j] = from_f32<T>(0.0f);
    }
  }
  float wt[VW][K], bs[VW];
#pragma unroll
  for (int j = 0; j < VW; ++j) {
    bs[j] = bias ? to_f32(bias[c0 + j]) : 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) wt[j][k] = to_f32(w[(size_t)(c0 + j) * K + k]);
  }
#pragma unroll
  for (int t = 0; t < CONV_TS; ++t) {
    const int s = s0 + t;
    if (s >= S) break;
    float a[VW];
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      float acc = bs[j];
#pragma unroll
      for (int k = 0; k < K; ++k) acc = fmaf(wt[j][k], to_f32(rows[t + k].e[j]), acc);
      a[j] = acc;
    }
    Row<T, VW> out;
    if (act) {
#pragma unroll
      for (int j = 0; j + 1 < VW; j += 2) round2_to<T>(a[j], a[j + 1]);
      if (VW & 1) a[VW - 1] = round_to<T>(a[VW - 1]);
#pragma unroll
      for (int j = 0; j < VW; ++j) out.e[j] = from_f32<T>(silu(a[j]));
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) out.e[j] = from_f32<T>(a[j]);
    }
    store_row<T, VW>(yb + (size_t)s * D, out);
  }
}

template <typename T, int VW>
int launch_conv_vw(const void* x, const void* w, const void* bias, void* y, int B, int S, int D, int K, int act,
                   hipStream_t st) {
  const int nt = (S + CONV_TS - 1) / CONV_TS;
  const int64_t nitems = (int64_t)B * nt * (D / VW);
  const int64_t blocks = (nitems + CONV_BLOCK - 1) / CONV_BLOCK;
  if (blocks > 0x7fffffff) return set_error(XL_ERR_UNSUPPORTED, "xl_causal_conv1d_fwd: input too large");
  const T *xp = (const T*)x, *wp = (const T*)w, *bp = (const T*)bias;
  T* yp = (T*)y;
#define XL_CONV_CASE(KK)                                                                                  \
  case KK:                                                                                                \
    hipLaunchKernelGGL((causal_conv1d_kernel<T, VW, KK>), dim3((unsigned)blocks), dim3(CONV_BLOCK), 0, st, xp, wp, \
                       bp, yp, S, D, nt, nitems, act);                                                    \
    break;
  switch (K) {
    XL_CONV_CASE(1) XL_CONV_CASE(2) XL_CONV_CASE(3) XL_CONV_CASE(4)
    XL_CONV_CASE(5) XL_CONV_CASE(6) XL_CONV_CASE(7) XL_CONV_CASE(8)
    default: return set_error(XL_ERR_UNSUPPORTED, "xl_causal_conv1d_fwd: kernel size %d (1..8)", K);
  }
#undef XL_CONV_CASE
  return check_launch("xl_causal_conv1d_fwd");
}

template <typename T>
int launch_conv(const void* x, const void* w, const void* bias, void* y, int B, int S, int D, int K, int act,
                hipStream_t st) {
  constexpr int VW = 16 / sizeof(T);
  const bool vec = D % VW == 0 && ((((uintptr_t)x) | ((uintptr_t)y)) & 15u) == 0;
  return vec ? launch_conv_vw<T, VW>(x, w, bias, y, B, S, D, K, act, st)
             : launch_conv_vw<T, 1>(x, w, bias, y, B, S, D, K, act, st);
}

// --------------------------------------------------------------- group norm
constexpr int GN_BLOCK = 256;

__device__ __forceinline__ float team_sum(float v, int tl) {
  for (int o = tl >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One team of tl lanes per (row, group); NV > 0: the group's NVG = CG / VW
// vectors are held in registers (NVG <= tl * NV); NV == 0: a whole wave
// (tl = 64) streams the group three times.
template <typename T, int VW, int NV>
__global__ __launch_bounds__(GN_BLOCK) void group_norm_kernel(const T* x, const T* __restrict__ w,
                                                              const T* __restrict__ bias, T* y, int64_t nteams, int G,
                                                              int CG, int tl, float eps) {
  const int64_t gt = (int64_t)blockIdx.x * GN_BLOCK + threadIdx.x;
  const int64_t team = gt / tl;
  const int t = (int)(gt % tl);
  if (team >= nteams) return;  // whole teams leave together: no shuffle reads an exited lane
  const int g = (int)(team % G);
  const size_t base = (size_t)team * CG;  // rows are G * CG wide: team * CG = row * G * CG + g * CG
  const T* xg = x + base;
  T* yg = y + base;
  const int nvg = CG / VW;
  const float inv_n = 1.0f / (float)CG;
  const int cbase = g * CG;

  auto affine = [&](const Row<T, VW>& in, int v, float mean, float rstd) {
    Row<T, VW> out;
    const int c = cbase + v * VW;
    if (w) {
      const Row<T, VW> wr = load_row<T, VW>(w + c), br = load_row<T, VW>(bias + c);
#pragma unroll
      for (int j = 0; j < VW; ++j)
        out.e[j] = from_f32<T>(fmaf((to_f32(in.e[j]) - mean) * rstd, to_f32(wr.e[j]), to_f32(br.e[j])));
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) out.e[j] = from_f32<T>((to_f32(in.e[j]) - mean) * rstd);
    }
    return out;
  };

  if constexpr (NV > 0) {
    Row<T, VW> v[NV];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int vi = t + tl * k;
      if (vi < nvg) {
        v[k] = load_row<T, VW>(xg + (size_t)vi * VW);
#pragma unroll
        for (int j = 0; j < VW; ++j) s += to_f32(v[k].e[j]);
      }
    }
    const float mean = team_sum(s, tl) * inv_n;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (t + tl * k < nvg) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float d = to_f32(v[k].e[j]) - mean;
          q = fmaf(d, d, q);
        }
      }
    }
    const float rstd = __builtin_amdgcn_rsqf(team_sum(q, tl) * inv_n + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int vi = t + tl * k;
      if (vi < nvg) store_row<T, VW>(yg + (size_t)vi * VW, affine(v[k], vi, mean, rstd));
    }
  } else {
    float s = 0.0f;
    for (int vi = t; vi < nvg; vi += tl) {
      const Row<T, VW> r = load_row<T, VW>(xg + (size_t)vi * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j) s += to_f32(r.e[j]);
    }
    const float mean = team_sum(s, tl) * inv_n;
    float q = 0.0f;
    for (int vi = t; vi < nvg; vi += tl) {
      const Row<T, VW> r = load_row<T, VW>(xg + (size_t)vi * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float d = to_f32(r.e[j]) - mean;
        q = fmaf(d, d, q);
      }
    }
    const float rstd = __builtin_amdgcn_rsqf(team_sum(q, tl) * inv_n + eps);
    for (int vi = t; vi < nvg; vi += tl) store_row<T, VW>(yg + (size_t)vi * VW, affine(load_row<T, VW>(xg + (size_t)vi * VW), vi, mean, rstd));
  }
}

constexpr int GN_NV_MAX = 8;  // vectors per lane held in registers (a 64-lane team: 64 * 8 vectors)

template <typename T, int VW>
int launch_gn_vw(const void* x, const void* w, const void* bias, void* y, int64_t N, int G, int CG, float eps,
                 hipStream_t st) {
  const int nvg = CG / VW;
  int tl = 1;
  while (tl < nvg && tl < 64) tl <<= 1;
  const int nv = (nvg + tl - 1) / tl;
  const int64_t nteams = N * G;
  const int64_t blocks = (nteams * tl + GN_BLOCK - 1) / GN_BLOCK;
  if (blocks > 0x7fffffff) return set_error(XL_ERR_UNSUPPORTED, "xl_group_norm_fwd: input too large");
  const T *xp = (const T*)x, *wp = (const T*)w, *bp = (const T*)bias;
  T* yp = (T*)y;
  const dim3 grid((unsigned)blocks), blk(GN_BLOCK);
  if (nv <= 1)
    hipLaunchKernelGGL((group_norm_kernel<T, VW, 1>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, eps);
  else if (nv <= 2)
    hipLaunchKernelGGL((group_norm_kernel<T, VW, 2>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, eps);
  else if (nv <= 4)
    hipLaunchKernelGGL((group_norm_kernel<T, VW, 4>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, eps);
  else if (nv <= GN_NV_MAX)
    hipLaunchKernelGGL((group_norm_kernel<T, VW, 8>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, eps);
  else
    hipLaunchKernelGGL((group_norm_kernel<T, VW, 0>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, eps);
  return check_launch("xl_group_norm_fwd");
}

template <typename T>
int launch_gn(const void* x, const void* w, const void* bias, void* y, int64_t N, int G, int CG, float eps,
              hipStream_t st) {
  constexpr int VW = 16 / sizeof(T);
  const bool vec = CG % VW == 0 && ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)w) | ((uintptr_t)bias)) & 15u) == 0;
  return vec ? launch_gn_vw<T, VW>(x, w, bias, y, N, G, CG, eps, st)
             : launch_gn_vw<T, 1>(x, w, bias, y, N, G, CG, eps, st);
}

bool overlap(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
  return pa < pb + nb && pb < pa + na;
}

}  // namespace
}  // namespace xl

extern "C" int xl_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, void* y, int B, int S, int D,
                                    int K, int act, int dtype, void* stream) {
  using namespace xl;
  clear_error();
  if (B < 0 || S < 0 || D < 0)
    return set_error(XL_ERR_INVALID_ARG, "xl_causal_conv1d_fwd: negative size (B=%d S=%d D=%d)", B, S, D);
  if (!dtype_ok(dtype)) return set_error(XL_ERR_INVALID_ARG, "xl_causal_conv1d_fwd: unknown dtype %d", dtype);
  if (act != 0 && act != 1) return set_error(XL_ERR_INVALID_ARG, "xl_causal_conv1d_fwd: act=%d (0 none, 1 SiLU)", act);
  if (K < 1 || K > 8) return set_error(XL_ERR_UNSUPPORTED, "xl_causal_conv1d_fwd: kernel size %d (1..8)", K);
  if ((int64_t)B * S * D == 0) return XL_OK;
  if (!x || !weight || !y) return set_error(XL_ERR_INVALID_ARG, "xl_causal_conv1d_fwd: null pointer");
  const size_t nb = (size_t)B * S * D * dtype_size(dtype);
  if (overlap(x, nb, y, nb)) return set_error(XL_ERR_INVALID_ARG, "xl_causal_conv1d_fwd: y must not alias x");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case XL_DTYPE_F32: return launch_conv<float>(x, weight, bias, y, B, S, D, K, act, st);
    case XL_DTYPE_BF16: return launch_conv<bf16_t>(x, weight, bias, y, B, S, D, K, act, st);
    default: return launch_conv<f16_t>(x, weight, bias, y, B, S, D, K, act, st);
  }
}

extern "C" int xl_group_norm_fwd(const void* x, const void* weight, const void* bias, void* y, int64_t N, int G,
                                 int CG, float eps, int dtype, void* stream) {
  using namespace xl;
  clear_error();
  if (N < 0 || G < 1 || CG < 1)
    return set_error(XL_ERR_INVALID_ARG, "xl_group_norm_fwd: bad size (N=%lld G=%d CG=%d)", (long long)N, G, CG);
  if (!dtype_ok(dtype)) return set_error(XL_ERR_INVALID_ARG, "xl_group_norm_fwd: unknown dtype %d", dtype);
  if (!(eps >= 0.0f) || eps == INFINITY) return set_error(XL_ERR_INVALID_ARG, "xl_group_norm_fwd: eps must be finite and >= 0");
  if (!weight != !bias) return set_error(XL_ERR_INVALID_ARG, "xl_group_norm_fwd: weight and bias must both be given or both NULL");
  if (N == 0) return XL_OK;
  if (!x || !y) return set_error(XL_ERR_INVALID_ARG, "xl_group_norm_fwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case XL_DTYPE_F32: return launch_gn<float>(x, weight, bias, y, N, G, CG, eps, st);
    case XL_DTYPE_BF16: return launch_gn<bf16_t>(x, weight, bias, y, N, G, CG, eps, st);
    default: return launch_gn<f16_t>(x, weight, bias, y, N, G, CG, eps, st);
  }
}
