// The element-wise stages of the sLSTM layer around its time loop:
//
//  * causal_conv1d_kernel — the projection cell's depthwise causal conv1d over
//    time with the SiLU after it (channels last, x [B, S, D]).  Each thread owns
//    one 16-byte vector of channels (8 bf16/f16 or 4 f32) over TS consecutive
//    time steps: it requests the TS + K - 1 input rows of its tile first (all
//    loads in flight at once), then slides a K-row window over them, K fused
//    multiply-adds per element.  A workgroup spans several consecutive tiles,
//    so the K - 1 halo rows a tile shares with the tile before it mostly come
//    from the workgroup's own L2 and HBM sees x about once and y once.
//  * group_norm_kernel — the output cell's GroupNorm with one group per head:
//    rows of G groups of CG channels, each group normalised over its CG values.
//    A team of TL lanes (a power of two, at most one wave) holds two groups in
//    registers, reduces their sums and then their centred sums of squares with
//    lane shuffles, and writes the affine result; groups too large for
//    registers are streamed three times (sum, centred squares, output) by a
//    whole wave.
//
// Both are HBM streams (bytes per element: one read and one write of the
// element type); arithmetic is float32.
#include "common.h"

#include <type_traits>

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

// NT: a streamed tensor read once (nontemporal); otherwise a small operand
// every thread re-reads (weights), kept in the caches.
template <typename T, int VW, bool NT = true>
__device__ __forceinline__ Row<T, VW> load_row(const T* p) {
  Row<T, VW> r;
  if constexpr (Row<T, VW>::VEC) {
    if constexpr (NT)
      r.raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else
      r.raw = *reinterpret_cast<const u32x4*>(p);
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

// Packs VW floats into a row of T with the hardware conversions (round to
// nearest even, NaN kept): v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 for 16-bit T.
template <typename T, int VW>
__device__ __forceinline__ Row<T, VW> pack_row(const float (&a)[VW]) {
  Row<T, VW> out;
  if constexpr (!is_f32<T>::value && VW % 2 == 0) {
    uint32_t* o32 = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
    for (int j = 0; j < VW; j += 2) {
      const xl_f32x2 v = {a[j], a[j + 1]};
      if constexpr (sizeof(T) == 2 && std::is_same<T, bf16_t>::value)
        o32[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, xl_bf16x2));
      else
        o32[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, xl_f16x2));
    }
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) out.e[j] = from_f32<T>(a[j]);
  }
  return out;
}

// x * sigmoid(x) = x / (1 + e^{-x}) with the hardware exp2 and reciprocal
// (e^{-x} overflows to +inf for x < -88, giving -0: the true value is below
// 1e-36 there).
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// ------------------------------------------------------------ causal conv1d
constexpr int CONV_TS = 8;      // time steps per thread (config 4: 8 and 4 equal, 16 is 16 % slower)
constexpr int CONV_BLOCK = 256;

// y[b, s, c] = act(bias[c] + sum_j w[c, j] x[b, s - K + 1 + j, c]), x = 0 before s = 0.
// With a 16-bit T the convolution is rounded to T before the activation (the
// convolution's own output dtype) and the activation's result once more.
// A workgroup covers 2^cw_log2 channel vectors (a power of two, at most half a
// wave) x 256 / 2^cw_log2 consecutive time tiles of one batch row, so the K - 1
// halo rows a tile reads are mostly the rows of the tile before it in the same
// workgroup (same CU, same L2) rather than of a tile that may run on another XCD.
// Grid: x = channel-vector groups, y = time-tile groups, z = batch.
template <typename T, int VW, int K, bool ACT>
__global__ __launch_bounds__(CONV_BLOCK) void causal_conv1d_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                   const T* __restrict__ bias, T* __restrict__ y,
                                                                   int S, int D, int nt, int cw_log2) {
  const int nvr = D / VW;
  const int cv = (int)(blockIdx.x << cw_log2) + (int)(threadIdx.x & ((1u << cw_log2) - 1));
  const int st = (int)(blockIdx.y * (CONV_BLOCK >> cw_log2)) + (int)(threadIdx.x >> cw_log2);
  if (cv >= nvr || st >= nt) return;
  const int64_t b = blockIdx.z;
  const int c0 = cv * VW, s0 = st * CONV_TS;
  const T* xb = x + (size_t)b * S * D + c0;
  T* yb = y + (size_t)b * S * D + c0;

  // taps and bias first, with no branch: a load under a branch makes the
  // compiler wait for every load issued before it (the rows) at the join.
  // Without a bias the same addresses of w are read and the value dropped.
  const bool has_bias = bias != nullptr;
  const T* bsrc = has_bias ? bias : w;
  float wt[VW][K], bs[VW];
#pragma unroll
  for (int j = 0; j < VW; ++j) {
    const float bv = to_f32(bsrc[c0 + j]);
    bs[j] = has_bias ? bv : 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) wt[j][k] = to_f32(w[(size_t)(c0 + j) * K + k]);
  }
  // the tile's input rows s0 - K + 1 .. s0 + TS - 1, all requested before any use
  constexpr int NR = CONV_TS + K - 1;
  Row<T, VW> rows[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int s = s0 - (K - 1) + r;
    if (s >= 0 && s < S) {
      rows[r] = load_row<T, VW>(xb + (size_t)s * D);
    } else {
      rows[r].raw = u32x4{0u, 0u, 0u, 0u};
    }
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
    if constexpr (ACT) {
#pragma unroll
      for (int j = 0; j + 1 < VW; j += 2) round2_to<T>(a[j], a[j + 1]);
      if (VW & 1) a[VW - 1] = round_to<T>(a[VW - 1]);
#pragma unroll
      for (int j = 0; j < VW; ++j) a[j] = silu(a[j]);
    }
    store_row<T, VW>(yb + (size_t)s * D, pack_row<T, VW>(a));
  }
}

template <typename T, int VW>
int launch_conv_vw(const void* x, const void* w, const void* bias, void* y, int B, int S, int D, int K, int act,
                   hipStream_t st) {
  const int nt = (S + CONV_TS - 1) / CONV_TS;
  const int nvr = D / VW;
  // channel vectors per workgroup: the smallest power of two >= nvr, at most 32 (config 4: 32
  // vectors x 8 tiles 48.6 us, 64 x 4 50.8 us, 16 x 16 55.6 us)
  int cw_log2 = 0;
  while ((1 << cw_log2) < nvr && cw_log2 < 5) ++cw_log2;
  const int tiles_per_block = CONV_BLOCK >> cw_log2;
  const int64_t gx = (nvr + (1 << cw_log2) - 1) >> cw_log2, gy = (nt + tiles_per_block - 1) / tiles_per_block;
  if (gx > 0x7fffffff || gy > 65535 || B > 65535)
    return set_error(XL_ERR_UNSUPPORTED, "xl_causal_conv1d_fwd: input too large (B=%d S=%d D=%d)", B, S, D);
  const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)B);
  const T *xp = (const T*)x, *wp = (const T*)w, *bp = (const T*)bias;
  T* yp = (T*)y;
#define XL_CONV_CASE(KK)                                                                                     \
  case KK:                                                                                                   \
    if (act)                                                                                                 \
      hipLaunchKernelGGL((causal_conv1d_kernel<T, VW, KK, true>), grid, dim3(CONV_BLOCK), 0, st, xp, wp, bp, yp, S, \
                         D, nt, cw_log2);                                                                    \
    else                                                                                                     \
      hipLaunchKernelGGL((causal_conv1d_kernel<T, VW, KK, false>), grid, dim3(CONV_BLOCK), 0, st, xp, wp, bp, yp, \
                         S, D, nt, cw_log2);                                                                 \
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

// Sum over a team of tl lanes (an aligned power-of-two block of a wave).  With
// TLC = 64 the team is the whole wave: DPP row shifts and broadcasts put the
// total in lane 63, read back as a wave-uniform value (no LDS permutes);
// TLC = 0 takes tl at run time and exchanges through ds_bpermute.
template <int TLC>
__device__ __forceinline__ float team_sum(float v, int tl) {
  if constexpr (TLC == 64) {
    v = lane_of(wave_sum_dpp(v), 63);
  } else {
    for (int o = tl >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  }
  return v;
}

// One team of tl lanes per (row, group).  NV > 0: a team takes R consecutive
// groups and holds each group's NVG = CG / VW vectors in registers (NVG <= tl *
// NV); all R * NV loads are issued before the first reduction, so a wave keeps
// R times the bytes of one group in flight.  NV == 0: a whole wave (tl = 64)
// streams one group three times.
template <typename T, int VW, int NV, int R, int TLC>
__global__ __launch_bounds__(GN_BLOCK) void group_norm_kernel(const T* x, const T* __restrict__ w,
                                                              const T* __restrict__ bias, T* y, int64_t nteams, int G,
                                                              int CG, int tl_arg, float eps) {
  const int tl = TLC > 0 ? TLC : tl_arg;
  const int64_t gt = (int64_t)blockIdx.x * GN_BLOCK + threadIdx.x;
  const int64_t slot = gt / tl;
  const int t = (int)(gt % tl);
  if (slot * R >= nteams) return;  // whole teams leave together: no shuffle reads an exited lane
  const int nvg = CG / VW;
  const float inv_n = 1.0f / (float)CG;

  // rows are G * CG wide, so group `team` starts at team * CG.  The affine
  // parameters (each optional) are loaded without a branch (a load under a
  // branch makes the compiler wait for every earlier load at the join): a
  // missing one reads the same offsets of x (c < G * CG <= N * G * CG) and the
  // values are dropped.
  const bool has_w = w != nullptr, has_b = bias != nullptr;
  const T* wsrc = has_w ? w : x;
  const T* bsrc = has_b ? bias : x;
  auto affine = [&](const Row<T, VW>& in, int64_t team, int v, float mean, float rstd) {
    float o[VW];
    const int c = (int)(team % G) * CG + v * VW;
    const Row<T, VW> wr = load_row<T, VW, false>(wsrc + c), br = load_row<T, VW, false>(bsrc + c);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float xn = (to_f32(in.e[j]) - mean) * rstd;
      o[j] = fmaf(xn, has_w ? to_f32(wr.e[j]) : 1.0f, has_b ? to_f32(br.e[j]) : 0.0f);
    }
    return pack_row<T, VW>(o);
  };

  if constexpr (NV > 0) {
    // every load issued before the first use (a use inside the load's branch
    // would make the next load wait for it); missing vectors read as zeros
    Row<T, VW> v[R][NV];
    float s[R], q[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t team = slot * R + r;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int vi = t + tl * k;
        if (team < nteams && vi < nvg)
          v[r][k] = load_row<T, VW>(x + (size_t)team * CG + (size_t)vi * VW);
        else
          v[r][k].raw = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      s[r] = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int j = 0; j < VW; ++j) s[r] += to_f32(v[r][k].e[j]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = team_sum<TLC>(s[r], tl);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      s[r] *= inv_n;  // the mean
      q[r] = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (slot * R + r < nteams && t + tl * k < nvg) {
#pragma unroll
          for (int j = 0; j < VW; ++j) {
            const float d = to_f32(v[r][k].e[j]) - s[r];
            q[r] = fmaf(d, d, q[r]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) q[r] = team_sum<TLC>(q[r], tl);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t team = slot * R + r;
      if (team >= nteams) break;
      const float rstd = __builtin_amdgcn_rsqf(q[r] * inv_n + eps);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int vi = t + tl * k;
        if (vi < nvg)
          store_row<T, VW>(y + (size_t)team * CG + (size_t)vi * VW, affine(v[r][k], team, vi, s[r], rstd));
      }
    }
  } else {
    const int64_t team = slot;
    const T* xg = x + (size_t)team * CG;
    T* yg = y + (size_t)team * CG;
    float s = 0.0f;
    for (int vi = t; vi < nvg; vi += tl) {
      const Row<T, VW> r = load_row<T, VW>(xg + (size_t)vi * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j) s += to_f32(r.e[j]);
    }
    const float mean = team_sum<TLC>(s, tl) * inv_n;
    float q = 0.0f;
    for (int vi = t; vi < nvg; vi += tl) {
      const Row<T, VW> r = load_row<T, VW>(xg + (size_t)vi * VW);
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float d = to_f32(r.e[j]) - mean;
        q = fmaf(d, d, q);
      }
    }
    const float rstd = __builtin_amdgcn_rsqf(team_sum<TLC>(q, tl) * inv_n + eps);
    for (int vi = t; vi < nvg; vi += tl)
      store_row<T, VW>(yg + (size_t)vi * VW, affine(load_row<T, VW>(xg + (size_t)vi * VW), team, vi, mean, rstd));
  }
}

constexpr int GN_NV_MAX = 8;  // vectors per lane held in registers (a 64-lane team: 64 * 8 vectors)
constexpr int GN_R = 2;       // groups per team on the register path (2: 15 % faster than 1 at config 4; 4 no better)

template <typename T, int VW>
int launch_gn_vw(const void* x, const void* w, const void* bias, void* y, int64_t N, int G, int CG, float eps,
                 hipStream_t st) {
  const int nvg = CG / VW;
  int tl = 1;
  while (tl < nvg && tl < 64) tl <<= 1;
  const int nv = (nvg + tl - 1) / tl;
  const int64_t nteams = N * G;
  const int r = nv <= GN_NV_MAX ? GN_R : 1;  // groups per team
  const int64_t blocks = ((nteams + r - 1) / r * tl + GN_BLOCK - 1) / GN_BLOCK;
  if (blocks > 0x7fffffff) return set_error(XL_ERR_UNSUPPORTED, "xl_group_norm_fwd: input too large");
  const T *xp = (const T*)x, *wp = (const T*)w, *bp = (const T*)bias;
  T* yp = (T*)y;
  const dim3 grid((unsigned)blocks), blk(GN_BLOCK);
#define XL_GN_LAUNCH(NV, R)                                                                                  \
  do {                                                                                                       \
    if (tl == 64)                                                                                            \
      hipLaunchKernelGGL((group_norm_kernel<T, VW, NV, R, 64>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, \
                         eps);                                                                               \
    else                                                                                                     \
      hipLaunchKernelGGL((group_norm_kernel<T, VW, NV, R, 0>), grid, blk, 0, st, xp, wp, bp, yp, nteams, G, CG, tl, \
                         eps);                                                                               \
  } while (0)
  if (nv <= 1)
    XL_GN_LAUNCH(1, GN_R);
  else if (nv <= 2)
    XL_GN_LAUNCH(2, GN_R);
  else if (nv <= 4)
    XL_GN_LAUNCH(4, GN_R);
  else if (nv <= GN_NV_MAX)
    XL_GN_LAUNCH(8, GN_R);
  else
    XL_GN_LAUNCH(0, 1);
#undef XL_GN_LAUNCH
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
  if (N == 0) return XL_OK;
  if (!x || !y) return set_error(XL_ERR_INVALID_ARG, "xl_group_norm_fwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case XL_DTYPE_F32: return launch_gn<float>(x, weight, bias, y, N, G, CG, eps, st);
    case XL_DTYPE_BF16: return launch_gn<bf16_t>(x, weight, bias, y, N, G, CG, eps, st);
    default: return launch_gn<f16_t>(x, weight, bias, y, N, G, CG, eps, st);
  }
}
