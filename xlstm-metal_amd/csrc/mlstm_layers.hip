// The mLSTM output cell's element-wise stage after the chunkwise kernel:
// per-head RMS normalisation of h, the per-channel weight, and the output gate
// sigma(o), written as the flattened [B, S, NH * DH] input of the output
// projection — one pass over HBM instead of the reference's permute, float
// upcast, square, mean, divide, cast, weight product, sigmoid and gate product.
//
// One team of tl lanes (a power of two, at most one wave) per (b, s, head)
// group of DH channels, R = 2 groups per team with every load issued before the
// first reduction; the sum of squares is reduced with DPP when the team is the
// whole wave.  h may be read in the chunkwise kernel's [B, NH, S, DH] layout
// (the reference permutes it) or already as [B, S, NH, DH].  HBM-bound: h and
// the gate pre-activation read once, the output written once.
#include "common.h"

#include <type_traits>

namespace xl {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T, int VW>
union Vec {
  static constexpr bool VEC = VW * sizeof(T) == 16;
  u32x4 raw;
  T e[VW];
};

template <typename T, int VW, bool NT>
__device__ __forceinline__ Vec<T, VW> ld(const T* p) {
  Vec<T, VW> r;
  if constexpr (Vec<T, VW>::VEC) {
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
__device__ __forceinline__ void st_nt(T* p, const float (&a)[VW]) {
  Vec<T, VW> out;
  if constexpr (!is_f32<T>::value && VW % 2 == 0) {
    uint32_t* o32 = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
    for (int j = 0; j < VW; j += 2) {
      const xl_f32x2 v = {a[j], a[j + 1]};
      if constexpr (std::is_same<T, bf16_t>::value)
        o32[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, xl_bf16x2));
      else
        o32[j / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, xl_f16x2));
    }
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) out.e[j] = from_f32<T>(a[j]);
  }
  if constexpr (Vec<T, VW>::VEC) {
    __builtin_nontemporal_store(out.raw, reinterpret_cast<u32x4*>(p));
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) p[j] = out.e[j];
  }
}

template <int TLC>
__device__ __forceinline__ float team_sum(float v, int tl) {
  if constexpr (TLC == 64) {
    v = lane_of(wave_sum_dpp(v), 63);
  } else {
    for (int o = tl >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  }
  return v;
}

constexpr int RMS_BLOCK = 256;
constexpr int RMS_R = 2;        // groups per team (one with 16 vectors per lane)
constexpr int RMS_NV_MAX = 16;  // vectors per lane held in registers
constexpr int RMS_SB = 8;       // steps per block of teams when h is [B, NH, S, DH]

// Teams visit the groups in blocks of SB consecutive steps x all NH heads:
// team = ((b * nsb + sblk) * NH + nh) * SB + si, step s = sblk * SB + si (teams
// with s >= S do nothing).  With h in [B, NH, S, DH] and SB = 8 a block reads
// h as NH runs of 8 rows and o / writes y as one run of 8 * NH rows (visiting
// (b, s, nh) in order instead read h in 1-row pieces S * DH apart: 13 % slower
// at config 2); with h in [B, S, NH, DH], SB = 1 is that order and every
// stream is one run.  The reference's roundings for a 16-bit T: (h / rms) cast
// to T, times the weight in T, sigmoid of the gate in T, the product in T.
template <typename T, int VW, int NV, int TLC, int R>
__global__ __launch_bounds__(RMS_BLOCK) void mh_rmsnorm_gate_kernel(const T* __restrict__ h, const T* __restrict__ w,
                                                                    const T* __restrict__ o, T* __restrict__ y,
                                                                    int64_t nteams, int S, int NH, int DH, int SB,
                                                                    int h_heads_first, int tl_arg, float eps) {
  const int tl = TLC > 0 ? TLC : tl_arg;
  const int64_t gt = (int64_t)blockIdx.x * RMS_BLOCK + threadIdx.x;
  const int64_t slot = gt / tl;
  const int t = (int)(gt % tl);
  if (slot * R >= nteams) return;  // whole teams leave together
  const uint32_t nsb = (uint32_t)(S + SB - 1) / (uint32_t)SB;
  // (b, s, nh) of a team (32-bit: the host keeps the team count below 2^31);
  // s >= S marks a padding team of the last step block
  auto coords = [&](uint32_t team, uint32_t& b, uint32_t& s, uint32_t& nh) {
    const uint32_t q = team / (uint32_t)SB, si = team - q * (uint32_t)SB;
    const uint32_t bb = q / (uint32_t)NH;
    nh = q - bb * (uint32_t)NH;
    b = bb / nsb;
    s = (bb - b * nsb) * (uint32_t)SB + si;
  };
  const int nvg = DH / VW;
  constexpr bool LOWP = !is_f32<T>::value;

  // taps of the optional operands read branch-free (a load under a branch makes
  // the compiler wait for all earlier loads at the join): without them the same
  // offsets of h are read and the values dropped
  const bool has_w = w != nullptr, has_o = o != nullptr;
  const T* wsrc = has_w ? w : h;
  const T* osrc = has_o ? o : h;

  Vec<T, VW> xv[R][NV], ov[R][NV];
  float ss[R];
  size_t yoff[R];
  uint32_t head[R];
  bool live[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t team = slot * R + r;
    uint32_t b, s, nh;
    coords((uint32_t)team, b, s, nh);
    head[r] = nh;
    live[r] = team < nteams && s < (uint32_t)S;
    yoff[r] = ((size_t)(b * S + s) * NH + nh) * DH;  // also o's offset and h's in [B, S, NH, DH]
    const size_t hoff = h_heads_first ? ((size_t)(b * NH + nh) * S + s) * DH : yoff[r];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int vi = t + tl * k;
      if (live[r] && vi < nvg) {
        xv[r][k] = ld<T, VW, true>(h + hoff + (size_t)vi * VW);
        ov[r][k] = ld<T, VW, true>(osrc + (has_o ? yoff[r] : hoff) + (size_t)vi * VW);
      } else {
        xv[r][k].raw = u32x4{0u, 0u, 0u, 0u};
        ov[r][k].raw = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    ss[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float xf = to_f32(xv[r][k].e[j]);
        ss[r] = fmaf(xf, xf, ss[r]);
      }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) ss[r] = team_sum<TLC>(ss[r], tl);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (!live[r]) continue;
    const float inv_rms = __builtin_amdgcn_rsqf(ss[r] / (float)DH + eps);
    const int nh = (int)head[r];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int vi = t + tl * k;
      if (vi >= nvg) continue;
      const Vec<T, VW> wv = ld<T, VW, false>(wsrc + (has_w ? (size_t)nh * DH : 0) + (size_t)vi * VW);
      // 16-bit roundings two at a time with the packed hardware conversion
      auto round_all = [&](float (&a)[VW]) {
        if constexpr (LOWP) {
#pragma unroll
          for (int j = 0; j + 1 < VW; j += 2) round2_to<T>(a[j], a[j + 1]);
          if constexpr (VW & 1) a[VW - 1] = round_to<T>(a[VW - 1]);
        }
      };
      float out[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) out[j] = to_f32(xv[r][k].e[j]) * inv_rms;
      round_all(out);
      if (has_w) {
#pragma unroll
        for (int j = 0; j < VW; ++j) out[j] *= to_f32(wv.e[j]);
        round_all(out);
      }
      if (has_o) {
        float g[VW];
#pragma unroll
        for (int j = 0; j < VW; ++j)
          g[j] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * to_f32(ov[r][k].e[j])));
        round_all(g);
#pragma unroll
        for (int j = 0; j < VW; ++j) out[j] *= g[j];
      }
      st_nt<T, VW>(y + yoff[r] + (size_t)vi * VW, out);
    }
  }
}

template <typename T, int VW>
int launch_vw(const void* h, const void* w, const void* o, void* y, int B, int NH, int S, int DH, int layout,
              float eps, hipStream_t st) {
  const int nvg = DH / VW;
  int tl = 1;
  while (tl < nvg && tl < 64) tl <<= 1;
  const int nv = (nvg + tl - 1) / tl;
  if (nv > RMS_NV_MAX)
    return set_error(XL_ERR_UNSUPPORTED, "xl_mh_rmsnorm_gate_fwd: head dim %d above %d", DH, 64 * RMS_NV_MAX * VW);
  const int SB = layout ? RMS_SB : 1;
  const int64_t nteams = (int64_t)B * ((S + SB - 1) / SB) * SB * NH;  // with the last block's padding teams
  if (nteams + RMS_R > 0x7fffffff)
    return set_error(XL_ERR_UNSUPPORTED, "xl_mh_rmsnorm_gate_fwd: B*S*NH = %lld groups (below 2^31)", (long long)nteams);
  const int r = nv <= 8 ? RMS_R : 1;
  const int64_t blocks = ((nteams + r - 1) / r * tl + RMS_BLOCK - 1) / RMS_BLOCK;
  if (blocks > 0x7fffffff) return set_error(XL_ERR_UNSUPPORTED, "xl_mh_rmsnorm_gate_fwd: input too large");
  const T *hp = (const T*)h, *wp = (const T*)w, *op = (const T*)o;
  T* yp = (T*)y;
  const dim3 grid((unsigned)blocks), blk(RMS_BLOCK);
#define XL_RMS_LAUNCH(NV, RR)                                                                                     \
  do {                                                                                                            \
    if (tl == 64)                                                                                                 \
      hipLaunchKernelGGL((mh_rmsnorm_gate_kernel<T, VW, NV, 64, RR>), grid, blk, 0, st, hp, wp, op, yp, nteams, S, NH, \
                         DH, SB, layout, tl, eps);                                                                    \
    else                                                                                                          \
      hipLaunchKernelGGL((mh_rmsnorm_gate_kernel<T, VW, NV, 0, RR>), grid, blk, 0, st, hp, wp, op, yp, nteams, S, NH,  \
                         DH, SB, layout, tl, eps);                                                                    \
  } while (0)
  if (nv <= 1)
    XL_RMS_LAUNCH(1, RMS_R);
  else if (nv <= 2)
    XL_RMS_LAUNCH(2, RMS_R);
  else if (nv <= 4)
    XL_RMS_LAUNCH(4, RMS_R);
  else if (nv <= 8)
    XL_RMS_LAUNCH(8, RMS_R);
  else
    XL_RMS_LAUNCH(16, 1);
#undef XL_RMS_LAUNCH
  return check_launch("xl_mh_rmsnorm_gate_fwd");
}

template <typename T>
int launch(const void* h, const void* w, const void* o, void* y, int B, int NH, int S, int DH, int layout, float eps,
           hipStream_t st) {
  constexpr int VW = 16 / sizeof(T);
  const bool vec =
      DH % VW == 0 && ((((uintptr_t)h) | ((uintptr_t)w) | ((uintptr_t)o) | ((uintptr_t)y)) & 15u) == 0;
  return vec ? launch_vw<T, VW>(h, w, o, y, B, NH, S, DH, layout, eps, st)
             : launch_vw<T, 1>(h, w, o, y, B, NH, S, DH, layout, eps, st);
}

bool overlap(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
  return pa < pb + nb && pb < pa + na;
}

}  // namespace
}  // namespace xl

extern "C" int xl_mh_rmsnorm_gate_fwd(const void* h, const void* weight, const void* o_preact, void* y, int B, int NH,
                                      int S, int DH, int h_layout, float eps, int dtype, void* stream) {
  using namespace xl;
  clear_error();
  if (B < 0 || NH < 0 || S < 0 || DH < 0)
    return set_error(XL_ERR_INVALID_ARG, "xl_mh_rmsnorm_gate_fwd: negative size (B=%d NH=%d S=%d DH=%d)", B, NH, S, DH);
  if (!dtype_ok(dtype)) return set_error(XL_ERR_INVALID_ARG, "xl_mh_rmsnorm_gate_fwd: unknown dtype %d", dtype);
  if (h_layout != 0 && h_layout != 1)
    return set_error(XL_ERR_INVALID_ARG, "xl_mh_rmsnorm_gate_fwd: h_layout=%d (0 [B,S,NH,DH], 1 [B,NH,S,DH])", h_layout);
  if (!(eps >= 0.0f) || eps == INFINITY)
    return set_error(XL_ERR_INVALID_ARG, "xl_mh_rmsnorm_gate_fwd: eps must be finite and >= 0");
  if ((int64_t)B * NH * S * DH == 0) return XL_OK;
  if (!h || !y) return set_error(XL_ERR_INVALID_ARG, "xl_mh_rmsnorm_gate_fwd: null pointer");
  const size_t nb = (size_t)B * NH * S * DH * dtype_size(dtype);
  if (overlap(h, nb, y, nb) || (o_preact && overlap(o_preact, nb, y, nb)))
    return set_error(XL_ERR_INVALID_ARG, "xl_mh_rmsnorm_gate_fwd: y must not alias h or o_preact");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case XL_DTYPE_F32: return launch<float>(h, weight, o_preact, y, B, NH, S, DH, h_layout, eps, st);
    case XL_DTYPE_BF16: return launch<bf16_t>(h, weight, o_preact, y, B, NH, S, DH, h_layout, eps, st);
    default: return launch<f16_t>(h, weight, o_preact, y, B, NH, S, DH, h_layout, eps, st);
  }
}
