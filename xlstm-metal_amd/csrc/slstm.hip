// sLSTM step (xl_slstm_step_fwd) and sequence (xl_slstm_seq_fwd).
//
// Reference math, torch-native variant (xlstm_metal/torch_native/blocks/
// slstm/slstm_layers/stepwise/slstm_metal_kernel.py:45-63), per (b, h, d):
//   m' = max(m + logsig(f), i);  ig = exp(i - m');  fg = exp(m + logsig(f) - m')
//   c' = fg c + ig tanh(z);      n' = fg n + ig;    h = sigmoid(o) c' / (|n'| + eps)
// Gates are per (b, h) and there is no recurrent matrix, so the recurrence is
// elementwise: one thread per (b, h, d), coalesced along d.  The sequence
// kernel splits the time axis over the waves of a workgroup (see below).
#include "common.h"

#include <type_traits>

namespace xl {

struct SGate {
  float ig, fg, og, mn;
};

__device__ __forceinline__ SGate slstm_gates(float ipre, float fpre, float opre, float m) {
  SGate g;
  const float lsf = logsigmoid(fpre);
  g.mn = fmaxf(m + lsf, ipre);
  g.ig = expf(ipre - g.mn);
  g.fg = expf(m + lsf - g.mn);
  g.og = sigmoid(opre);
  return g;
}

template <typename TZ, typename TG, typename TH>
__global__ __launch_bounds__(256) void slstm_step_kernel(const TZ* __restrict__ z, const TG* __restrict__ ip,
                                                         const TG* __restrict__ fp, const TG* __restrict__ op,
                                                         const float* c, const float* n, const float* __restrict__ m,
                                                         TH* __restrict__ h, float* c_new, float* n_new,
                                                         float* __restrict__ m_new, int64_t total, int H,
                                                         float eps) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t bh = idx / H;
  const SGate g = slstm_gates(to_f32(ip[bh]), to_f32(fp[bh]), to_f32(op[bh]), m[bh]);
  const float cn = g.fg * c[idx] + g.ig * tanh_f32(to_f32(z[idx]));
  const float nn = g.fg * n[idx] + g.ig;
  c_new[idx] = cn;
  n_new[idx] = nn;
  h[idx] = from_f32<TH>(g.og * cn / (fabsf(nn) + eps));
  if (idx - bh * H == 0) m_new[bh] = g.mn;
}

// ---------------------------------------------------------------- sequence
// The per-element recurrence is linear in (c, n) once the gates are known,
// and the stabiliser m depends on the gates of its head only.  So the time
// axis is split: one workgroup per (b, h, 64 consecutive d) with SEQ_WAVES
// waves, wave w owning the time segment [w*SL, (w+1)*SL) (SL = ceil(S/16)).
//  * Gates, 64 steps at a time with lane = step: m_t = max(m_{t-1} + logsig f_t, i_t)
//    is the scan of the max-plus maps m -> max(m + a, b), a = logsig f_t,
//    b = i_t, composed as (a, b) o (a', b') = (a + a', max(b + a', b')).  The
//    map of a span carries the sums of logsig f over sub-spans only, so m has
//    the rounding of the step-by-step recurrence (exact where i_t resets it).
//  * Pass 0: each wave composes the map of its segment; the incoming m of
//    segment w is m0 pushed through the maps of segments 0 .. w-1 (LDS).
//  * Pass 1: each wave forms c at its segment's end from c = 0 (per lane) as
//    a weighted sum of tanh z_t (one multiply-add per element and step), and
//    the scans give the segment's F = prod fg and n from 0 (uniform), to LDS.
//  * Pass 2: each wave composes its start state c = F c + c_seg over the
//    earlier segments and reruns its segment from it, writing h; the wave of
//    the last step writes the final states.  Without an initial n, n is the
//    same for every d of a head and h = c * og / (|n| + eps) takes one
//    multiply per element (the scale is formed per step in the gate phase).
// z is read twice: for a 16-bit z pass 1 keeps the first 64 steps of every
// segment in LDS (128 KB for 16 waves) and pass 2 reads them from there; the
// rest of the second read often hits the Infinity Cache.  Every step of both
// passes keeps z loads SEQ_PF steps ahead.
constexpr int SEQ_WAVES = 16;
constexpr int SEQ_PF = 16;
// 16-bit z of the first 64 steps of every segment is kept in LDS by pass 1
// and read from there by pass 2 (a quarter of the second z read at cfg4)
constexpr int SEQ_ZC = 64;
template <typename TZ> constexpr size_t seq_zc_bytes() { return sizeof(TZ) == 2 ? (size_t)SEQ_WAVES * SEQ_ZC * 64 * 2 : 0; }
template <typename TZ> __device__ __forceinline__ TZ zc_get(uint16_t v) {
  if constexpr (sizeof(TZ) == 2) return __builtin_bit_cast(TZ, v);
  else return TZ{};
}
template <typename TZ> __device__ __forceinline__ uint16_t zc_put(TZ v) {
  if constexpr (sizeof(TZ) == 2) return __builtin_bit_cast(uint16_t, v);
  else return 0;
}
constexpr float SEQ_LOG2E = 1.4426950408889634f;

// inclusive scan of the affine maps x -> F x + N (n from 0 and prod fg)
__device__ __forceinline__ void affine_scan(float& F, float& N) {
  const int idf = __float_as_int(1.f), idn = __float_as_int(0.f);
#define XL_AF_STEP(CTRL, ROWMASK)                                                                                 \
  {                                                                                                               \
    const float fe = __int_as_float(__builtin_amdgcn_update_dpp(idf, __float_as_int(F), CTRL, ROWMASK, 0xf, false)); \
    const float ne = __int_as_float(__builtin_amdgcn_update_dpp(idn, __float_as_int(N), CTRL, ROWMASK, 0xf, false)); \
    N = fmaf(ne, F, N);                                                                                           \
    F = fe * F;                                                                                                   \
  }
  XL_AF_STEP(0x111, 0xf)
  XL_AF_STEP(0x112, 0xf)
  XL_AF_STEP(0x114, 0xf)
  XL_AF_STEP(0x118, 0xf)
  XL_AF_STEP(0x142, 0xa)
  XL_AF_STEP(0x143, 0xc)
#undef XL_AF_STEP
}

// float -> T with one v_cvt_pk (round to nearest even, NaN kept) for the 16-bit types
template <typename T> __device__ __forceinline__ T from_f32_fast(float x) { return from_f32<T>(x); }
template <> __device__ __forceinline__ bf16_t from_f32_fast<bf16_t>(float x) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  const b2 r = __builtin_convertvector(f2{x, 0.f}, b2);
  return __builtin_bit_cast(bf16_t, r[0]);
}

__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(x * SEQ_LOG2E); }
__device__ __forceinline__ float logsig_f(float x) {
  return fminf(x, 0.f) - 0.6931471805599453f * __builtin_amdgcn_logf(1.0f + exp_f(-fabsf(x)));
}
// tanh(x) = sign(x) (1 - 2 / (1 + e^{2|x|})): absolute error ~1e-7, no branch
__device__ __forceinline__ float tanh_seq(float x) {
  const float e = __builtin_amdgcn_exp2f(fabsf(x) * (2.0f * SEQ_LOG2E));
  return copysignf(fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f), x);
}

// Gates of the 64 steps c0 + lane (< t1) given m at step c0 - 1; returns the
// per-lane fg, ig, og, the max-plus map of the chunk in lane 63 and m at its
// last valid step.
template <typename TG>
__device__ __forceinline__ void seq_gates(const TG* __restrict__ ip, const TG* __restrict__ fp,
                                          const TG* __restrict__ op, int64_t gbase, int gstride, int c0, int t1,
                                          int lane, float mprev, float& fg, float& ig, float& og, float& ma,
                                          float& mb, float& mlast) {
  const int t = c0 + lane;
  const bool ok = t < t1;
  const int64_t gi = gbase + (int64_t)(ok ? t : c0) * gstride;
  const float iv = to_f32(ip[gi]), fv = to_f32(fp[gi]), ov = to_f32(op[gi]);
  const float lsf = ok ? logsig_f(fv) : 0.f;
  float a = lsf, b = ok ? iv : -INFINITY;
  maxplus_scan(a, b);
  const float mt = fmaxf(mprev + a, b);                    // m_t
  float mp = __shfl_up(mt, 1, 64);                         // m_{t-1}
  if (lane == 0) mp = mprev;
  fg = exp_f(mp + lsf - mt);
  ig = exp_f(iv - mt);
  og = __builtin_amdgcn_rcpf(1.0f + exp_f(-ov));
  ma = a;
  mb = b;
  mlast = lane_of(mt, 63);  // invalid lanes repeat the last valid m
}

// Raw buffer access: wave-uniform resource and scalar byte offset, per-lane
// byte offset (the step address costs no vector instruction).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t seq_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// CP: cache policy bits of the access.  z keeps the default policy (the
// second pass re-reads it, often from the Infinity Cache; nontemporal z loads
// measured slower whenever z is cached), h is stored nontemporal (written once).
constexpr int SEQ_NT = 2;
template <typename T, int CP> __device__ __forceinline__ T buf_ld(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, CP));
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, CP));
  }
}
template <int CP, typename T> __device__ __forceinline__ void buf_st(T x, __amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), r, voff, soff, CP);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, x), r, voff, soff, CP);
  }
}

// Per-wave gate rows of the current 64-step chunk in LDS, read with one
// broadcast load per step (no v_readlane): {fg, ig, og or the h scale, w}.
struct SeqGateRow {
  float fg, ig, hs, w;
};

// UN (uniform n): no initial n, so n_t = fg_t n_{t-1} + ig_t is the same for
// every d of a head; it is formed per step in the gate phase (lane = step)
// together with the h scale og_t / (|n_t| + eps), and h = c * scale.
template <typename TZ, typename TG, typename TH, bool UN>
__global__ __launch_bounds__(64 * SEQ_WAVES) void slstm_seq_kernel(
    const TZ* __restrict__ z, const TG* __restrict__ ip, const TG* __restrict__ fp, const TG* __restrict__ op,
    const float* __restrict__ c0, const float* __restrict__ n0, const float* __restrict__ m0, TH* __restrict__ h,
    float* __restrict__ c_last, float* __restrict__ n_last, float* __restrict__ m_last, int S, int NH, int H,
    int ndb, float eps) {
  __shared__ float s_map[SEQ_WAVES][2];        // max-plus map of each segment
  __shared__ float s_aff[SEQ_WAVES][2];        // F, n-from-0 of each segment
  __shared__ float s_cseg[SEQ_WAVES][64];      // c from 0 at each segment's end, per lane
  __shared__ SeqGateRow s_gate[SEQ_WAVES][64]; // gate rows of the wave's current chunk
  extern __shared__ uint16_t s_zc[];            // [SEQ_WAVES][SEQ_ZC][64] raw 16-bit z (dynamic; 16-bit z only)
  constexpr bool ZC = sizeof(TZ) == 2;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;  // w: wave-uniform
  const int bh = blockIdx.x / ndb, db = blockIdx.x - bh * ndb;
  const int b = bh / NH, hh = bh - b * NH;
  const int d = 64 * db + lane;
  const bool dok = d < H;
  // lane byte offsets within the d block (lanes past H read lane 0's element)
  const uint32_t zlb = (dok ? lane : 0) * (uint32_t)sizeof(TZ), hlb = lane * (uint32_t)sizeof(TH);
  const int SL = (S + SEQ_WAVES - 1) / SEQ_WAVES;
  const int t0 = min(S, w * SL), t1 = min(S, t0 + SL);
  const int64_t gbase = (int64_t)b * S * NH + hh;  // gates[b, t, hh] = gbase + t * NH
  const int64_t zrow = (int64_t)NH * H;            // z[b, t, hh, d] = z + zblk + t * zrow + lane
  const int64_t zblk = (int64_t)b * S * zrow + (int64_t)hh * H + 64 * db;  // wave-uniform
  const int zrowb = (int)zrow * (int)sizeof(TZ), hrowb = (int)zrow * (int)sizeof(TH);  // bytes per step
  const float m_init = m0 ? m0[bh] : 0.f;
  SeqGateRow* gr = s_gate[w];

  // ---- pass 0: the max-plus map of this segment
  float sa = 0.f, sb = -INFINITY;
  for (int c = t0; c < t1; c += 64) {
    float fg, ig, og, ma, mb, ml;
    seq_gates(ip, fp, op, gbase, NH, c, t1, lane, 0.f, fg, ig, og, ma, mb, ml);
    const float ca = lane_of(ma, 63), cb = lane_of(mb, 63);
    sb = fmaxf(sb + ca, cb);
    sa += ca;
  }
  if (lane == 0) {
    s_map[w][0] = sa;
    s_map[w][1] = sb;
  }
  __syncthreads();
  float m_in = m_init;  // m at step t0 - 1
  for (int q = 0; q < w; ++q) m_in = fmaxf(m_in + s_map[q][0], s_map[q][1]);

  // One segment with the gates of its steps.  PASS 1: c at the segment end
  // from c = 0, as the weighted sum sum_t w_t tanh z_t per chunk (w_t = ig_t
  // prod_{s>t} fg_s, formed in the gate phase), and the segment's affine map of
  // n.  PASS 2: the recurrence from the true start state, writing h.  Step
  // indices are wave-uniform, so a step's z and h addresses are a scalar
  // base plus the lane offset.
  const bool dfull = 64 * (db + 1) <= H;  // uniform: every lane of the block is a real d
  auto run = [&](auto pass_tag, float& c, float& n) {
    constexpr int PASS = decltype(pass_tag)::value;
    float mprev = m_in, Fs = 1.f, Ns = 0.f;
    float nu = n;  // UN, pass 2: the uniform n
    TZ zq[SEQ_PF];  // raw prefetched z (converted when used, so the load is not waited for early)
    const int tlast = max(t1 - 1, 0);
    // z of step t relative to the chunk starting at step cb (byte offsets < 2^31: checked at launch)
    auto zat = [&](__amdgpu_buffer_rsrc_t r, int cb, int t) { return buf_ld<TZ, 0>(r, zlb, (t - cb) * zrowb); };
    // the segment's first chunk is kept in LDS (pass 1 writes, pass 2 reads) when it is a whole chunk
    const bool zc_seg = ZC && t0 + SEQ_ZC <= t1;
    uint16_t* zcw = s_zc + (size_t)w * SEQ_ZC * 64 + lane;
    {
      const int tp = (PASS == 2 && zc_seg) ? t0 + SEQ_ZC : t0;  // pass 2 prefetches past the kept steps
      const auto zr = seq_rsrc(z + zblk + (int64_t)tp * zrow);
#pragma unroll
      for (int j = 0; j < SEQ_PF; ++j) zq[j] = zat(zr, tp, min(tp + j, tlast));
    }
    for (int cst = t0; cst < t1; cst += 64) {
      float fg, ig, og, ma, mb, ml;
      seq_gates(ip, fp, op, gbase, NH, cst, t1, lane, mprev, fg, ig, og, ma, mb, ml);
      mprev = ml;
      const bool ok = cst + lane < t1;
      const float fgv = ok ? fg : 1.f, igv = ok ? ig : 0.f;
      float Fc = 1.f;  // PASS 1: prod fg over the chunk
      if (PASS == 1) {
        // suffix products prod_{s>=t} fg_s: inclusive scan of the lane-reversed fg
        float y = __shfl(fgv, 63 - lane, 64), yn = 0.f;
        affine_scan(y, yn);
        Fc = lane_of(y, 63);
        const float pin = __shfl(y, 63 - lane, 64);
        float pex = __shfl_down(pin, 1, 64);
        if (lane == 63) pex = 1.f;
        gr[lane].w = igv * pex;
        float F = fgv, N = igv;
        affine_scan(F, N);
        const float cF = lane_of(F, 63), cN = lane_of(N, 63);
        Ns = fmaf(Ns, cF, cN);
        Fs *= cF;
      } else {
        float hs = og;
        if (UN) {
          float F = fgv, N = igv;
          affine_scan(F, N);
          const float nt = fmaf(F, nu, N);  // n at step cst + lane
          hs = og * __builtin_amdgcn_rcpf(fabsf(nt) + eps);
          nu = lane_of(nt, 63);  // invalid lanes keep the last valid n
        }
        gr[lane] = SeqGateRow{fg, ig, hs, 0.f};
      }
      __builtin_amdgcn_wave_barrier();
      const auto zr = seq_rsrc(z + zblk + (int64_t)cst * zrow);
      const auto hr = seq_rsrc(h + zblk + (int64_t)cst * zrow);
      float acc = 0.f;  // PASS 1: sum_t w_t tanh z_t over the chunk
      auto step = [&](int j, float zt, auto store_tag) {
        const float tz = tanh_seq(zt);
        if (PASS == 1) {
          acc = fmaf(gr[j].w, tz, acc);
        } else {
          const SeqGateRow gj = gr[j];
          c = fmaf(gj.fg, c, gj.ig * tz);
          float hv;
          if (UN) {
            hv = c * gj.hs;
          } else {
            n = fmaf(gj.fg, n, gj.ig);
            hv = gj.hs * c * __builtin_amdgcn_rcpf(fabsf(n) + eps);
          }
          if (decltype(store_tag)::value || dok) buf_st<SEQ_NT>(from_f32_fast<TH>(hv), hr, hlb, j * hrowb);
        }
      };
      if (PASS == 2 && zc_seg && cst == t0) {  // kept in LDS by pass 1 (the ring holds the next chunk)
        auto chunk = [&](auto store_tag) {
#pragma unroll
          for (int j = 0; j < 64; ++j) {
            if (j % 8 == 0) __builtin_amdgcn_sched_barrier(0);  // LDS reads at most 8 steps ahead (registers)
            step(j, to_f32(zc_get<TZ>(zcw[64 * j])), store_tag);
          }
        };
        if (dfull) chunk(std::true_type{});
        else chunk(std::false_type{});
      } else if (cst + 64 <= t1) {
        auto chunk = [&](auto store_tag, auto keep_tag) {
#pragma unroll
          for (int j = 0; j < 64; ++j) {
            const TZ zraw = zq[j % SEQ_PF];
            if (decltype(keep_tag)::value) zcw[64 * j] = zc_put(zraw);
            zq[j % SEQ_PF] = zat(zr, cst, min(cst + j + SEQ_PF, tlast));
            step(j, to_f32(zraw), store_tag);
          }
        };
        if (PASS == 1 && zc_seg && cst == t0) chunk(std::true_type{}, std::true_type{});  // pass 1: no h stores
        else if (dfull) chunk(std::true_type{}, std::false_type{});
        else chunk(std::false_type{}, std::false_type{});
      } else {  // partial chunk at the segment end: no prefetch
        for (int j = 0; j < t1 - cst; ++j) step(j, to_f32(zat(zr, cst, cst + j)), std::false_type{});
      }
      if (PASS == 1) c = fmaf(Fc, c, acc);
      __builtin_amdgcn_wave_barrier();
    }
    if (PASS == 1) {
      n = Ns;
      if (lane == 0) {
        s_aff[w][0] = Fs;
        s_aff[w][1] = Ns;
      }
    }
    if (PASS == 2 && UN) n = nu;
    return mprev;
  };

  // ---- pass 1: this segment from c = 0
  float c = 0.f, n = 0.f;
  run(std::integral_constant<int, 1>{}, c, n);
  s_cseg[w][lane] = c;
  __syncthreads();
  // ---- start state of this segment, then pass 2
  c = (c0 && dok) ? c0[(int64_t)bh * H + d] : 0.f;
  n = (n0 && dok) ? n0[(int64_t)bh * H + d] : 0.f;
  for (int q = 0; q < w; ++q) {
    const float F = s_aff[q][0];
    c = fmaf(F, c, s_cseg[q][lane]);
    n = fmaf(F, n, s_aff[q][1]);
  }
  const float m_end = run(std::integral_constant<int, 2>{}, c, n);
  if (c_last && t0 < t1 && t1 == S && dok) {  // the wave of the last step
    c_last[(int64_t)bh * H + d] = c;
    n_last[(int64_t)bh * H + d] = n;
    if (d == 0) m_last[bh] = m_end;
  }
}

template <typename TZ, typename TG, typename TH>
static int launch_step3(const void* z, const void* i, const void* f, const void* o, const float* c, const float* n,
                        const float* m, void* h, float* c1, float* n1, float* m1, int64_t total, int H, float eps,
                        hipStream_t s) {
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipLaunchKernelGGL((slstm_step_kernel<TZ, TG, TH>), dim3(blocks), dim3(256), 0, s, (const TZ*)z, (const TG*)i,
                     (const TG*)f, (const TG*)o, c, n, m, (TH*)h, c1, n1, m1, total, H, eps);
  return check_launch("xl_slstm_step_fwd");
}

template <typename TZ, typename TG, typename TH>
static int launch_seq3(const void* z, const void* i, const void* f, const void* o, const float* c, const float* n,
                       const float* m, void* h, float* c1, float* n1, float* m1, int S, int NH, int H,
                       int64_t total, float eps, hipStream_t s) {
  const int ndb = (H + 63) / 64;  // 64-element d blocks per head
  const int64_t blocks = total / H * ndb;
  auto kern = n ? slstm_seq_kernel<TZ, TG, TH, false> : slstm_seq_kernel<TZ, TG, TH, true>;
  const size_t zc = seq_zc_bytes<TZ>();
  if (zc) {
    const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)zc);
    if (e != hipSuccess)
      return set_error(XL_ERR_LAUNCH, "xl_slstm_seq_fwd: LDS attribute failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * SEQ_WAVES), zc, s, (const TZ*)z, (const TG*)i,
                     (const TG*)f, (const TG*)o, c, n, m, (TH*)h, c1, n1, m1, S, NH, H, ndb, eps);
  return check_launch("xl_slstm_seq_fwd");
}

// Dispatches a functor template over the three dtypes of z, gates and h.
template <template <typename, typename, typename> class Fn, typename... A>
static int dispatch3(int dz, int dg, int dh, A... args) {
#define XL_D3(TZ, TG)                                                      \
  switch (dh) {                                                            \
    case XL_DTYPE_F32: return Fn<TZ, TG, float>::run(args...);            \
    case XL_DTYPE_BF16: return Fn<TZ, TG, bf16_t>::run(args...);          \
    default: return Fn<TZ, TG, f16_t>::run(args...);                      \
  }
#define XL_D2(TZ)                                                          \
  switch (dg) {                                                            \
    case XL_DTYPE_F32: { XL_D3(TZ, float) }                               \
    case XL_DTYPE_BF16: { XL_D3(TZ, bf16_t) }                             \
    default: { XL_D3(TZ, f16_t) }                                         \
  }
  switch (dz) {
    case XL_DTYPE_F32: { XL_D2(float) }
    case XL_DTYPE_BF16: { XL_D2(bf16_t) }
    default: { XL_D2(f16_t) }
  }
#undef XL_D2
#undef XL_D3
}

template <typename TZ, typename TG, typename TH>
struct StepFn {
  template <typename... A>
  static int run(A... a) { return launch_step3<TZ, TG, TH>(a...); }
};
template <typename TZ, typename TG, typename TH>
struct SeqFn {
  template <typename... A>
  static int run(A... a) { return launch_seq3<TZ, TG, TH>(a...); }
};

}  // namespace xl

extern "C" int xl_slstm_step_fwd(const void* z, const void* i, const void* f, const void* o, const float* c,
                                 const float* n, const float* m, void* h, float* c_new, float* n_new, float* m_new,
                                 int B, int NH, int H, float eps, int dtype_z, int dtype_gates, int dtype_h,
                                 void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_slstm_step_fwd";
  if (B <= 0 || NH <= 0 || H <= 0)
    return set_error(XL_ERR_INVALID_ARG, "%s: dimensions must be positive (B=%d NH=%d H=%d)", who, B, NH, H);
  if (!dtype_ok(dtype_z) || !dtype_ok(dtype_gates) || !dtype_ok(dtype_h))
    return set_error(XL_ERR_INVALID_ARG, "%s: unknown dtype", who);
  if (!z || !i || !f || !o || !c || !n || !m || !h || !c_new || !n_new || !m_new)
    return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if (m_new == m) return set_error(XL_ERR_INVALID_ARG, "%s: m_new must not alias m", who);
  const int64_t total = (int64_t)B * NH * H;
  if ((total + 255) / 256 > 0x7fffffffLL) return set_error(XL_ERR_INVALID_ARG, "%s: too large", who);
  return dispatch3<StepFn>(dtype_z, dtype_gates, dtype_h, z, i, f, o, c, n, m, h, c_new, n_new, m_new, total, H, eps,
                           (hipStream_t)stream);
}

extern "C" int xl_slstm_seq_fwd(const void* z, const void* i, const void* f, const void* o, const float* c0,
                                const float* n0, const float* m0, void* h, float* c_last, float* n_last,
                                float* m_last, int B, int S, int NH, int H, float eps, int dtype_z, int dtype_gates,
                                int dtype_h, void* stream) {
  using namespace xl;
  clear_error();
  const char* who = "xl_slstm_seq_fwd";
  if (B <= 0 || S <= 0 || NH <= 0 || H <= 0)
    return set_error(XL_ERR_INVALID_ARG, "%s: dimensions must be positive (B=%d S=%d NH=%d H=%d)", who, B, S, NH, H);
  if (!dtype_ok(dtype_z) || !dtype_ok(dtype_gates) || !dtype_ok(dtype_h))
    return set_error(XL_ERR_INVALID_ARG, "%s: unknown dtype", who);
  if (!z || !i || !f || !o || !h) return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!((c0 && n0 && m0) || (!c0 && !n0 && !m0)))
    return set_error(XL_ERR_INVALID_ARG, "%s: initial states must be given together", who);
  if (!((c_last && n_last && m_last) || (!c_last && !n_last && !m_last)))
    return set_error(XL_ERR_INVALID_ARG, "%s: last states must be requested together", who);
  if (m_last && m_last == m0) return set_error(XL_ERR_INVALID_ARG, "%s: m_last must not alias m0", who);
  const int64_t total = (int64_t)B * NH * H;
  if ((total + 255) / 256 > 0x7fffffffLL) return set_error(XL_ERR_INVALID_ARG, "%s: too large", who);
  // the kernel addresses z and h within a 64-step chunk (plus its prefetch) with 32-bit offsets
  if ((int64_t)(64 + SEQ_PF) * NH * H * 4 > 0x7fffffffLL)
    return set_error(XL_ERR_INVALID_ARG, "%s: NH * H = %lld too large", who, (long long)NH * H);
  return dispatch3<SeqFn>(dtype_z, dtype_gates, dtype_h, z, i, f, o, c0, n0, m0, h, c_last, n_last, m_last, S, NH,
                          H, total, eps, (hipStream_t)stream);
}
