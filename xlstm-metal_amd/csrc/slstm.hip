// sLSTM step (xl_slstm_step_fwd) and sequence (xl_slstm_seq_fwd).
//
// Reference math, torch-native variant (xlstm_metal/torch_native/blocks/
// slstm/slstm_layers/stepwise/slstm_metal_kernel.py:45-63), per (b, h, d):
//   m' = max(m + logsig(f), i);  ig = exp(i - m');  fg = exp(m + logsig(f) - m')
//   c' = fg c + ig tanh(z);      n' = fg n + ig;    h = sigmoid(o) c' / (|n'| + eps)
// Gates are per (b, h) and there is no recurrent matrix, so the recurrence is
// elementwise: one thread per (b, h, d), coalesced along d.  The sequence
// kernel keeps c, n, m in registers across all S steps and prefetches the
// next step's z and gates while the current one is computed.
#include "common.h"

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

template <typename TZ, typename TG, typename TH>
__global__ __launch_bounds__(256) void slstm_seq_kernel(const TZ* __restrict__ z, const TG* __restrict__ ip,
                                                        const TG* __restrict__ fp, const TG* __restrict__ op,
                                                        const float* __restrict__ c0, const float* __restrict__ n0,
                                                        const float* __restrict__ m0, TH* __restrict__ h,
                                                        float* __restrict__ c_last, float* __restrict__ n_last,
                                                        float* __restrict__ m_last, int S, int NH, int H,
                                                        int64_t total, float eps) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // over B*NH*H
  if (idx >= total) return;
  const int64_t bh = idx / H;
  const int d = (int)(idx - bh * H);
  const int64_t b = bh / NH;
  const int hh = (int)(bh - b * NH);
  float c = c0 ? c0[idx] : 0.f;
  float n = n0 ? n0[idx] : 0.f;
  float m = m0 ? m0[bh] : 0.f;
  // z[b, t, hh, d] and gates[b, t, hh]
  const int64_t zstride = (int64_t)NH * H, gstride = NH;
  const TZ* zp = z + b * S * zstride + (int64_t)hh * H + d;
  TH* hp = h + b * S * zstride + (int64_t)hh * H + d;
  const int64_t g0 = b * S * gstride + hh;
  float zn = to_f32(zp[0]);
  float in = to_f32(ip[g0]), fn = to_f32(fp[g0]), on = to_f32(op[g0]);
  for (int t = 0; t < S; ++t) {
    const float zc = zn, ic = in, fc = fn, oc = on;
    if (t + 1 < S) {  // prefetch step t+1
      zn = to_f32(zp[(int64_t)(t + 1) * zstride]);
      const int64_t gi = g0 + (int64_t)(t + 1) * gstride;
      in = to_f32(ip[gi]);
      fn = to_f32(fp[gi]);
      on = to_f32(op[gi]);
    }
    const SGate g = slstm_gates(ic, fc, oc, m);
    c = g.fg * c + g.ig * tanh_f32(zc);
    n = g.fg * n + g.ig;
    m = g.mn;
    hp[(int64_t)t * zstride] = from_f32<TH>(g.og * c / (fabsf(n) + eps));
  }
  if (c_last) {
    c_last[idx] = c;
    n_last[idx] = n;
    if (d == 0) m_last[bh] = m;
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
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipLaunchKernelGGL((slstm_seq_kernel<TZ, TG, TH>), dim3(blocks), dim3(256), 0, s, (const TZ*)z, (const TG*)i,
                     (const TG*)f, (const TG*)o, c, n, m, (TH*)h, c1, n1, m1, S, NH, H, total, eps);
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
  return dispatch3<SeqFn>(dtype_z, dtype_gates, dtype_h, z, i, f, o, c0, n0, m0, h, c_last, n_last, m_last, S, NH,
                          H, total, eps, (hipStream_t)stream);
}
