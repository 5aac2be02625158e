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
// waves, and time runs in blocks of SEQ_WAVES * WS steps (WS = 64 steps per
// wave, fewer when S is short), wave w owning steps [w WS, (w + 1) WS) of
// every block.  Per block:
//  * Gates, lane = step: m_t = max(m_{t-1} + logsig f_t, i_t) is the scan of
//    the max-plus maps m -> max(m + a, b), a = logsig f_t, b = i_t, composed
//    as (a, b) o (a', b') = (a + a', max(b + a', b')).  The map of a span
//    carries the sums of logsig f over sub-spans only, so m has the rounding
//    of the step-by-step recurrence (exact where i_t resets it).  The maps of
//    the block's segments meet in LDS: each wave composes the ones before its
//    own (its incoming m) and all of them (the next block's incoming m).
//  * Pass 1: each wave evaluates tanh z_t over its segment once, keeps the
//    WS values in registers, and forms c at the segment's end from c = 0 as
//    the weighted sum sum_t w_t tanh z_t (one multiply-add per element and
//    step; the weights ig_t prod_{s>t} fg_s come from the gate scans); the
//    segment's F = prod fg and n from 0 go to LDS.
//  * Pass 2: each wave composes its start state c = F c + c_seg over the
//    earlier segments of the block (and every wave the block's end state, the
//    next block's start) and reruns c = fg c + ig tanh z from the kept values,
//    writing h.
// So z crosses HBM once (nontemporal loads: nothing reads it again) and tanh
// is evaluated once per element.  z is requested SEQ_PF steps ahead, into the
// registers that will hold its tanh (the next block's first steps into those
// pass 2 has consumed), and the gates one block ahead; a segment cut short by
// the end of the sequence reads its z directly, twice.  Without an initial n,
// n is the same for every d of a head and h = c * og / (|n| + eps) takes one
// multiply per element (the scale is formed per step in the gate phase).
constexpr int SEQ_WAVES = 12;  // 3 waves per SIMD: up to 168 registers, 64 of them the kept tanh z
constexpr int SEQ_WS = 64;     // steps per wave and block (lane = step in the gate phase)
constexpr int SEQ_PF = 16;
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
// tanh(x) = 1 - 2 / (1 + e^{2x}) on either sign (e^{2x} -> 0 gives -1, -> inf gives 1): absolute
// error below 2e-7 over every bf16 input, no branch, no sign fix-up
__device__ __forceinline__ float tanh_seq(float x) {
  const float e = __builtin_amdgcn_exp2f(x * (2.0f * SEQ_LOG2E));
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f);
}

// Raw buffer access: wave-uniform resource and scalar byte offset, per-lane
// byte offset (the step address costs no vector instruction).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t seq_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// CP: cache policy bits of the access; z and h are streamed (each crosses HBM
// once), so both use the nontemporal policy.
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
// raw z bits parked in a float register until converted (16-bit z zero-extended)
template <typename TZ> __device__ __forceinline__ float z_park(TZ v) {
  if constexpr (sizeof(TZ) == 4) return __builtin_bit_cast(float, v);
  else return __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(uint16_t, v));
}
template <typename TZ> __device__ __forceinline__ TZ z_unpark(float v) {
  if constexpr (sizeof(TZ) == 4) return __builtin_bit_cast(TZ, v);
  else return __builtin_bit_cast(TZ, (uint16_t)__builtin_bit_cast(uint32_t, v));
}

// Per-wave gate rows of the current segment in LDS, read with one broadcast
// load per step (no v_readlane): {fg, ig, og or the h scale, w}.
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
    int ndb, int WS, float eps) {
  // [block & 1]: a block's maps are published one block early, its segment states read while the
  // faster waves write the next block's
  __shared__ float s_map[2][SEQ_WAVES][2];     // max-plus map of each segment of the block
  __shared__ float s_aff[2][SEQ_WAVES][2];     // F, n-from-0 of each segment
  __shared__ float s_cseg[2][SEQ_WAVES][64];   // c from 0 at each segment's end, per lane
  __shared__ SeqGateRow s_gate[SEQ_WAVES][64]; // gate rows of the wave's segment
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;  // w: wave-uniform
  const int bh = blockIdx.x / ndb, db = blockIdx.x - bh * ndb;
  const int b = bh / NH, hh = bh - b * NH;
  const int d = 64 * db + lane;
  const bool dok = d < H;
  const bool dfull = 64 * (db + 1) <= H;  // uniform: every lane of the block is a real d
  // lane byte offsets within the d block (lanes past H read lane 0's element)
  const uint32_t zlb = (dok ? lane : 0) * (uint32_t)sizeof(TZ), hlb = lane * (uint32_t)sizeof(TH);
  const int TB = SEQ_WAVES * WS;                   // steps per block
  const int64_t gbase = (int64_t)b * S * NH + hh;  // gates[b, t, hh] = gbase + t * NH
  const int64_t zrow = (int64_t)NH * H;            // z[b, t, hh, d] = z + zblk + t * zrow + lane
  const int64_t zblk = (int64_t)b * S * zrow + (int64_t)hh * H + 64 * db;  // wave-uniform
  const int zrowb = (int)zrow * (int)sizeof(TZ), hrowb = (int)zrow * (int)sizeof(TH);  // bytes per step
  SeqGateRow* gr = s_gate[w];

  // state entering the block (identical in every wave): c, n per lane (n uniform when UN), m
  float c_blk = (c0 && dok) ? c0[(int64_t)bh * H + d] : 0.f;
  float n_blk = (n0 && dok) ? n0[(int64_t)bh * H + d] : 0.f;
  float m_blk = m0 ? m0[bh] : 0.f;

  // gates of a wave's segment starting at step ts (< te): lane = step, clamped loads
  auto load_gates = [&](int ts, int te, float& iv, float& fv, float& ov) {
    const int t = min(ts + lane, max(te - 1, 0));
    const int64_t gi = gbase + (int64_t)t * NH;
    iv = to_f32(ip[gi]);
    fv = to_f32(fp[gi]);
    ov = to_f32(op[gi]);
  };
  // tz: the raw z of a whole segment's next steps, then its tanh z (pass 1 converts in place,
  // SEQ_PF steps requested ahead; pass 2 reads the values and requests the next segment's first
  // SEQ_PF steps into the registers it has consumed)
  float tz[SEQ_WS];
  auto request_first = [&](int ts) {  // the first SEQ_PF steps of a whole segment starting at ts
    const auto zr = seq_rsrc(z + zblk + (int64_t)ts * zrow);
#pragma unroll
    for (int j = 0; j < SEQ_PF; ++j) tz[j] = z_park<TZ>(buf_ld<TZ, SEQ_NT>(zr, zlb, j * zrowb));
  };
  int t0 = min(S, w * WS), t1 = min(S, t0 + WS);
  // gate scans of a segment (lane = step): the segment's logsig f, i, o, its prefix max-plus maps
  // (a, bb), and its map published in s_map[par][w]
  struct GScan {
    float lsf, iv, ov, a, bb;
  };
  auto gate_scan = [&](int ts, int te, float iv_, float fv_, float ov_, int par) {
    const bool okg = lane < te - ts;
    GScan gsc;
    gsc.lsf = okg ? logsig_f(fv_) : 0.f;
    gsc.iv = iv_;
    gsc.ov = ov_;
    gsc.a = gsc.lsf;
    gsc.bb = okg ? iv_ : -INFINITY;
    maxplus_scan(gsc.a, gsc.bb);
    if (lane == 63) {
      s_map[par][w][0] = gsc.a;
      s_map[par][w][1] = gsc.bb;
    }
    return gsc;
  };
  float iv, fv, ov;
  load_gates(t0, t1, iv, fv, ov);
  if (t1 - t0 == SEQ_WS) request_first(t0);
  GScan gs = gate_scan(t0, t1, iv, fv, ov, 0);
  {
    const int t0n = min(S, t0 + TB), t1n = min(S, t0n + WS);
    if (t0n < t1n) load_gates(t0n, t1n, iv, fv, ov);  // the next block's gates
  }
  __syncthreads();  // the first block's maps

  for (int blk = 0, par = 0; blk < S; blk += TB, par ^= 1) {
    const int nst = t1 - t0;  // steps of this wave's segment (0 .. WS)
    const bool ok = lane < nst;
    // the next block's segment of this wave
    const int t0n = min(S, t0 + TB), t1n = min(S, t0n + WS);
    const float lsf = gs.lsf, ivc = gs.iv, ovc = gs.ov, a = gs.a, bb = gs.bb;
    float m_in = m_blk;  // m at step t0 - 1
    for (int q = 0; q < w; ++q) m_in = fmaxf(m_in + s_map[par][q][0], s_map[par][q][1]);
    {
      float mb = m_blk;
      for (int q = 0; q < SEQ_WAVES; ++q) mb = fmaxf(mb + s_map[par][q][0], s_map[par][q][1]);
      m_blk = mb;  // m entering the next block
    }
    const float mt = fmaxf(m_in + a, bb);  // m_t (invalid lanes repeat the last valid m)
    float mp = __shfl_up(mt, 1, 64);       // m_{t-1}
    if (lane == 0) mp = m_in;
    const float fgv = ok ? exp_f(mp + lsf - mt) : 1.f;
    const float igv = ok ? exp_f(ivc - mt) : 0.f;
    const float og = __builtin_amdgcn_rcpf(1.0f + exp_f(-ovc));
    const float m_seg = lane_of(mt, 63);
    // pass-1 weights w_t = ig_t prod_{s>t} fg_s: suffix products as a scan of the lane-reversed fg
    float y = __shfl(fgv, 63 - lane, 64), yn = 0.f;
    affine_scan(y, yn);
    const float Fc = lane_of(y, 63);
    const float pin = __shfl(y, 63 - lane, 64);
    float pex = __shfl_down(pin, 1, 64);
    if (lane == 63) pex = 1.f;
    gr[lane].w = igv * pex;
    float F = fgv, N = igv;  // the affine maps of n: prefix scan (n from 0 at every step)
    affine_scan(F, N);
    const float cN = lane_of(N, 63);
    __builtin_amdgcn_wave_barrier();

    // ---- pass 1: tanh z of the segment into registers, c at its end from c = 0
    float acc = 0.f;
    if (nst == SEQ_WS) {
      const auto zr = seq_rsrc(z + zblk + (int64_t)t0 * zrow);
#pragma unroll
      for (int j = 0; j < SEQ_WS; ++j) {
        if (j % 8 == 0) __builtin_amdgcn_sched_barrier(0);  // weights read from LDS at most 8 steps ahead
        if (j + SEQ_PF < SEQ_WS) tz[j + SEQ_PF] = z_park<TZ>(buf_ld<TZ, SEQ_NT>(zr, zlb, (j + SEQ_PF) * zrowb));
        tz[j] = tanh_seq(to_f32(z_unpark<TZ>(tz[j])));
        acc = fmaf(gr[j].w, tz[j], acc);
      }
    } else if (nst > 0) {  // short or partial segment: no prefetch, z read again by pass 2
      const auto zr = seq_rsrc(z + zblk + (int64_t)t0 * zrow);
      for (int j = 0; j < nst; ++j) acc = fmaf(gr[j].w, tanh_seq(to_f32(buf_ld<TZ, 0>(zr, zlb, j * zrowb))), acc);
      if (t1n - t0n == SEQ_WS) request_first(t0n);
    }
    s_cseg[par][w][lane] = acc;
    if (lane == 0) {
      s_aff[par][w][0] = Fc;
      s_aff[par][w][1] = cN;
    }
    // the next block's gate scans and map (its gates arrived during this block), and the gates of
    // the block after it
    {
      const int t0nn = min(S, t0n + TB), t1nn = min(S, t0nn + WS);
      gs = gate_scan(t0n, t1n, iv, fv, ov, par ^ 1);
      if (t0nn < t1nn) load_gates(t0nn, t1nn, iv, fv, ov);
    }
    __syncthreads();  // every segment's c, F and n from 0; the next block's maps
    // ---- the segment's start state, and the block's end state (the next block's start)
    float c = c_blk, n = n_blk;
    for (int q = 0; q < w; ++q) {
      const float Fq = s_aff[par][q][0];
      c = fmaf(Fq, c, s_cseg[par][q][lane]);
      n = fmaf(Fq, n, s_aff[par][q][1]);
    }
    {
      float ce = c, ne = n;
      for (int q = w; q < SEQ_WAVES; ++q) {
        const float Fq = s_aff[par][q][0];
        ce = fmaf(Fq, ce, s_cseg[par][q][lane]);
        ne = fmaf(Fq, ne, s_aff[par][q][1]);
      }
      c_blk = ce;
      n_blk = ne;
    }
    // ---- pass 2: the segment from its start state and the kept tanh z, h out
    float hs = og;
    if (UN) {
      const float nt = fmaf(F, n, N);  // n at step t0 + lane (uniform over d)
      hs = og * __builtin_amdgcn_rcpf(fabsf(nt) + eps);
      n = lane_of(nt, 63);  // invalid lanes keep the last valid n
    }
    gr[lane] = SeqGateRow{fgv, igv, hs, 0.f};
    __builtin_amdgcn_wave_barrier();
    const auto hr = seq_rsrc(h + zblk + (int64_t)t0 * zrow);
    auto step = [&](int j, float tzj, auto store_tag) {
      const SeqGateRow gj = gr[j];
      c = fmaf(gj.fg, c, gj.ig * tzj);
      float hv;
      if (UN) {
        hv = c * gj.hs;
      } else {
        n = fmaf(gj.fg, n, gj.ig);
        hv = gj.hs * c * __builtin_amdgcn_rcpf(fabsf(n) + eps);
      }
      if (decltype(store_tag)::value || dok) buf_st<SEQ_NT>(from_f32_fast<TH>(hv), hr, hlb, j * hrowb);
    };
    if (nst == SEQ_WS) {
      // the next block's segment, when whole, has its first steps requested as registers free up
      const bool nfull = t1n - t0n == SEQ_WS;
      const auto zn = seq_rsrc(z + zblk + (int64_t)(nfull ? t0n : t0) * zrow);
      auto seg = [&](auto store_tag) {
#pragma unroll
        for (int j = 0; j < SEQ_WS; ++j) {
          if (j % 8 == 0) __builtin_amdgcn_sched_barrier(0);  // LDS reads at most 8 steps ahead (registers)
          step(j, tz[j], store_tag);
          if (j < SEQ_PF && nfull) tz[j] = z_park<TZ>(buf_ld<TZ, SEQ_NT>(zn, zlb, j * zrowb));
        }
      };
      if (dfull) seg(std::true_type{});
      else seg(std::false_type{});
    } else {
      const auto zr = seq_rsrc(z + zblk + (int64_t)t0 * zrow);
      for (int j = 0; j < nst; ++j) step(j, tanh_seq(to_f32(buf_ld<TZ, 0>(zr, zlb, j * zrowb))), std::false_type{});
    }
    if (c_last && nst > 0 && t1 == S && dok) {  // the wave of the last step
      c_last[(int64_t)bh * H + d] = c;
      n_last[(int64_t)bh * H + d] = n;
      if (d == 0) m_last[bh] = m_seg;
    }
    __builtin_amdgcn_wave_barrier();
    t0 = t0n;
    t1 = t1n;
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
  // steps per wave and block: the register-held maximum, fewer for a short sequence (one block)
  const int WS = min(SEQ_WS, (S + SEQ_WAVES - 1) / SEQ_WAVES);
  auto kern = n ? slstm_seq_kernel<TZ, TG, TH, false> : slstm_seq_kernel<TZ, TG, TH, true>;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * SEQ_WAVES), 0, s, (const TZ*)z, (const TG*)i,
                     (const TG*)f, (const TG*)o, c, n, m, (TH*)h, c1, n1, m1, S, NH, H, ndb, WS, eps);
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
