// C-ABI entry point of the chunkwise mLSTM forward: validation and the choice
// between the single-pass MFMA kernels (the pipelined schedule by default, for bf16
// or f16 q/k/v; the fused schedule, bf16 only, on request) and the two-pass kernels.
#include "chunkwise.h"

namespace xl {

static bool valid_L(int L) { return L == 16 || L == 32 || L == 64 || L == 128; }
// the single-pass algorithms (fused and pipelined schedules) take any S (ragged last chunk)
static bool single_pass(int algo) { return algo == XL_CHUNKWISE_FUSED || algo == XL_CHUNKWISE_PIPELINED; }

int chunkwise_check_args(const ChunkwiseArgs& a, int algo) {
  const char* who = "xl_mlstm_chunkwise_fwd";
  if (a.B <= 0 || a.NH <= 0 || a.S <= 0 || a.DQK <= 0 || a.DV <= 0)
    return set_error(XL_ERR_INVALID_ARG, "%s: dimensions must be positive (B=%d NH=%d S=%d DQK=%d DV=%d)", who, a.B,
                     a.NH, a.S, a.DQK, a.DV);
  if (!valid_L(a.L)) return set_error(XL_ERR_UNSUPPORTED, "%s: chunk_size=%d not in {16,32,64,128}", who, a.L);
  // the reference's contract; the fused algorithm, asked for explicitly, runs 64-token
  // chunks with a ragged last chunk and accepts any S
  if (a.S % a.L != 0 && !single_pass(algo))
    return set_error(XL_ERR_INVALID_ARG, "%s: Sequence length %d is not divisible by chunk size %d.", who, a.S, a.L);
  if (!dtype_ok(a.dtype_qkv) || !dtype_ok(a.dtype_gates)) return set_error(XL_ERR_INVALID_ARG, "%s: unknown dtype", who);
  if (algo < XL_CHUNKWISE_AUTO || algo > XL_CHUNKWISE_PIPELINED)
    return set_error(XL_ERR_INVALID_ARG, "%s: unknown algo %d", who, algo);
  if (!a.q || !a.k || !a.v || !a.i || !a.f || !a.h) return set_error(XL_ERR_INVALID_ARG, "%s: null pointer", who);
  // q, k, v, h and the float32 states move in 16-byte pieces
  if ((((uintptr_t)a.q) | ((uintptr_t)a.k) | ((uintptr_t)a.v) | ((uintptr_t)a.h) | ((uintptr_t)a.c0) |
       ((uintptr_t)a.n0) | ((uintptr_t)a.c_last) | ((uintptr_t)a.n_last)) & 15u)
    return set_error(XL_ERR_INVALID_ARG, "%s: q, k, v, h, c0, n0, c_last and n_last must be 16-byte aligned", who);
  if (!((a.c0 && a.n0 && a.m0) || (!a.c0 && !a.n0 && !a.m0)))
    return set_error(XL_ERR_INVALID_ARG, "%s: initial states must be given together", who);
  if (!((a.c_last && a.n_last && a.m_last) || (!a.c_last && !a.n_last && !a.m_last)))
    return set_error(XL_ERR_INVALID_ARG, "%s: last states must be requested together", who);
  if (a.c_last && (a.c_last == a.c0 || a.n_last == a.n0 || a.m_last == a.m0))
    return set_error(XL_ERR_INVALID_ARG, "%s: last states must not alias the initial states", who);
  const long long BNH = (long long)a.B * a.NH;
  if (BNH * ((a.S + a.L - 1) / a.L) * ((a.DV + 63) / 64) > 0x7fffffffLL)
    return set_error(XL_ERR_INVALID_ARG, "%s: too large", who);
  return XL_OK;
}

static int pick(const ChunkwiseArgs& a, int algo, int* chosen) {
  const char* why = nullptr;
  const bool pipe_ok = chunkwise_fused_supported(a, &why, algo != XL_CHUNKWISE_FUSED);
  if (single_pass(algo) && !pipe_ok)
    return set_error(XL_ERR_UNSUPPORTED, "xl_mlstm_chunkwise_fwd: %s algorithm unsupported here: %s",
                     algo == XL_CHUNKWISE_FUSED ? "fused" : "pipelined", why);
  *chosen = (algo == XL_CHUNKWISE_TWO_PASS) ? XL_CHUNKWISE_TWO_PASS
            : single_pass(algo)             ? algo
            : pipe_ok                       ? XL_CHUNKWISE_PIPELINED
                                            : XL_CHUNKWISE_TWO_PASS;
  return XL_OK;
}

}  // namespace xl

extern "C" size_t xl_mlstm_chunkwise_workspace_size(int B, int NH, int S, int DQK, int DV, int L, int dtype_qkv,
                                                    int algo) {
  using namespace xl;
  if (B <= 0 || NH <= 0 || S <= 0 || DQK <= 0 || DV <= 0 || !valid_L(L)) return 0;
  if (S % L && !single_pass(algo)) return 0;
  ChunkwiseArgs a = {};
  a.B = B; a.NH = NH; a.S = S; a.DQK = DQK; a.DV = DV; a.L = L;
  a.dtype_qkv = dtype_qkv; a.dtype_gates = dtype_qkv;
  int chosen = XL_CHUNKWISE_TWO_PASS;
  if (pick(a, algo, &chosen) != XL_OK) return 0;
  return single_pass(chosen) ? chunkwise_fused_workspace(B, NH, S, DQK, DV, kChunkwiseMaxSegments)
                                     : chunkwise_two_pass_workspace(B, NH, S, DQK, DV, L);
}

extern "C" int xl_mlstm_chunkwise_algo(int B, int NH, int S, int DQK, int DV, int L, int dtype_qkv, int algo) {
  using namespace xl;
  clear_error();
  if (B <= 0 || NH <= 0 || S <= 0 || DQK <= 0 || DV <= 0)
    return set_error(XL_ERR_INVALID_ARG, "xl_mlstm_chunkwise_algo: dimensions must be positive");
  if (!valid_L(L)) return set_error(XL_ERR_UNSUPPORTED, "xl_mlstm_chunkwise_algo: chunk_size=%d not in {16,32,64,128}", L);
  if (!dtype_ok(dtype_qkv)) return set_error(XL_ERR_INVALID_ARG, "xl_mlstm_chunkwise_algo: unknown dtype");
  if (algo < XL_CHUNKWISE_AUTO || algo > XL_CHUNKWISE_PIPELINED)
    return set_error(XL_ERR_INVALID_ARG, "xl_mlstm_chunkwise_algo: unknown algo %d", algo);
  if (S % L && !single_pass(algo))
    return set_error(XL_ERR_INVALID_ARG, "xl_mlstm_chunkwise_algo: Sequence length %d is not divisible by chunk size %d.",
                     S, L);
  ChunkwiseArgs a = {};
  a.B = B; a.NH = NH; a.S = S; a.DQK = DQK; a.DV = DV; a.L = L;
  a.dtype_qkv = dtype_qkv; a.dtype_gates = dtype_qkv;
  int chosen = XL_CHUNKWISE_TWO_PASS;
  const int rc = pick(a, algo, &chosen);
  if (rc) return rc;
  const char* why = nullptr;
  if (chosen == XL_CHUNKWISE_TWO_PASS && algo == XL_CHUNKWISE_AUTO && !chunkwise_fused_supported(a, &why, true))
    set_error(XL_OK, "fused algorithm not taken: %s", why);  // informational: why auto fell back
  return chosen;
}

extern "C" int xl_mlstm_chunkwise_fwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                                      const float* c0, const float* n0, const float* m0, void* h, float* c_last,
                                      float* n_last, float* m_last, int B, int NH, int S, int DQK, int DV, int L,
                                      float qk_scale, float eps, int dtype_qkv, int dtype_gates, int algo,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  using namespace xl;
  clear_error();
  ChunkwiseArgs a = {q, k, v, i, f, c0, n0, m0, h, c_last, n_last, m_last, B, NH, S, DQK, DV, L,
                     qk_scale, eps, dtype_qkv, dtype_gates, workspace, workspace_bytes, stream,
                     kChunkwiseMaxSegments};
  int rc = chunkwise_check_args(a, algo);
  if (rc) return rc;
  int chosen = XL_CHUNKWISE_TWO_PASS;
  rc = pick(a, algo, &chosen);
  if (rc) return rc;
  const bool fused = single_pass(chosen);
  a.pipelined = chosen == XL_CHUNKWISE_PIPELINED;
  const size_t need = fused ? chunkwise_fused_workspace(B, NH, S, DQK, DV, kChunkwiseMaxSegments)
                            : chunkwise_two_pass_workspace(B, NH, S, DQK, DV, L);
  if (!workspace || workspace_bytes < need)
    return set_error(XL_ERR_WORKSPACE, "xl_mlstm_chunkwise_fwd: %s workspace needs %zu bytes, got %zu",
                     fused ? "fused" : "two-pass", need, workspace ? workspace_bytes : (size_t)0);
  if (((uintptr_t)workspace) & 255u)
    return set_error(XL_ERR_INVALID_ARG, "xl_mlstm_chunkwise_fwd: workspace must be 256-byte aligned");
  return fused ? chunkwise_fused(a) : chunkwise_two_pass(a);
}
