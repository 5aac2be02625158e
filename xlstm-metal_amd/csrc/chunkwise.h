// Internal interface between the chunkwise C-ABI entry point and its kernels.
#pragma once

#include "common.h"

namespace xl {

struct ChunkwiseArgs {
  const void *q, *k, *v, *i, *f;
  const float *c0, *n0, *m0;
  void* h;
  float *c_last, *n_last, *m_last;
  int B, NH, S, DQK, DV, L;
  float qk_scale, eps;
  int dtype_qkv, dtype_gates;
  void* workspace;
  size_t workspace_bytes;
  void* stream;
  int max_segments;  // fused algorithm: at most this many sequence segments (1: no split)
  int pipelined;     // fused algorithm: the pipelined schedule (chunkwise_pipe.hip)
};

// Per-chunk gate prefix: sb[t] = sum_{u<=t} logsig(f_u) in sequential order
// (torch's CPU cumsum order), si[t] = i_t, for the L tokens from g0.  Called by
// every thread of the block; needs 2 barriers.
template <typename TG, int L>
__device__ __forceinline__ void chunk_gate_prefix(const TG* __restrict__ ig, const TG* __restrict__ fg, size_t g0,
                                                  float* sb, float* si) {
  const int tid = threadIdx.x;
  if (tid < L) {
    sb[tid] = logsigmoid(to_f32(fg[g0 + tid]));
    si[tid] = to_f32(ig[g0 + tid]);
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int t = 0; t < L; ++t) {
      acc += sb[t];
      sb[t] = acc;
    }
  }
  __syncthreads();
}

// Argument checks of xl_mlstm_chunkwise_fwd for the given algorithm (0 or an XL_ERR_* code).
int chunkwise_check_args(const ChunkwiseArgs& a, int algo);

// Two-pass algorithm (states pass + output pass), float32 arithmetic.
size_t chunkwise_two_pass_workspace(int B, int NH, int S, int DQK, int DV, int L);
int chunkwise_two_pass(const ChunkwiseArgs& a);
// The states pass alone (S % L == 0): the state entering every chunk into Cst [BNH][NC][DQK][DV],
// nst [BNH][NC][DQK], mst [BNH][NC], the state after the last chunk into c_fin, n_fin, m_fin.
int chunkwise_states_pass(const ChunkwiseArgs& a, float* Cst, float* nst, float* mst, float* c_fin, float* n_fin,
                          float* m_fin);
// The states pass on the matrix cores (float32 / f16 q/k/v on float32 MFMA, bf16 on bf16 MFMA),
// the last states into a.c_last / n_last / m_last (each may be null); 1, launching nothing,
// where its tiles do not fit (DV % 64, DQK not in {64, 128, 256}, L not in {16, 32, 64}),
// otherwise XL_OK or a negative XL_ERR_* code.  gprep: room for the bf16 scan's gate prefix,
// kChunkGatePrefix floats per chunk of every head.
int chunkwise_states_mfma(const ChunkwiseArgs& a, float* Cst, float* nst, float* mst, float* gprep);
// floats per chunk of the bf16 chunk scans' gate prefix: b[64], a[64], the chunk's log-decay, max a,
// two spare, and (the backward's fused path, written by its stats pass over a) the dC scan's
// per-token b - m_comb in place of a and qk_scale / divisor [64]
constexpr int kChunkGatePrefix = 196;

// The single-pass algorithms.  fused_supported() says whether a shape/dtype is covered by the
// pipelined schedule (pipelined: bf16 or f16 q/k/v) or the fused one (bf16 only), and why not,
// in `why`, when it is not.
bool chunkwise_fused_supported(const ChunkwiseArgs& a, const char** why, bool pipelined);
// Workspace of the fused algorithm: the gate prep (1280 bytes per 64-token chunk of every
// head) and, when the sequence is split into segments (few heads), two sets of per-segment
// states.  max_segments 1 disables the split.
constexpr int kChunkwiseMaxSegments = 16;
size_t chunkwise_fused_workspace(int B, int NH, int S, int DQK, int DV, int max_segments);
int chunkwise_fused_segments(int B, int NH, int S, int DQK, int DV, int max_segments);
int chunkwise_fused(const ChunkwiseArgs& a);

}  // namespace xl
