/*
 * xlstm_hip.h — C-ABI of the MI355X (gfx950) mLSTM/sLSTM kernel library
 * (libxlstm_hip.so).
 *
 * Drop-in boundary for the torch-native kernel backend of MLXPorts/xLSTM-metal.
 * Each entry point replaces one reference function (paths relative to the
 * reference root, see the comment on each).  The reference has no C ABI of its
 * own for these functions: its native launchers are pybind11/Objective-C++
 * (e.g. xlstm_metal/torch_native/blocks/mlstm/mlstm_chunkwise/forward/
 * mlstm_chunkwise_recurrent_fw_C_extension.mm:62-149, soft_cap_extension.mm:
 * 60-95).  This ABI is plain C: pointers, sizes, scalars.
 *
 * Conventions
 *  - Tensors are dense, row-major, contiguous, in the reference's layouts
 *    ([B, NH, S, D] etc.).  Device pointers.
 *  - Every buffer is owned by the caller.  No entry point allocates device
 *    memory; scratch comes in through `workspace` (size from the matching
 *    *_workspace_size call).
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *    the call returns without synchronising.  Entry points are re-entrant and
 *    keep no state between calls.
 *  - Return 0 on success, a negative XL_ERR_* code on failure; the message is
 *    then available from xl_last_error() on the calling thread.
 *  - States (C, n, m) are always float32.  q/k/v/z and gates may be float32,
 *    bfloat16 or float16 (XL_DTYPE_*); arithmetic is float32, MFMA operands
 *    of the single-pass chunkwise kernels are q/k/v's 16-bit type (float32
 *    operands as hi + lo pairs of it).
 */
#ifndef XLSTM_HIP_H
#define XLSTM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XL_ABI_VERSION 2

enum xl_dtype { XL_DTYPE_F32 = 0, XL_DTYPE_BF16 = 1, XL_DTYPE_F16 = 2 };

enum xl_status {
  XL_OK = 0,
  XL_ERR_INVALID_ARG = -1,   /* bad shape, null pointer, aliasing, bad dtype */
  XL_ERR_UNSUPPORTED = -2,   /* valid request this build does not implement */
  XL_ERR_WORKSPACE = -3,     /* workspace missing or too small */
  XL_ERR_LAUNCH = -4         /* the HIP runtime rejected a launch */
};

/* Chunkwise algorithm selector for xl_mlstm_chunkwise_fwd. */
enum xl_chunkwise_algo {
  XL_CHUNKWISE_AUTO = 0,     /* pipelined when supported, else two-pass */
  XL_CHUNKWISE_TWO_PASS = 1, /* states kernel + output kernel, float32 math */
  XL_CHUNKWISE_FUSED = 2,    /* single pass, bf16 MFMA, states in registers (bf16 q/k/v only) */
  XL_CHUNKWISE_PIPELINED = 3 /* XL_CHUNKWISE_FUSED's math and shapes, bf16 or f16 q/k/v; each
                                chunk's state update overlaps the previous outputs (two-phase
                                schedule) */
};

/* ABI version of the loaded library (XL_ABI_VERSION at build time). */
int xl_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* xl_last_error(void);

/*
 * y = cap * tanh(x / cap), elementwise over numel elements; cap <= 0 copies x.
 * Replaces soft_cap(x, cap) (xlstm_metal/torch_native/blocks/soft_cap/
 * softcap_metal.py:29-31 -> soft_cap_extension.mm:60-95 -> soft_cap_kernel.
 * metal:4-15) and SoftCapCell.forward (softcap.py:25-31).  x and y have the
 * same dtype; y may alias x.
 */
int xl_soft_cap_fwd(const void* x, void* y, int64_t numel, float cap, int dtype, void* stream);

/*
 * One recurrent mLSTM decode step.  Replaces mlstm_recurrent_step__native
 * (kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent/
 * native_step.py:8-133).
 *   q, k [B,NH,DQK], v [B,NH,DV] (dtype_qkv); i, f [B,NH] (dtype_gates);
 *   c_old [B,NH,DQK,DV], n_old [B,NH,DQK], m_old [B,NH] float32;
 *   h [B,NH,DV] (dtype_qkv); c_new, n_new, m_new float32, same shapes.
 * c_new may equal c_old (in-place update).  n_new / m_new must not alias
 * n_old / m_old.  The reference's dtype roundings for a bfloat16/float16 q
 * (q*scale, k v^T, C' and n' cast to q's dtype for the h products, the
 * products rounded to q's dtype) are reproduced.
 */
int xl_mlstm_step_fwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                      const float* c_old, const float* n_old, const float* m_old,
                      void* h, float* c_new, float* n_new, float* m_new,
                      int B, int NH, int DQK, int DV, float qk_scale, float eps,
                      int dtype_qkv, int dtype_gates, void* stream);

/*
 * Measurement aid, no counterpart in the reference: the HBM ceiling of
 * xl_mlstm_step_fwd's state stream.  Copies c_old [B,NH,DQK,DV] float32 to
 * c_new (may be the same pointer; both 16-byte aligned) with the decode step's
 * grid, block, thread-to-element map, 16-byte nontemporal loads and stores and
 * its read-then-write order, and nothing else, so its time is what the step's
 * access pattern alone costs.
 */
int xl_mlstm_step_copy_ceiling(const float* c_old, float* c_new, int B, int NH, int DQK, int DV, void* stream);

/*
 * Chunkwise mLSTM forward.  Replaces mlstm_chunkwise / mlstm_chunkwise_fw
 * (kernel_development/xlstm/mlstm_block/mlstm_chunkwise/vendored/torch/
 * native/fw.py:257-412) and its registry form mlstm_chunkwise__native_autograd
 * (.../native/fwbw.py:192-229).
 *   q, k [B,NH,S,DQK], v [B,NH,S,DV] (dtype_qkv); i, f [B,NH,S] (dtype_gates);
 *   c0 [B,NH,DQK,DV], n0 [B,NH,DQK], m0 [B,NH] float32, all three NULL for
 *   zero initial states (or all three non-NULL);
 *   h [B,NH,S,DV] (dtype_qkv); c_last, n_last, m_last float32 (all NULL when
 *   the last states are not wanted).
 * S % L == 0 (fw.py:303-305).  L in {16, 32, 64, 128}.  With algo =
 * XL_CHUNKWISE_FUSED (bf16 q/k/v, DQK 128 or 256) or XL_CHUNKWISE_PIPELINED (bf16 or f16 q/k/v,
 * DQK 32, 64, 96, 128, 192 or 256), and DV % 64 == 0, any S >= 1 is accepted: the kernel runs 64-token chunks and a ragged last chunk
 * (the forward is chunk-size invariant, so L only names the reference's
 * chunking there).
 * workspace: xl_mlstm_chunkwise_workspace_size(...) bytes, 256-byte aligned
 * (fused algorithm: the per-chunk gate prep, 1280 bytes per 64 tokens of
 * every head; two-pass algorithm: the chunk-entry states and the states
 * pass's gate prefix, 784 bytes per chunk).  q, k, v, h, c0,
 * n0, c_last and n_last 16-byte aligned (XL_ERR_INVALID_ARG otherwise).
 */
size_t xl_mlstm_chunkwise_workspace_size(int B, int NH, int S, int DQK, int DV, int L,
                                         int dtype_qkv, int algo);
/*
 * The algorithm xl_mlstm_chunkwise_fwd takes for these arguments:
 * XL_CHUNKWISE_TWO_PASS, XL_CHUNKWISE_FUSED or XL_CHUNKWISE_PIPELINED, or a negative XL_ERR_* code for
 * arguments it rejects.  When algo = XL_CHUNKWISE_AUTO falls back to the
 * two-pass algorithm, xl_last_error() says why the fused one was not taken.
 * (The reference has no algorithm choice: its torch-native chunkwise is one
 * code path, VTN fw.py:257-369.)
 */
int xl_mlstm_chunkwise_algo(int B, int NH, int S, int DQK, int DV, int L, int dtype_qkv, int algo);
int xl_mlstm_chunkwise_fwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                           const float* c0, const float* n0, const float* m0,
                           void* h, float* c_last, float* n_last, float* m_last,
                           int B, int NH, int S, int DQK, int DV, int L, float qk_scale, float eps,
                           int dtype_qkv, int dtype_gates, int algo,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * Chunkwise mLSTM forward that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc).  Same arguments and results as xl_mlstm_chunkwise_fwd
 * with algo = XL_CHUNKWISE_FUSED (bf16 q/k/v, DQK 128 or 256, DV % 64 == 0,
 * any S >= 1); the fused algorithm's gate-prep scratch lives in a static
 * device array of XL_NOALLOC_SCRATCH_BYTES per GPU (1280 bytes per 64 tokens
 * of every head: B*NH*ceil(S/64) <= 13107), held until the process ends.
 * Larger requests return XL_ERR_UNSUPPORTED.  The stream's device must be the
 * current device.  Every call on a GPU shares that GPU's array; outside graph
 * capture the calls are ordered (a call on another stream than the previous
 * call's waits on an event recorded behind it; the first call on a device
 * creates that event).  A stream under capture gets no such wait: a replay of
 * a captured call that overlaps another call on the same GPU races.
 */
#define XL_NOALLOC_SCRATCH_BYTES (16u * 1024u * 1024u)
size_t xl_mlstm_chunkwise_noalloc_max_bytes(void);
int xl_mlstm_chunkwise_fwd_noalloc(const void* q, const void* k, const void* v, const void* i, const void* f,
                                   const float* c0, const float* n0, const float* m0,
                                   void* h, float* c_last, float* n_last, float* m_last,
                                   int B, int NH, int S, int DQK, int DV, int L, float qk_scale, float eps,
                                   int dtype_qkv, int dtype_gates, void* stream);

/*
 * Recurrent mLSTM over a whole sequence in one launch (the time loop runs on
 * the GPU, states stay on chip).  Replaces mlstm_recurrent_sequence__native_fw
 * (kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent/
 * native_sequence.py:18-170), used by the arbitrary-length wrapper for tails
 * (kernel_development/xlstm/mlstm_block/mslstm_parallel/torch/
 * kernel_wrappers.py:151-170).  Shapes as for xl_mlstm_chunkwise_fwd with any
 * S >= 1; same dtype semantics as xl_mlstm_step_fwd.
 */
int xl_mlstm_sequence_fwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                          const float* c0, const float* n0, const float* m0,
                          void* h, float* c_last, float* n_last, float* m_last,
                          int B, int NH, int S, int DQK, int DV, float qk_scale, float eps,
                          int dtype_qkv, int dtype_gates, void* stream);

/*
 * One sLSTM step.  Replaces slstm_step_pytorch (xlstm_metal/torch_native/
 * blocks/slstm/slstm_layers/stepwise/slstm_metal_kernel.py:14-65) and
 * sLSTMStepwiseKernelCell.forward (.../stepwise/slstm_stepwise_kernel_cell.
 * py:47-97).
 *   z [B,NH,H] (dtype_z); i, f, o [B,NH] (dtype_gates);
 *   c, n [B,NH,H], m [B,NH] float32; h [B,NH,H] (dtype_h);
 *   c_new, n_new [B,NH,H], m_new [B,NH] float32 (c_new/n_new may alias c/n,
 *   m_new must not alias m).
 */
int xl_slstm_step_fwd(const void* z, const void* i, const void* f, const void* o,
                      const float* c, const float* n, const float* m,
                      void* h, float* c_new, float* n_new, float* m_new,
                      int B, int NH, int H, float eps, int dtype_z, int dtype_gates, int dtype_h,
                      void* stream);

/*
 * sLSTM over a sequence in one launch: the per-timestep loop of
 * sLSTMNeuron.forward (xlstm_metal/torch_native/blocks/slstm/slstm_layers/
 * slstm_neuron.py:132-143) with states in registers.
 *   z [B,S,NH,H] (dtype_z); i, f, o [B,S,NH] (dtype_gates);
 *   c0, n0 [B,NH,H], m0 [B,NH] float32 or all NULL (zero state);
 *   h [B,S,NH,H] (dtype_h); c_last, n_last, m_last float32 or all NULL.
 */
int xl_slstm_seq_fwd(const void* z, const void* i, const void* f, const void* o,
                     const float* c0, const float* n0, const float* m0,
                     void* h, float* c_last, float* n_last, float* m_last,
                     int B, int S, int NH, int H, float eps, int dtype_z, int dtype_gates, int dtype_h,
                     void* stream);

/*
 * Depthwise causal conv1d over time, channels last, with an optional SiLU.
 * Replaces CausalConv1d.forward with groups == channels (xlstm_metal/
 * torch_native/blocks/slstm/slstm_layers/causal_conv1d/causal_conv1d.py:51-67:
 * left pad of K - 1 zeros, then nn.Conv1d) and, with act = 1, the nn.SiLU after
 * it in sLSTMProjectionCell.forward (.../slstm_layers/slstm_projection_cell.py:
 * 110-115), on the [B, S, D] input that cell permutes to [B, D, S].
 *   x, y [B,S,D]; weight [D,K] (nn.Conv1d's [D,1,K]); bias [D] or NULL; all of
 *   one dtype.  y[b,s,c] = act(bias[c] + sum_j weight[c,j] x[b, s-K+1+j, c]),
 *   x = 0 before s = 0 (weight[c, K-1] multiplies the current step).  With a
 *   16-bit dtype the convolution is rounded to that dtype before the SiLU, as
 *   the two reference modules do.  1 <= K <= 8; act 0 = none, 1 = SiLU; y must
 *   not overlap x.
 */
int xl_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, void* y,
                         int B, int S, int D, int K, int act, int dtype, void* stream);

/*
 * GroupNorm of rows of G groups of CG channels: each group normalised by its
 * own mean and biased variance, y = (x - mean) / sqrt(var + eps) * weight[c]
 * + bias[c].  Replaces nn.GroupNorm(num_groups=NH, num_channels=NH*H) in
 * sLSTMOutputCell.forward (xlstm_metal/torch_native/blocks/slstm/slstm_layers/
 * slstm_output_cell.py:72-83), applied to the kernel output h [B,S,NH,H]
 * viewed as [B*S, NH*H].
 *   x, y [N, G*CG]; weight, bias [G*CG], each optional (NULL: 1 / 0); all of
 *   one dtype; y may alias x.  With the weight alone it is also the
 *   MultiHeadLayerNorm of xlstm_metal/torch_native/blocks/mlstm/multihead_norm/
 *   multihead_norm.py:27-40 on x [B,S,NH,DH] viewed as [B*S, NH*DH].
 */
int xl_group_norm_fwd(const void* x, const void* weight, const void* bias, void* y,
                      int64_t N, int G, int CG, float eps, int dtype, void* stream);

/*
 * The mLSTM output cell's stage before its output projection, fused: per-head
 * RMS normalisation of the kernel output h, the per-channel weight and the
 * output gate sigma(o).  Replaces MultiHeadRMSNorm.forward (xlstm_metal/
 * torch_native/blocks/mlstm/multihead_norm/multihead_norm.py:56-64) and the
 * permute, sigmoid and product around it in mLSTMOutputCell.forward
 * (.../mlstm/mlstm_chunkwise/mlstm_output_cell.py:84-93).
 *   h: [B,NH,S,DH] (h_layout 1, the chunkwise output) or [B,S,NH,DH]
 *   (h_layout 0); weight [NH*DH] or NULL; o_preact [B,S,NH*DH] (the gate
 *   projection before the sigmoid) or NULL (no gate: the norm alone);
 *   y [B,S,NH*DH]; all of one dtype.
 *   y = (h / sqrt(mean_DH(h^2) + eps)) * weight * sigmoid(o), with the
 *   reference's roundings to a 16-bit dtype after the division, the weight
 *   product and the sigmoid.  DH <= 8192 (16-bit) or 4096 (float32) when DH is
 *   a multiple of 16 bytes, else DH <= 1024; y must not overlap h or o_preact.
 */
int xl_mh_rmsnorm_gate_fwd(const void* h, const void* weight, const void* o_preact, void* y,
                           int B, int NH, int S, int DH, int h_layout, float eps, int dtype,
                           void* stream);

/*
 * Gate projection with the soft-cap epilogue: y[m, n] = cap * tanh(z / cap),
 * z = (b[n] + sum_d x[m, d] w[n, d]) rounded to the dtype (the Linear's output),
 * for the gate pre-activations of the projection cells.  cap_rounding 0: the
 * soft-cap in float32, rounded once (SoftCapCell, which the mLSTM projection
 * cell uses); 1: cap, z / cap, tanh and the product each rounded to the dtype,
 * as torch evaluates cap * tanh(x / cap) on 16-bit tensors in
 * sLSTMProjectionCell.soft_cap (xlstm_metal/torch_native/blocks/slstm/
 * slstm_layers/slstm_projection_cell.py:84-89).  Replaces
 * soft_cap(igate_proj(x)), soft_cap(fgate_proj(x)) in mLSTMProjectionCell.
 * forward (xlstm_metal/torch_native/blocks/mlstm/mlstm_chunkwise/
 * mlstm_projection_cell.py:97-103) and the i, f (on the conv output) and o
 * gates of sLSTMProjectionCell.forward (.../slstm/slstm_layers/
 * slstm_projection_cell.py:118-121), with the gates' weights stacked.
 *   x [M, D], w [G, D] (nn.Linear's weight), bias [G] or NULL, y [M, G]; bf16
 *   or f16 (float32: XL_ERR_UNSUPPORTED); G <= 64; D a multiple of 8; x and
 *   w 16-byte aligned; cap <= 0: no soft-cap.
 */
int xl_gate_proj_softcap_fwd(const void* x, const void* weight, const void* bias, void* y,
                             int M, int D, int G, float cap, int cap_rounding, int dtype, void* stream);

/*
 * Chunkwise mLSTM backward: the reference's custom backward mlstm_chunkwise_bw
 * (kernel_development/xlstm/mlstm_block/mlstm_chunkwise/vendored/torch/native/
 * bw.py:198-352, wrapped by _mlstm_chunkwise_fwbw.backward, fwbw.py:102-173 and
 * mlstm_chunkwise__native_custbw, fwbw.py:232-281), float32 accumulation (bf16
 * inputs: bf16 matrix-core products, float32 operands as bf16 hi + lo pairs).  The
 * states are recomputed from the inputs (recompute_states_in_bw) and the
 * per-token denominator max(|q n|, exp(-m)) + eps is treated as a constant, as
 * there.  Inputs as for xl_mlstm_chunkwise_fwd plus dh [B,NH,S,DV] (dtype_qkv)
 * and dc_last [B,NH,DQK,DV] float32 or NULL (the gradient of the last C state).
 * Outputs: dq, dk [B,NH,S,DQK], dv [B,NH,S,DV] in dtype_qkv; di, df [B,NH,S] in
 * dtype_gates; dc0 [B,NH,DQK,DV] float32 or NULL (only with initial states; the
 * gradients of n0 and m0 are zero in the reference).  S % L == 0, L in
 * {16, 32, 64} (the Python autograd runs chunk_size 128 and ragged sequences
 * at 64: the custom backward does not depend on the chunk size).  Workspace:
 * xl_mlstm_chunkwise_bwd_workspace_size bytes, 256-byte aligned (every chunk's
 * state and its gradient in float32, and every chunk's gate prefix).  q, k, v, dh, dq, dk, dv, c0, n0,
 * dc_last and dc0 16-byte aligned (XL_ERR_INVALID_ARG otherwise).
 */
size_t xl_mlstm_chunkwise_bwd_workspace_size(int B, int NH, int S, int DQK, int DV, int L);
int xl_mlstm_chunkwise_bwd(const void* q, const void* k, const void* v, const void* i, const void* f,
                           const float* c0, const float* n0, const float* m0, const void* dh,
                           const float* dc_last, void* dq, void* dk, void* dv, void* di, void* df,
                           float* dc0, int B, int NH, int S, int DQK, int DV, int L, float qk_scale,
                           float eps, int dtype_qkv, int dtype_gates, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Logit projection with the soft-cap epilogue: y[m, v] = cap * tanh(z / cap),
 * z = (sum_d x[m, d] w[v, d]) rounded to the dtype, the soft-cap in float32 and
 * rounded once.  Replaces soft_cap(lm_head(out_norm(x)), output_logit_soft_cap)
 * for the rows a decoder needs logits of (a decode step's tokens, a prompt's
 * last positions): nn.Linear(embedding_dim, vocab_size, bias=False)
 * (xlstm_metal/torch_native/models/wired_xlstm.py:123-131,176) followed by
 * soft_cap (xlstm_metal/torch_native/generate.py:131;
 * xlstm_metal/mlx_jit/generate.py:201).  The weights are streamed from HBM once
 * for all M rows.
 *   x [M, D], w [V, D] (nn.Linear's weight), y [M, V]; bf16 or f16 (float32:
 *   XL_ERR_UNSUPPORTED); M <= 16 and M * (D + 8) * 2 <= 160 KiB (the limit of
 *   the kernel form that stages the token rows in LDS, applied to every call;
 *   logits of every position of a prompt are a GEMM: XL_ERR_UNSUPPORTED); D a
 *   multiple of 8; x and w 16-byte aligned; cap <= 0: no soft-cap.
 */
int xl_lm_head_softcap_fwd(const void* x, const void* weight, void* y, int M, int D, int V, float cap,
                           int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XLSTM_HIP_H */
