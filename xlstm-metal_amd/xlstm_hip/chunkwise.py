"""Chunkwise mLSTM with the reference's signatures, on HIP.

Drop-in for ``mlstm_chunkwise`` (kernel_development/xlstm/mlstm_block/
mlstm_chunkwise/vendored/torch/native/fw.py:372-412) and the registry forms
``mlstm_chunkwise__native_autograd`` and ``mlstm_chunkwise__native_custbw``
(.../native/fwbw.py:192-281).

The op's backward is the reference's custom backward (bw.py:198-352, the one
``__native_custbw`` uses): the states are recomputed from the inputs, the
per-token divisor max(|q n|, exp(-m)) + eps is a constant, the gradients of the
last n and m are dropped and those of the initial n and m are zero.  For the
mLSTM layer (the multi-head norm after h removes each row's scale) it equals
autograd's gradient, which ``__native_autograd`` gets in the reference by
differentiating its forward; a loss that sees the scale of h, m0 or the
last-state path's df (see ``oracle.mlstm.mlstm_chunkwise_bw``) differs from
autograd there.  S must be a multiple of ``chunk_size`` (16, 32 or 64) for the
backward.

Differences from the reference, by design: the states are always float32
(the reference keeps them in ``matK.dtype``, fw.py:65).

``chunk_size`` keeps the reference's contract (S must be a multiple of it,
fw.py:303-305).  The forward is chunk-size invariant, so with bf16 or f16 q/k/v
and S a multiple of 64 the single-pass kernel runs every chunk size on 64-token chunks;
results then differ from the reference's at that chunk size by rounding only.
``algo="two_pass"`` runs the chunk size as given.
"""

from __future__ import annotations

import warnings

import torch

from . import _lib
from .ops import mlstm_chunkwise_op

__all__ = ["mlstm_chunkwise", "mlstm_chunkwise__native_autograd", "mlstm_chunkwise__native_custbw"]


def mlstm_chunkwise(matQ, matK, matV, vecI, vecF, matC_initial=None, vecN_initial=None, scaM_initial=None,
                    qk_scale=None, return_last_states=False, chunk_size=64, eps=1e-6, algo="auto"):
    """h (B, NH, S, DHV), or (h, (C (B,NH,DHQK,DHV), n (B,NH,DHQK), m (B,NH,1))) when
    ``return_last_states``.  ``algo``: "auto" | "fused" | "pipelined" | "two_pass"."""
    if qk_scale is None:
        qk_scale = matQ.shape[-1] ** -0.5
    h, C, n, m = mlstm_chunkwise_op(matQ, matK, matV, vecI, vecF, matC_initial, vecN_initial, scaM_initial,
                                    float(qk_scale), int(chunk_size), float(eps), bool(return_last_states),
                                    _lib.ALGO[algo])
    if return_last_states:
        return h, (C, n, m)
    return h


_autograd_warned = False


def _warn_custom_gradients(c_initial, n_initial, m_initial, return_last_states, tensors) -> None:
    """Once per process: under the __native_autograd name the gradients come from the reference's
    custom backward, which differ from exact autograd where a loss sees the last states or the
    initial n and m (see mlstm_chunkwise__native_autograd)."""
    global _autograd_warned
    if _autograd_warned or not torch.is_grad_enabled():
        return
    if not any(t is not None and t.requires_grad for t in tensors):
        return
    why = []
    if return_last_states:
        why.append("the last states are returned")
    if any(t is not None and t.requires_grad for t in (n_initial, m_initial)):
        why.append("n_initial / m_initial require grad")
    if not why:
        return
    _autograd_warned = True
    warnings.warn("mlstm_chunkwise__native_autograd: gradients come from the reference's custom backward "
                  "(bw.py:198-352), not exact autograd: " + " and ".join(why) + ", and there the last-state "
                  "path of df, and the gradients of n_initial and m_initial (zeros), differ from torch.autograd "
                  "of the forward", RuntimeWarning, stacklevel=3)


def mlstm_chunkwise__native_autograd(q, k, v, i, f, c_initial=None, n_initial=None, m_initial=None,
                                     return_last_states=False, eps=1e-6, chunk_size=64, **kwargs):
    """Registry form (fwbw.py:192-229); extra kwargs such as ``autocast_kernel_dtype`` are accepted.

    The reference's function of this name differentiates its forward with torch.autograd; here the
    gradients come from the reference's custom backward (the one mlstm_chunkwise__native_custbw
    names), which treats each token's divisor and the stabilisers as constants, gives zero
    gradients to n_initial and m_initial, and leaves a <dC_last, C_last> sigmoid(-f) term out of df
    on the last-state path.  A loss that sees h only through the mLSTM layer's multi-head norm gets
    identical gradients; otherwise a RuntimeWarning says so, once per process."""
    _warn_custom_gradients(c_initial, n_initial, m_initial, return_last_states,
                           (q, k, v, i, f, c_initial, n_initial, m_initial))
    return mlstm_chunkwise(q, k, v, i, f, c_initial, n_initial, m_initial, qk_scale=None,
                           return_last_states=return_last_states, chunk_size=chunk_size, eps=eps,
                           algo=kwargs.get("algo", "auto"))


def mlstm_chunkwise__native_custbw(q, k, v, i, f, c_initial=None, n_initial=None, m_initial=None,
                                   return_last_states=False, eps=1e-6, chunk_size=64,
                                   autocast_kernel_dtype=torch.float32, **kwargs):
    """Registry form with the custom backward (fwbw.py:232-281).  ``autocast_kernel_dtype`` casts
    q, k, v, i, f to that dtype when autocast is on, as the reference's custom_fwd does."""
    if torch.is_autocast_enabled():
        q, k, v, i, f = (t.to(autocast_kernel_dtype) for t in (q, k, v, i, f))
    h = mlstm_chunkwise(q, k, v, i, f, c_initial, n_initial, m_initial, qk_scale=None,
                        return_last_states=return_last_states, chunk_size=chunk_size, eps=eps,
                        algo=kwargs.get("algo", "auto"))
    return h
