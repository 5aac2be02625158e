"""Chunkwise mLSTM forward with the reference's signatures, on HIP.

Drop-in for ``mlstm_chunkwise`` (kernel_development/xlstm/mlstm_block/
mlstm_chunkwise/vendored/torch/native/fw.py:372-412) and the registry form
``mlstm_chunkwise__native_autograd`` (.../native/fwbw.py:192-229).

Differences from the reference, by design: the states are always float32
(the reference keeps them in ``matK.dtype``, fw.py:65), and the op is
forward-only (no autograd formula is registered; calling backward raises).

``chunk_size`` keeps the reference's contract (S must be a multiple of it,
fw.py:303-305).  The forward is chunk-size invariant, so with bf16 q/k/v and
S a multiple of 64 the fused kernel runs every chunk size on 64-token chunks;
results then differ from the reference's at that chunk size by rounding only.
``algo="two_pass"`` runs the chunk size as given.
"""

from __future__ import annotations

import torch

from . import _lib
from .ops import mlstm_chunkwise_op

__all__ = ["mlstm_chunkwise", "mlstm_chunkwise__native_autograd"]


def mlstm_chunkwise(matQ, matK, matV, vecI, vecF, matC_initial=None, vecN_initial=None, scaM_initial=None,
                    qk_scale=None, return_last_states=False, chunk_size=64, eps=1e-6, algo="auto"):
    """h (B, NH, S, DHV), or (h, (C (B,NH,DHQK,DHV), n (B,NH,DHQK), m (B,NH,1))) when
    ``return_last_states``.  ``algo``: "auto" | "fused" | "two_pass"."""
    if qk_scale is None:
        qk_scale = matQ.shape[-1] ** -0.5
    h, C, n, m = mlstm_chunkwise_op(matQ, matK, matV, vecI, vecF, matC_initial, vecN_initial, scaM_initial,
                                    float(qk_scale), int(chunk_size), float(eps), bool(return_last_states),
                                    _lib.ALGO[algo])
    if return_last_states:
        return h, (C, n, m)
    return h


def mlstm_chunkwise__native_autograd(q, k, v, i, f, c_initial=None, n_initial=None, m_initial=None,
                                     return_last_states=False, eps=1e-6, chunk_size=64, **kwargs):
    """Registry form (fwbw.py:192-229); extra kwargs such as ``autocast_kernel_dtype`` are accepted."""
    return mlstm_chunkwise(q, k, v, i, f, c_initial, n_initial, m_initial, qk_scale=None,
                           return_last_states=return_last_states, chunk_size=chunk_size, eps=eps,
                           algo=kwargs.get("algo", "auto"))
