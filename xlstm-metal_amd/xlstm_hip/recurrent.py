"""Recurrent mLSTM (decode step and sequence loop) with the reference's signatures, on HIP.

Drop-in for ``mlstm_recurrent_step__native`` / ``mlstm_recurrent_step__native_fw``
(kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent/native_step.py:
8-133) and ``mlstm_recurrent_sequence__native_fw`` (.../native_sequence.py:
131-170).  States are float32 (``dtype_state`` other than float32 raises).
"""

from __future__ import annotations

import torch

from .ops import mlstm_sequence_op, mlstm_step_inplace_op, mlstm_step_op

__all__ = ["mlstm_recurrent_step__native", "mlstm_recurrent_step__native_fw", "mlstm_recurrent_step_",
           "mlstm_recurrent_sequence__native_fw"]


def _state_dtype(dtype_state):
    if dtype_state != torch.float32:
        raise NotImplementedError(f"xlstm_hip keeps mLSTM states in float32 (dtype_state={dtype_state})")


def mlstm_recurrent_step__native_fw(matC_old, vecN_old, scaM_old, vecQ, vecK, vecV, scaI, scaF, eps=1e-6,
                                    dtype_state=torch.float32, **kwargs):
    """(h (B,NH,DHV), (C (B,NH,DHQK,DHV), n (B,NH,DHQK), m (B,NH,1)))  (native_step.py:8-102)."""
    _state_dtype(dtype_state)
    h, C, n, m = mlstm_step_op(vecQ, vecK, vecV, scaI, scaF, matC_old, vecN_old, scaM_old, float(eps),
                               vecQ.shape[-1] ** -0.5)
    return h, (C, n, m)


def mlstm_recurrent_step__native(q, k, v, i, f, c, n, m, eps=1e-6, dtype_state=torch.float32, **kwargs):
    """Keyword form used by the arbitrary-length wrapper (native_step.py:105-133)."""
    return mlstm_recurrent_step__native_fw(c, n, m, q, k, v, i, f, eps=eps, dtype_state=dtype_state)


def mlstm_recurrent_step_(q, k, v, i, f, c, n, m, eps=1e-6):
    """Serving variant: updates the float32 C state in place; returns (h, (c, n', m'))."""
    h, n2, m2 = mlstm_step_inplace_op(q, k, v, i, f, c, n, m, float(eps), q.shape[-1] ** -0.5)
    return h, (c, n2, m2)


def mlstm_recurrent_sequence__native_fw(q, k, v, i, f, c_initial=None, n_initial=None, m_initial=None,
                                        return_last_states=False, eps=1e-6, dtype_state=torch.float32, **kwargs):
    """Whole time loop in one launch (native_sequence.py:131-170)."""
    _state_dtype(dtype_state)
    h, C, n, m = mlstm_sequence_op(q, k, v, i, f, c_initial, n_initial, m_initial, q.shape[-1] ** -0.5,
                                   float(eps), bool(return_last_states))
    if return_last_states:
        return h, (C, n, m)
    return h
