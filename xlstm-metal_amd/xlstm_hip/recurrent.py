"""Recurrent mLSTM (decode step and sequence loop) with the reference's signatures, on HIP.

Drop-in for ``mlstm_recurrent_step__native`` / ``mlstm_recurrent_step__native_fw``
(kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent/native_step.py:
8-133) and ``mlstm_recurrent_sequence__native_fw`` (.../native_sequence.py:
131-170).  States are float32 (``dtype_state`` other than float32 raises).

``mLSTMRecurrentKernelCell`` is the model-level decode caller
(xlstm_metal/torch_native/blocks/mlstm/mlstm_chunkwise/
mlstm_recurrent_kernel_cell.py:19-161): one token with a carried state runs the
decode-step kernel, longer inputs (or no state) the sequence kernel.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from .ops import mlstm_sequence_op, mlstm_step_inplace_op, mlstm_step_op

__all__ = ["mlstm_recurrent_step__native", "mlstm_recurrent_step__native_fw", "mlstm_recurrent_step_",
           "mlstm_recurrent_sequence__native_fw", "mLSTMRecurrentKernelCell"]


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


class mLSTMRecurrentKernelCell(nn.Module):
    """``mlstm_recurrent_kernel_cell.py:19-161``: q, k [B, NH, S, DHQK], v [B, NH, S, DHV], gates
    [B, NH, S], state (C, n, m [B, NH]) or None -> (h [B, NH, S, DHV], (C, n, m)).

    Inputs are cast to ``compute_dtype`` as the reference does (``:87-91``); h comes back in it.
    The kernels carry the state in float32 from step to step and cast it to ``state_dtype`` once at
    the end (the reference rounds it to ``state_dtype`` every step), and use the stable
    log-sigmoid where the reference's ``-log(1 + exp(-f))`` (``:129``) overflows (f < -88 in
    float32).
    """

    def __init__(self, num_heads: int, qk_dim_per_head: int, v_dim_per_head: int, eps: float = 1e-6,
                 compute_dtype: torch.dtype = torch.float32, state_dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.qk_dim_per_head = qk_dim_per_head
        self.v_dim_per_head = v_dim_per_head
        self.eps = eps
        self.compute_dtype = compute_dtype
        self.state_dtype = state_dtype

    def forward(self, q: Tensor, k: Tensor, v: Tensor, i_preact: Tensor, f_preact: Tensor,
                state: Optional[Tuple[Tensor, Tensor, Tensor]] = None) -> Tuple[Tensor, Tuple[Tensor, Tensor, Tensor]]:
        B, NH, S, _ = q.shape
        cd = self.compute_dtype
        q, k, v, i, f = (t.to(dtype=cd) for t in (q, k, v, i_preact, f_preact))
        if state is not None:
            C0, n0, m0 = state
            C0, n0, m0 = C0.to(torch.float32), n0.to(torch.float32), m0.to(torch.float32).reshape(B, NH, 1)
        if S == 1 and state is not None:  # one decode step: the HBM-bound step kernel
            h, (C, n, m) = mlstm_recurrent_step__native_fw(C0, n0, m0, q[:, :, 0], k[:, :, 0], v[:, :, 0],
                                                           i[:, :, :1], f[:, :, :1], eps=self.eps)
            h = h[:, :, None]
        else:
            init = (None, None, None) if state is None else (C0, n0, m0)
            h, (C, n, m) = mlstm_recurrent_sequence__native_fw(q, k, v, i, f, *init, return_last_states=True,
                                                               eps=self.eps)
        sd = self.state_dtype
        return h, (C.to(sd), n.to(sd), m.reshape(B, NH).to(sd))
