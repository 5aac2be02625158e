"""sLSTM step and sequence with the reference's signatures, on HIP.

Drop-in for ``slstm_step_pytorch`` (xlstm_metal/torch_native/blocks/slstm/
slstm_layers/stepwise/slstm_metal_kernel.py:14-65), ``sLSTMStepwiseKernelCell``
(.../stepwise/slstm_stepwise_kernel_cell.py:18-97) and the time loop of
``sLSTMNeuron.forward`` (.../slstm_layers/slstm_neuron.py:132-143).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .ops import slstm_sequence_op, slstm_step_op, state_views

__all__ = ["slstm_step", "slstm_step_pytorch", "slstm_sequence", "sLSTMStepwiseKernelCell"]


def slstm_step(z, i_preact, f_preact, o_preact, c_state, n_state, m_state, eps: float = 1e-6):
    """Returns (h [B,NH,H], c [B,NH,H], n [B,NH,H], m [B,NH])."""
    h, st = slstm_step_op(z, i_preact, f_preact, o_preact, c_state, n_state, m_state, float(eps))
    return (h, *state_views(st, *z.shape))


slstm_step_pytorch = slstm_step


def slstm_sequence(z, i_preact, f_preact, o_preact, state=None, eps: float = 1e-6):
    """z [B,S,NH,H], gates [B,S,NH] -> (h [B,S,NH,H], (c, n, m)); one launch for all S."""
    c0, n0, m0 = state if state is not None else (None, None, None)
    h, st = slstm_sequence_op(z, i_preact, f_preact, o_preact, c0, n0, m0, float(eps))
    B, _, NH, H = z.shape
    return h, state_views(st, B, NH, H)


class sLSTMStepwiseKernelCell(nn.Module):
    """Single-step sLSTM recurrence (slstm_stepwise_kernel_cell.py:18-97)."""

    def __init__(self, num_heads: int, head_dim: int, eps: float = 1e-6):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.eps = eps

    def forward(self, z, i_preact, f_preact, o_preact,
                state: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None):
        B, NH, H = z.shape
        if state is None:
            c = torch.zeros((B, NH, H), dtype=z.dtype, device=z.device)
            n = torch.zeros((B, NH, H), dtype=z.dtype, device=z.device)
            m = torch.zeros((B, NH), dtype=z.dtype, device=z.device)
        else:
            c, n, m = state
        h, st = slstm_step_op(z, i_preact, f_preact, o_preact, c, n, m, float(self.eps))
        return h, state_views(st, B, NH, H)
