"""CPU oracle for the sLSTM step and the soft-cap: test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module; the product path never does.

Reference (paths relative to the MLXPorts/xLSTM-metal root):

* ``slstm_step``: ``xlstm_metal/torch_native/blocks/slstm/slstm_layers/
  stepwise/slstm_metal_kernel.py:14-65`` (``slstm_step_pytorch``), identical
  math in ``.../stepwise/slstm_stepwise_kernel_cell.py:47-97``.  This is the
  torch-native variant: ``tanh(z)`` input and ``|n|`` in the denominator.
  The MLX Metal kernel (clamped exponentials, no abs) and ``sLSTMCell`` are
  different numerics and are deliberately not followed.
* ``slstm_sequence``: the per-timestep loop of ``sLSTMNeuron.forward``
  (``.../slstm_layers/slstm_neuron.py:132-143``) over z [B,S,NH,H] and gates
  [B,S,NH], zero initial state (``slstm_stepwise_kernel_cell.py:75-78``).
* ``soft_cap``: ``cap * tanh(x / cap)``, identity for ``cap <= 0``
  (``xlstm_metal/torch_native/blocks/soft_cap/softcap.py:25-31``,
  ``soft_cap_kernel.metal:14``, CPU form ``.../slstm_projection_cell.py:84-89``).

Pinned by closed forms evaluated with the ``math`` module and by the soft-cap
known answers of ``kernel_development/soft_cap/mlx_fast_kernels/
test_softcap.py:6-56`` (tests/test_oracle_slstm_softcap.py).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["slstm_step", "slstm_sequence", "soft_cap"]


def slstm_step(z, i_preact, f_preact, o_preact, c_state, n_state, m_state, eps=1e-6):
    """``slstm_metal_kernel.py:45-65``: returns ``(h, c', n', m')``."""
    lsf = F.logsigmoid(f_preact)
    m_new = torch.maximum(m_state + lsf, i_preact)
    ig = torch.exp(i_preact - m_new)
    fg = torch.exp(m_state + lsf - m_new)
    og = torch.sigmoid(o_preact)
    c_new = fg.unsqueeze(-1) * c_state + ig.unsqueeze(-1) * torch.tanh(z)
    n_new = fg.unsqueeze(-1) * n_state + ig.unsqueeze(-1)
    h = og.unsqueeze(-1) * c_new / (torch.abs(n_new) + eps)
    return h, c_new, n_new, m_new


def slstm_sequence(z, i_preact, f_preact, o_preact, state=None, eps=1e-6):
    """Loop of ``slstm_neuron.py:132-143`` over S; returns ``(h [B,S,NH,H], (c, n, m))``."""
    B, S, NH, H = z.shape
    if state is None:
        c = torch.zeros((B, NH, H), dtype=z.dtype)
        n = torch.zeros((B, NH, H), dtype=z.dtype)
        m = torch.zeros((B, NH), dtype=z.dtype)
    else:
        c, n, m = state
    hs = []
    for t in range(S):
        h, c, n, m = slstm_step(z[:, t], i_preact[:, t], f_preact[:, t], o_preact[:, t], c, n, m, eps)
        hs.append(h)
    return torch.stack(hs, dim=1), (c, n, m)


def soft_cap(x, cap):
    """``cap * tanh(x / cap)``; identity when ``cap <= 0`` (``softcap.py:27-28``)."""
    cap = float(cap)
    if cap <= 0.0:
        return x
    return cap * torch.tanh(x / cap)
