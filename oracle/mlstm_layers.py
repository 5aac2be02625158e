"""CPU oracle for the mLSTM output cell's multi-head RMSNorm x sigmoid(o): test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module; the product path never does.  numpy,
float64 arithmetic on the (possibly 16-bit) inputs.

Reference (paths relative to the MLXPorts/xLSTM-metal root, ``TNM`` =
``xlstm_metal/torch_native/blocks/mlstm``):

* ``TNM/multihead_norm/multihead_norm.py:56-64`` (``MultiHeadRMSNorm.forward``):
  rms = sqrt(mean(x.float()^2) + eps) per head; ``(x / rms).type_as(x)`` (the
  division in float32, rounded to x's dtype); flattened to [B, S, NH * DH]; times
  the weight in the module dtype (rounded again for a 16-bit model).
* ``TNM/mlstm_chunkwise/mlstm_output_cell.py:84-93``: h [B, NH, S, DH] permuted to
  [B, S, NH, DH] first; ``sigmoid(ogate_proj(x))`` in the module dtype (rounded);
  the gate product (rounded to the output dtype by the caller's comparison).
  The reference's ``view`` of the permuted tensor raises; the oracle flattens
  as ``reshape`` would.

* ``gate_proj_softcap``: the gate projections of the projection cells with
  their soft-cap, ``soft_cap(igate_proj(x))`` etc.
  (``TNM/mlstm_chunkwise/mlstm_projection_cell.py:97-103``,
  ``xlstm_metal/torch_native/blocks/slstm/slstm_layers/slstm_projection_cell.py:
  118-121``): x w^T + b rounded to the module dtype (the Linear's output),
  then cap * tanh(z / cap): in float64 for the mLSTM cell's SoftCapCell (which
  computes in float32 and casts once), or with cap, z / cap, tanh and the product
  each rounded to the dtype (``cap_in_dtype``) for the sLSTM cell, which
  evaluates ``cap * torch.tanh(x / cap)`` on tensors of x's dtype
  (``slstm_projection_cell.py:84-89``).

Pinned (tests/test_oracle_mlstm_layers.py) against torch's CPU
``F.rms_norm`` in float64, the closed forms of a constant head (x / rms =
sign(x) for eps = 0) and of the output's root mean square, ``math.exp`` for the
sigmoid, and torch's own bf16 type promotion of the reference's expression.
"""

from __future__ import annotations

import numpy as np
import torch

__all__ = ["mh_rmsnorm_gate", "gate_proj_softcap"]


def _np64(t):
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


def _round_to(a, dtype):
    if dtype in (None, torch.float32, torch.float64):
        return a
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(torch.float64).numpy()


def mh_rmsnorm_gate(h, weight=None, o_preact=None, eps=1e-6, heads_first=True, dtype=None):
    """h [B, NH, S, DH] (heads_first) or [B, S, NH, DH]; weight [NH * DH] or None; o_preact
    [B, S, NH * DH] or None.  Returns float64 [B, S, NH * DH] before the final rounding."""
    if dtype is None and isinstance(h, torch.Tensor):
        dtype = h.dtype
    x = _np64(h)
    if heads_first:
        x = x.transpose(0, 2, 1, 3)  # mlstm_output_cell.py:84
    B, S, NH, DH = x.shape
    rms = np.sqrt((x ** 2).mean(axis=-1, keepdims=True) + eps)  # multihead_norm.py:59
    y = _round_to(x / rms, dtype).reshape(B, S, NH * DH)  # :60-61
    if weight is not None:
        y = _round_to(y * _np64(weight), dtype)  # :62-63
    if o_preact is not None:
        o = _np64(o_preact).reshape(B, S, NH * DH)
        y = y * _round_to(1.0 / (1.0 + np.exp(-o)), dtype)  # mlstm_output_cell.py:90-93
    return y


def gate_proj_softcap(x, weight, bias=None, cap=15.0, dtype=None, cap_in_dtype=False):
    """x [..., D], weight [G, D], bias [G] or None.  Returns float64 [..., G] before the final
    rounding: the Linear's output rounded to ``dtype`` (x's by default), then the soft-cap
    (with ``cap_in_dtype``: cap, z / cap and tanh each rounded to ``dtype`` first)."""
    if dtype is None and isinstance(x, torch.Tensor):
        dtype = x.dtype
    z = _np64(x) @ _np64(weight).T
    if bias is not None:
        z = z + _np64(bias)
    z = _round_to(z, dtype)
    if cap <= 0:
        return z
    if cap_in_dtype:
        capr = float(_round_to(np.float64(cap), dtype))
        return capr * _round_to(np.tanh(_round_to(z / capr, dtype)), dtype)
    return cap * np.tanh(z / cap)
