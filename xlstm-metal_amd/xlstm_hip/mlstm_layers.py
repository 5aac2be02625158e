"""The mLSTM output cell's stage after the chunkwise kernel, on HIP.

Drop-ins (paths relative to the reference root, ``TNM`` =
``xlstm_metal/torch_native/blocks/mlstm``):

* ``MultiHeadLayerNorm`` (``TNM/multihead_norm/multihead_norm.py:5-40``): per-head
  LayerNorm, on the GroupNorm kernel with one group per head.
* ``MultiHeadRMSNorm`` (``TNM/multihead_norm/multihead_norm.py:43-64``): per-head
  RMS normalisation of [B, S, NH, DH], flattened to [B, S, NH * DH], optional
  per-channel weight.
* ``mLSTMOutputCell`` (``TNM/mlstm_chunkwise/mlstm_output_cell.py:22-99``): the
  permute of the kernel output, the norm, sigmoid(ogate_proj(x)) and the gate
  product are one kernel (``mh_rmsnorm_gate_kernel``) reading h in the chunkwise
  layout [B, NH, S, DH]; the two projections stay ``nn.Linear``.  The reference's
  ``x_norm.view(B, S, -1)`` raises on the permuted (non-contiguous) tensor; the
  kernel writes the flattening that ``reshape`` would give.

* ``mLSTMProjectionCell`` (``TNM/mlstm_chunkwise/mlstm_projection_cell.py:18-106``): the
  q, k, v projections stay ``nn.Linear``; the two gate projections and their soft-cap are one
  kernel (``gate_proj_kernel``) over the stacked gate weights.

State-dict keys match the reference modules.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .ops import gate_proj_softcap_op, mh_rmsnorm_gate_op
from .soft_cap import soft_cap

__all__ = ["mh_rmsnorm_gate", "gate_proj_softcap", "stacked_linears", "MultiHeadRMSNorm", "MultiHeadLayerNorm",
           "mLSTMProjectionCell", "mLSTMOutputCell"]


def gate_proj_softcap(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None,
                      cap: Optional[float] = None, cap_in_dtype: bool = False) -> Tensor:
    """``cap * tanh(F.linear(x, weight, bias) / cap)`` for a few gate outputs (weight [G, D], G <= 64).

    bf16 / f16: one kernel reading x once (the Linear's output rounded to x's dtype before the
    soft-cap, as the reference's two modules do); float32: ``F.linear`` then the soft-cap kernel.
    ``cap_in_dtype``: the soft-cap's operations are each rounded to x's dtype, as torch evaluates
    ``cap * tanh(x / cap)`` on 16-bit tensors (sLSTMProjectionCell.soft_cap,
    slstm_projection_cell.py:84-89); otherwise it is computed in float32 and rounded once
    (SoftCapCell, which mLSTMProjectionCell uses).  ``cap`` None or <= 0: no soft-cap.
    """
    c = 0.0 if cap is None else float(cap)
    if x.dtype == torch.float32:
        y = F.linear(x, weight, bias)
        return soft_cap(y, c) if c > 0 else y
    return gate_proj_softcap_op(x, weight, bias, c, 1 if cap_in_dtype else 0)


def stacked_linears(*linears: nn.Linear):
    """(weight, bias) of several Linear layers over the same input, stacked row-wise (a missing bias
    is zeros; None when none has one)."""
    w = torch.cat([lin.weight for lin in linears])
    if all(lin.bias is None for lin in linears):
        return w, None
    b = torch.cat([lin.bias if lin.bias is not None else lin.weight.new_zeros(lin.out_features) for lin in linears])
    return w, b


def mh_rmsnorm_gate(h: Tensor, weight: Optional[Tensor] = None, o_preact: Optional[Tensor] = None,
                    eps: float = 1e-6, heads_first: bool = True) -> Tensor:
    """(h / rms(h over DH)) * weight * sigmoid(o_preact) as [B, S, NH * DH].

    h is [B, NH, S, DH] (``heads_first``, the chunkwise output) or [B, S, NH, DH]; weight
    [NH * DH] or None; o_preact [B, S, NH * DH] (the gate projection before its sigmoid) or None.
    """
    return mh_rmsnorm_gate_op(h, weight, o_preact, bool(heads_first), float(eps))


class MultiHeadRMSNorm(nn.Module):
    """``multihead_norm.py:43-64``: x [B, S, NH, DH] -> [B, S, NH * DH]."""

    def __init__(self, num_heads: int, head_dim: int, eps: float = 1e-6, use_weight: bool = True) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.eps = eps
        if use_weight:
            self.weight = nn.Parameter(torch.ones(num_heads * head_dim))
        else:
            self.register_parameter("weight", None)

    def forward(self, x: Tensor) -> Tensor:
        B, S, NH, DH = x.shape
        if NH != self.num_heads or DH != self.head_dim:
            raise ValueError(f"Expected shape [B,S,{self.num_heads},{self.head_dim}], got {x.shape}")
        return mh_rmsnorm_gate(x, self.weight, None, self.eps, heads_first=False)


class mLSTMProjectionCell(nn.Module):
    """``mlstm_projection_cell.py:18-106``: q, k, v [B, NH, S, DH] (permuted views) and the soft-capped
    gate pre-activations i, f [B, NH, S] (permuted views) of x [B, S, input_size]."""

    def __init__(self, input_size: int, num_heads: int, qk_dim_per_head: int, v_dim_per_head: int,
                 use_bias: bool = False, gate_soft_cap: Optional[float] = None) -> None:
        super().__init__()
        self.input_size = input_size
        self.num_heads = num_heads
        self.qk_dim_per_head = qk_dim_per_head
        self.v_dim_per_head = v_dim_per_head
        self.gate_soft_cap = gate_soft_cap
        qk_dim, v_dim = num_heads * qk_dim_per_head, num_heads * v_dim_per_head
        self.q_proj = nn.Linear(input_size, qk_dim, bias=use_bias)
        self.k_proj = nn.Linear(input_size, qk_dim, bias=use_bias)
        self.v_proj = nn.Linear(input_size, v_dim, bias=use_bias)
        self.igate_proj = nn.Linear(input_size, num_heads)
        self.fgate_proj = nn.Linear(input_size, num_heads)

    def forward(self, x: Tensor):
        B, S, _ = x.shape
        NH = self.num_heads
        q = self.q_proj(x).view(B, S, NH, self.qk_dim_per_head).permute(0, 2, 1, 3)
        k = self.k_proj(x).view(B, S, NH, self.qk_dim_per_head).permute(0, 2, 1, 3)
        v = self.v_proj(x).view(B, S, NH, self.v_dim_per_head).permute(0, 2, 1, 3)
        g = gate_proj_softcap(x, *stacked_linears(self.igate_proj, self.fgate_proj), self.gate_soft_cap)
        return q, k, v, g[..., :NH].permute(0, 2, 1), g[..., NH:].permute(0, 2, 1)


class MultiHeadLayerNorm(nn.Module):
    """``multihead_norm.py:5-40``: per-head LayerNorm of x [B, S, NH, DH] -> [B, S, NH * DH], optional
    weight and bias.  Runs ``group_norm_kernel`` (one group per head) on the [B * S, NH * DH] view,
    with float32 statistics and one rounding of the output; the reference takes the mean and
    variance in x's own dtype."""

    def __init__(self, num_heads: int, head_dim: int, eps: float = 1e-6, use_weight: bool = True,
                 use_bias: bool = False) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.eps = eps
        self.use_weight = use_weight
        self.use_bias = use_bias
        if use_weight:
            self.weight = nn.Parameter(torch.ones(num_heads * head_dim))
        else:
            self.register_parameter("weight", None)
        if use_bias:
            self.bias = nn.Parameter(torch.zeros(num_heads * head_dim))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: Tensor) -> Tensor:
        B, S, NH, DH = x.shape
        if NH != self.num_heads or DH != self.head_dim:
            raise ValueError(f"Expected shape [B,S,{self.num_heads},{self.head_dim}], got {x.shape}")
        from .slstm_layers import group_norm
        return group_norm(x.reshape(B * S, NH * DH), NH, self.weight, self.bias, self.eps).view(B, S, NH * DH)


class mLSTMOutputCell(nn.Module):
    """``mlstm_output_cell.py:22-99``: norm(h) * sigmoid(ogate_proj(x_orig)), then out_proj."""

    def __init__(self, input_size: int, num_heads: int, v_dim_per_head: int, use_bias: bool = False,
                 eps: float = 1e-6) -> None:
        super().__init__()
        self.input_size = input_size
        self.num_heads = num_heads
        self.v_dim_per_head = v_dim_per_head
        v_dim = num_heads * v_dim_per_head
        self.norm = MultiHeadRMSNorm(num_heads=num_heads, head_dim=v_dim_per_head, eps=eps)
        self.ogate_proj = nn.Linear(input_size, v_dim, bias=use_bias)
        self.out_proj = nn.Linear(v_dim, input_size, bias=use_bias)

    def gated(self, h: Tensor, x_orig: Tensor) -> Tensor:
        """h [B, NH, S, DH_v] (the kernel output), x_orig [B, S, input_size] -> [B, S, NH * DH_v]."""
        return mh_rmsnorm_gate(h, self.norm.weight, self.ogate_proj(x_orig), self.norm.eps, heads_first=True)

    def forward(self, h: Tensor, x_orig: Tensor) -> Tensor:
        return self.out_proj(self.gated(h, x_orig))
