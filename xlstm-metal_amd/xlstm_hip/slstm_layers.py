"""The sLSTM layer's stages either side of its time loop, on HIP.

Drop-ins for the torch-native sLSTM layer modules (paths relative to the
reference root, ``SL`` = ``xlstm_metal/torch_native/blocks/slstm/slstm_layers``):

* ``CausalConv1d`` (``SL/causal_conv1d/causal_conv1d.py:14-83``): same
  constructor and ``conv`` parameters, forward on [B, C, S]; the depthwise case
  (groups == channels) runs ``causal_conv1d_kernel``.  Other groupings raise
  ``NotImplementedError`` (no CPU path).
* ``sLSTMProjectionCell`` (``SL/slstm_projection_cell.py:25-126``): the conv and
  its SiLU are one kernel on the channels-last input (no permuted copies); the
  gate projections with their soft-cap are ``gate_proj_kernel`` (i and f
  stacked over the conv output, o over the input; float32 takes ``nn.Linear``
  and ``soft_cap_kernel``); the z projection is ``nn.Linear`` (a library GEMM).
* ``sLSTMOutputCell`` (``SL/slstm_output_cell.py:18-91``): the per-head
  ``nn.GroupNorm`` runs ``group_norm_kernel``; ``out_proj`` is ``nn.Linear``.

State-dict keys match the reference modules, so their checkpoints load as is.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from .ops import CONV_ACTS, causal_conv1d_op, group_norm_op
from .soft_cap import soft_cap

__all__ = ["causal_conv1d", "group_norm", "CausalConv1d", "sLSTMProjectionCell", "sLSTMOutputCell"]


def causal_conv1d(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None,
                  activation: Optional[str] = None) -> Tensor:
    """Depthwise causal conv over time of a channels-last x [B, S, D]; weight [D, K] or nn.Conv1d's
    [D, 1, K], bias [D] or None; ``activation`` None or "silu".  Returns [B, S, D] in x's dtype."""
    if activation not in CONV_ACTS:
        raise ValueError(f"causal_conv1d: activation must be None or 'silu', got {activation!r}")
    return causal_conv1d_op(x, weight, bias, CONV_ACTS[activation])


def group_norm(x: Tensor, num_groups: int, weight: Optional[Tensor] = None, bias: Optional[Tensor] = None,
               eps: float = 1e-5) -> Tensor:
    """``F.group_norm`` of a 2-D x [N, C] (groups of C / num_groups consecutive channels)."""
    return group_norm_op(x, int(num_groups), weight, bias, float(eps))


class CausalConv1d(nn.Module):
    """``causal_conv1d.py:14-83``: left pad of kernel_size - 1, then a (depthwise) nn.Conv1d."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, groups: int = 1,
                 bias: bool = True) -> None:
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = kernel_size
        self.groups = groups
        self.conv = nn.Conv1d(in_channels=in_channels, out_channels=out_channels, kernel_size=kernel_size,
                              groups=groups, bias=bias)
        self.padding = kernel_size - 1

    def _check_depthwise(self) -> None:
        if not (self.groups == self.in_channels == self.out_channels):
            raise NotImplementedError(
                f"CausalConv1d: only the depthwise form (groups == in_channels == out_channels) has a HIP kernel; "
                f"got in={self.in_channels} out={self.out_channels} groups={self.groups}")

    def forward_channels_last(self, x: Tensor, activation: Optional[str] = None) -> Tensor:
        """x [B, S, C] -> [B, S, C], with the activation fused."""
        self._check_depthwise()
        return causal_conv1d(x, self.conv.weight, self.conv.bias, activation)

    def forward(self, x: Tensor) -> Tensor:
        """x [B, C, S] -> [B, C, S] (the reference's layout; a permuted view of channels-last memory
        is read in place)."""
        return self.forward_channels_last(x.permute(0, 2, 1)).permute(0, 2, 1)

    def get_config(self) -> dict:
        return {"in_channels": self.in_channels, "out_channels": self.out_channels,
                "kernel_size": self.kernel_size, "groups": self.groups}


class sLSTMProjectionCell(nn.Module):
    """``slstm_projection_cell.py:25-126``: conv + SiLU -> i, f; raw input -> z, o; gates soft-capped."""

    def __init__(self, input_size: int, num_heads: int, head_dim: int, conv1d_kernel_size: int = 4,
                 use_bias: bool = False, gate_soft_cap: float = 15.0) -> None:
        super().__init__()
        self.input_size = input_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.conv1d_kernel_size = conv1d_kernel_size
        self.gate_soft_cap = gate_soft_cap
        hidden_size = num_heads * head_dim
        if conv1d_kernel_size > 0:
            self.conv1d = CausalConv1d(input_size, input_size, conv1d_kernel_size, groups=input_size)
            self.conv_act = nn.SiLU()
        else:
            self.conv1d = None
        self.igate_proj = nn.Linear(input_size, num_heads)
        self.fgate_proj = nn.Linear(input_size, num_heads)
        self.ogate_proj = nn.Linear(input_size, num_heads)
        self.z_proj = nn.Linear(input_size, hidden_size, bias=use_bias)

    def soft_cap(self, x: Tensor) -> Tensor:
        return x if self.gate_soft_cap is None else soft_cap(x, float(self.gate_soft_cap))

    def forward(self, x: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
        """x [B, S, D] -> z [B, S, NH, H], i, f, o pre-activations [B, S, NH], x_conv [B, S, D].

        i and f are one gate-projection kernel over x_conv (their weights stacked), o one over x."""
        from .mlstm_layers import gate_proj_softcap, stacked_linears
        B, S, _ = x.shape
        NH = self.num_heads
        x_conv = x if self.conv1d is None else self.conv1d.forward_channels_last(x, activation="silu")
        # the reference soft-caps with torch ops in x's dtype (slstm_projection_cell.py:84-89)
        gif = gate_proj_softcap(x_conv, *stacked_linears(self.igate_proj, self.fgate_proj), self.gate_soft_cap,
                                cap_in_dtype=True)
        o_preact = gate_proj_softcap(x, self.ogate_proj.weight, self.ogate_proj.bias, self.gate_soft_cap,
                                     cap_in_dtype=True)
        z = self.z_proj(x).view(B, S, NH, self.head_dim)
        return z, gif[..., :NH], gif[..., NH:], o_preact, x_conv


class sLSTMOutputCell(nn.Module):
    """``slstm_output_cell.py:18-91``: per-head GroupNorm, then the output projection."""

    def __init__(self, input_size: int, num_heads: int, head_dim: int, use_bias: bool = False,
                 eps: float = 1e-6) -> None:
        super().__init__()
        self.input_size = input_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        hidden_size = num_heads * head_dim
        self.group_norm = nn.GroupNorm(num_groups=num_heads, num_channels=hidden_size, eps=eps)
        self.out_proj = nn.Linear(hidden_size, input_size, bias=use_bias)

    def normalize(self, h: Tensor) -> Tensor:
        """h [B, S, NH, H] -> the GroupNorm output [B, S, NH * H]."""
        B, S, NH, H = h.shape
        gn = self.group_norm
        w, b = (gn.weight, gn.bias) if gn.affine else (None, None)
        return group_norm(h.reshape(B * S, NH * H), gn.num_groups, w, b, gn.eps).view(B, S, NH * H)

    def forward(self, h: Tensor) -> Tensor:
        return self.out_proj(self.normalize(h))
