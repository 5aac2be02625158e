"""soft_cap on HIP: drop-in for ``soft_cap(x, cap)`` and ``SoftCapCell``, and the logit
projection with the soft-cap fused into its epilogue.

Reference: xlstm_metal/torch_native/blocks/soft_cap/softcap_metal.py:29-31 and
softcap.py:14-31 (cap <= 0 returns x itself).  float32, bfloat16 and float16
(arithmetic in float32).  ``lm_head_softcap(x, weight, cap)`` is
``soft_cap(F.linear(x, weight), cap)``, the tail of the model's forward
(xlstm_metal/torch_native/models/wired_xlstm.py:176 and generate.py:131).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

import torch.nn.functional as F

from .ops import LM_HEAD_MAX_LDS, LM_HEAD_MAX_ROWS, lm_head_softcap_op, soft_cap_op

__all__ = ["soft_cap", "SoftCapCell", "lm_head_softcap"]


def soft_cap(x: torch.Tensor, cap: float) -> torch.Tensor:
    if float(cap) <= 0.0:
        return x
    return soft_cap_op(x, float(cap))


class SoftCapCell(nn.Module):
    """Module form (softcap.py:14-31)."""

    def __init__(self, cap_value: Optional[float] = None) -> None:
        super().__init__()
        self.register_buffer("_cap", torch.tensor(float(cap_value) if cap_value is not None else 0.0),
                             persistent=False)

    def forward(self, x: torch.Tensor, cap_value: Optional[float] = None) -> torch.Tensor:
        cap = float(cap_value) if cap_value is not None else float(self._cap.item())
        return soft_cap(x, cap)


def lm_head_softcap(x: torch.Tensor, weight: torch.Tensor, cap: float) -> torch.Tensor:
    """soft_cap(F.linear(x, weight), cap) for x [..., D], weight [V, D] (bf16 / f16).

    Up to 16 rows of x (a decode step's tokens, a prompt's last positions) run the fused kernel,
    which streams the weights once for all rows and soft-caps in the epilogue; more rows (the
    logits of every position; rows of D beyond the kernel's 160 KiB of LDS staging) run as the
    Linear then the soft_cap kernel."""
    D = x.shape[-1]
    rows = x.numel() // max(D, 1)
    if x.dtype == torch.float32 or rows > LM_HEAD_MAX_ROWS or rows * (D + 8) * 2 > LM_HEAD_MAX_LDS:
        return soft_cap(F.linear(x, weight), cap)
    return lm_head_softcap_op(x, weight, float(cap))
