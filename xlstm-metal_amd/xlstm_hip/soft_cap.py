"""soft_cap on HIP: drop-in for ``soft_cap(x, cap)`` and ``SoftCapCell``.

Reference: xlstm_metal/torch_native/blocks/soft_cap/softcap_metal.py:29-31 and
softcap.py:14-31 (cap <= 0 returns x itself).  float32, bfloat16 and float16
(arithmetic in float32).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .ops import soft_cap_op

__all__ = ["soft_cap", "SoftCapCell"]


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
