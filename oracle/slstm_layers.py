"""CPU oracle for the sLSTM layer's conv1d + SiLU and per-head GroupNorm: test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module; the product path never does.  numpy,
float64 arithmetic on the (possibly 16-bit) inputs.

Reference (paths relative to the MLXPorts/xLSTM-metal root,
``SL`` = ``xlstm_metal/torch_native/blocks/slstm/slstm_layers``):

* ``causal_conv1d``: ``SL/causal_conv1d/causal_conv1d.py:51-67`` on the CPU:
  ``F.pad(x, (K - 1, 0))`` then ``nn.Conv1d(groups=channels)``, i.e. the
  cross-correlation y[s] = b + sum_j w[j] x[s - K + 1 + j] (w[K-1] on the
  current step).  The Metal depthwise kernel (``depthwise_kernel.metal:35-39``)
  pairs w[k] with x[s - k], the taps in the opposite order; it is not followed.
  ``activation="silu"`` adds the ``nn.SiLU`` of ``SL/slstm_projection_cell.py:
  110-115``.  With a 16-bit dtype the convolution's output is rounded to that
  dtype before the SiLU (each reference module returns its input's dtype).
* ``group_norm``: ``nn.GroupNorm(num_groups=NH, num_channels=NH*H, eps)`` of
  ``SL/slstm_output_cell.py:53,72-83`` on ``h.view(B*S, NH*H)``: per row and
  group, (x - mean) / sqrt(biased var + eps) * weight + bias.

Pinned (tests/test_oracle_slstm_layers.py) against torch's own CPU
``F.conv1d`` / ``F.group_norm`` in float64 (the reference's computation), by the
impulse response (which fixes the tap order), K = 1 (an affine map), and the
moments of the normalised output.
"""

from __future__ import annotations

import numpy as np
import torch

__all__ = ["causal_conv1d", "group_norm"]


def _np64(t):
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


def _round_to(a: np.ndarray, dtype) -> np.ndarray:
    if dtype in (None, torch.float32, torch.float64):
        return a
    return torch.from_numpy(a).to(dtype).to(torch.float64).numpy()


def causal_conv1d(x, weight, bias=None, activation=None, dtype=None):
    """x [B, S, D] (channels last), weight [D, K] or [D, 1, K], bias [D] or None.

    Returns float64 [B, S, D].  ``dtype``: the module dtype whose rounding of
    the convolution precedes the SiLU (default: x's dtype when x is a tensor).
    """
    if dtype is None and isinstance(x, torch.Tensor):
        dtype = x.dtype
    xv = _np64(x)
    w = _np64(weight)
    w = w.reshape(w.shape[0], -1)
    B, S, D = xv.shape
    K = w.shape[1]
    xp = np.concatenate([np.zeros((B, K - 1, D)), xv], axis=1)  # left pad K - 1 (causal_conv1d.py:63-64)
    y = np.zeros((B, S, D))
    for j in range(K):  # nn.Conv1d: output s reads padded positions s .. s + K - 1 with taps 0 .. K - 1
        y += w[:, j] * xp[:, j:j + S, :]
    if bias is not None:
        y += _np64(bias)
    if activation == "silu":
        a = _round_to(y, dtype)
        y = a / (1.0 + np.exp(-a))
    elif activation is not None:
        raise ValueError(f"unknown activation {activation!r}")
    return y


def group_norm(x, num_groups, weight=None, bias=None, eps=1e-5):
    """x [N, C] with C = num_groups * CG; weight, bias [C] or None, each optional (the
    MultiHeadLayerNorm of
    ``xlstm_metal/torch_native/blocks/mlstm/multihead_norm/multihead_norm.py:27-40`` has a
    weight and no bias by default).  Returns float64 [N, C]."""
    xv = _np64(x)
    N, C = xv.shape
    G = int(num_groups)
    xg = xv.reshape(N, G, C // G)
    mean = xg.mean(axis=2, keepdims=True)
    var = ((xg - mean) ** 2).mean(axis=2, keepdims=True)
    y = ((xg - mean) / np.sqrt(var + eps)).reshape(N, C)
    if weight is not None:
        y = y * _np64(weight)
    if bias is not None:
        y = y + _np64(bias)
    return y
