"""Independent numpy restatement of the recurrent mLSTM: test infrastructure only.

Written as a second, framework-free statement of the recurrence so that the
torch oracle (``oracle.mlstm``) can be checked against something that shares
none of its code.  It follows the reference's own parity helper
``tests/parity/canonical_reference.py:59-111`` (``canonical_mlstm_recurrent_
sequence``) and its ``_logsigmoid`` (``:14-15``): per step
``m' = max(logsig f + m, i)``, ``C' = e^{logsig f + m - m'} C + e^{i - m'} k v^T``,
``n' = ... n + ... k``, ``h = (q/sqrt(D)) C' / (max(|(q/sqrt(D)) n'|, e^{-m'}) + eps)``.
It runs in whatever float dtype its inputs have (float64 for fixtures).

Also holds :func:`brute_force_h`, the stabiliser-free O(S^2) closed form of
the same model used to pin both restatements.
"""

from __future__ import annotations

import numpy as np

__all__ = ["logsigmoid", "recurrent_sequence", "brute_force_h"]


def logsigmoid(x):
    """``-log(1 + exp(-x))`` computed stably (``canonical_reference.py:14-15``)."""
    return -np.logaddexp(0.0, -x)


def recurrent_sequence(q, k, v, i_pre, f_pre, eps, state=None):
    """``canonical_reference.py:59-111``; q,k [B,NH,S,DK], v [B,NH,S,DV], gates [B,NH,S]."""
    B, NH, S, DK = q.shape
    DV = v.shape[-1]
    dt = q.dtype
    if state is None:
        C = np.zeros((B, NH, DK, DV), dtype=dt)
        n = np.zeros((B, NH, DK), dtype=dt)
        m = np.zeros((B, NH, 1), dtype=dt)
    else:
        C, n, m = (np.array(s, dtype=dt, copy=True) for s in state)
    scale = 1.0 / np.sqrt(DK)
    hs = []
    for t in range(S):
        ig = i_pre[:, :, t][:, :, None]
        fl = logsigmoid(f_pre[:, :, t][:, :, None])
        m_new = np.maximum(fl + m, ig)
        fa = np.exp(fl + m - m_new)
        ia = np.exp(ig - m_new)
        C = fa[..., None] * C + ia[..., None] * (k[:, :, t, :, None] * v[:, :, t, None, :])
        n = fa * n + ia * k[:, :, t, :]
        m = m_new
        qs = q[:, :, t, :] * scale
        num = np.einsum("bhd,bhdv->bhv", qs, C)
        qn = np.einsum("bhd,bhd->bh", qs, n)
        den = np.maximum(np.abs(qn), np.exp(-m[..., 0])) + eps
        hs.append(num / den[..., None])
    return np.stack(hs, axis=2), (C, n, m)


def brute_force_h(q, k, v, i_pre, f_pre, eps, m0=0.0):
    """Closed form of the model from zero initial C and n, no stabiliser.

    ``num_t = sum_{j<=t} (q_t.k_j / sqrt(D)) exp(sum_{l=j+1..t} logsig f_l + i_j) v_j``,
    ``den_t`` the same without ``v_j``; with the running max
    ``m_t = max(b_t + m0, max_{j<=t} (b_t - b_j + i_j))`` (b = cumsum logsig f)
    the output is ``h_t = num_t e^{-m_t} / (max(|den_t|, 1) e^{-m_t} + eps)``.
    For eps = 0 this is ``num_t / max(|den_t|, 1)``, independent of m.
    Loops in Python: small inputs only.
    """
    B, NH, S, DK = q.shape
    out = np.zeros(v.shape[:3] + (v.shape[-1],), dtype=np.float64)
    scale = 1.0 / np.sqrt(DK)
    for b in range(B):
        for h in range(NH):
            lsf = logsigmoid(np.asarray(f_pre[b, h], dtype=np.float64))
            cum = np.cumsum(lsf)
            for t in range(S):
                logw = cum[t] - cum[: t + 1] + i_pre[b, h, : t + 1]
                m_t = max(cum[t] + m0, float(np.max(logw)))
                w = np.exp(logw - m_t) * (k[b, h, : t + 1] @ q[b, h, t]) * scale
                num = w @ v[b, h, : t + 1]
                den = max(abs(w.sum()), np.exp(-m_t))
                out[b, h, t] = num / (den + eps)
    return out
