"""The oracle's restatement of the reference's custom chunkwise backward (oracle.mlstm.mlstm_chunkwise_bw,
VTN/bw.py:198-352), pinned in float64 against torch.autograd through the oracle's forward.

The reference's backward treats each token's divisor max(|den|, exp(-m)) + eps and the stabilisers as
constants.  That is exact for a loss that sees h only through each row's direction h / |h| (the
mLSTM layer's multi-head norm removes the per-row scale), so there its gradients must equal
autograd's — a dropped term, a wrong sign or a transposed product in any of dq, dk, dv, di, df, dc0
shows up as a mismatch.  On the last-state path the reference's suffix-sum form of df leaves out
the constant <G, C_true> (C_true = C_last exp(m_last)) times sigmoid(-f); the test pins that too.
"""

import pytest
import torch

from oracle import mlstm as om

F64 = torch.float64


def _inputs(B, NH, S, DQK, DV, seed, states=False):
    g = torch.Generator().manual_seed(seed)
    # q, k with a positive mean keep every denominator well above exp(-m), so the forward's
    # max(|den|, exp(-m)) takes the |den| branch everywhere (where the reference's backward is exact)
    q = torch.randn(B, NH, S, DQK, generator=g, dtype=F64) * 0.5 + 1.0
    k = torch.randn(B, NH, S, DQK, generator=g, dtype=F64) * 0.5 + 1.0
    v = torch.randn(B, NH, S, DV, generator=g, dtype=F64)
    i = torch.randn(B, NH, S, generator=g, dtype=F64) + 2.0
    f = torch.randn(B, NH, S, generator=g, dtype=F64) + 2.0
    st = None
    if states:
        st = (torch.randn(B, NH, DQK, DV, generator=g, dtype=F64) * 0.3,
              torch.rand(B, NH, DQK, generator=g, dtype=F64) + 0.5,
              torch.randn(B, NH, 1, generator=g, dtype=F64) * 0.5)
    return (q, k, v, i, f), st


def _direction_loss(h, W):
    return (W * h / h.norm(dim=-1, keepdim=True)).sum()


def _close(a, b, what, tol=1e-9):
    err = float((a - b).abs().max() / b.abs().max().clamp_min(1e-300))
    assert err <= tol, f"{what}: rel-err {err:.3e}"


@pytest.mark.parametrize("states", [False, True])
@pytest.mark.parametrize("L", [16, 32])
def test_equals_autograd_for_a_scale_invariant_loss(states, L):
    B, NH, S, DQK, DV = 1, 2, 64, 8, 12
    x, st = _inputs(B, NH, S, DQK, DV, seed=3 + L + states, states=states)
    xs = [t.clone().requires_grad_(True) for t in x]
    sts = [t.clone().requires_grad_(True) for t in st] if states else [None, None, None]
    h, n_out, m_out, _, _ = om.mlstm_chunkwise_fw(*xs, *sts, chunk_size=L)
    # the exact-branch premise of the test itself
    assert bool((n_out > torch.exp(-m_out) * 1.01).all())
    W = torch.randn(h.shape, generator=torch.Generator().manual_seed(99), dtype=F64)
    loss = _direction_loss(h, W)
    grads = torch.autograd.grad(loss, xs + [t for t in sts if t is not None])
    hh = h.detach().requires_grad_(True)
    dH = torch.autograd.grad(_direction_loss(hh, W), hh)[0]
    got = om.mlstm_chunkwise_bw(*x, dH, *(st or (None, None, None)), chunk_size=L)
    names = ["dq", "dk", "dv", "di", "df"]
    for nm, a, b in zip(names, got[:5], grads[:5]):
        _close(a, b, nm)
    if states:
        _close(got[5], grads[5], "dc0")
        assert float(grads[6].abs().max()) < 1e-12  # n0 only enters the divisor: zero, as the reference returns
        assert torch.equal(got[6], torch.zeros_like(st[1]))


def test_last_state_path():
    """Loss <G, C_last exp(m_last)>: dk, dv, di, dc0 equal autograd's, dq is zero, and df equals
    autograd's minus <G, C_true> sigmoid(-f)."""
    B, NH, S, DQK, DV, L = 1, 2, 48, 6, 5, 16
    x, st = _inputs(B, NH, S, DQK, DV, seed=11, states=True)
    xs = [t.clone().requires_grad_(True) for t in x]
    sts = [t.clone().requires_grad_(True) for t in st]
    _, _, _, (C, n, m), _ = om.mlstm_chunkwise_fw(*xs, *sts, return_last_states=True, chunk_size=L)
    G = torch.randn(C.shape, generator=torch.Generator().manual_seed(5), dtype=F64)
    C_true = C * torch.exp(m)[..., None]
    loss = (G * C_true).sum()
    grads = torch.autograd.grad(loss, xs + [sts[0]], allow_unused=True)  # q does not reach C_last
    dC_last = (G * torch.exp(m)[..., None]).detach()
    got = om.mlstm_chunkwise_bw(*x, torch.zeros(B, NH, S, DV, dtype=F64), *st, matDeltaC_last=dC_last, chunk_size=L)
    assert float(got[0].abs().max()) == 0.0
    for nm, a, b in (("dk", got[1], grads[1]), ("dv", got[2], grads[2]), ("di", got[3], grads[3]),
                     ("dc0", got[5], grads[5])):
        _close(a, b, nm)
    const = (G * C_true.detach()).sum(dim=(-2, -1))[..., None]  # (B, NH, 1)
    _close(got[4] + const * torch.sigmoid(-x[4]), grads[4], "df + <G, C_true> sigmoid(-f)")
    # and the constant is not negligible here: without it df is far off
    assert float((got[4] - grads[4]).abs().max()) > 1e-3


def test_chunk_size_invariant():
    B, NH, S, DQK, DV = 2, 1, 64, 8, 8
    x, st = _inputs(B, NH, S, DQK, DV, seed=21, states=True)
    dH = torch.randn(B, NH, S, DV, generator=torch.Generator().manual_seed(1), dtype=F64)
    dCl = torch.randn(B, NH, DQK, DV, generator=torch.Generator().manual_seed(2), dtype=F64)
    a = om.mlstm_chunkwise_bw(*x, dH, *st, matDeltaC_last=dCl, chunk_size=16)
    b = om.mlstm_chunkwise_bw(*x, dH, *st, matDeltaC_last=dCl, chunk_size=64)
    for nm, u, w in zip(["dq", "dk", "dv", "di", "df", "dc0"], a[:6], b[:6]):
        _close(u, w, nm, tol=1e-10)


@pytest.mark.parametrize("S,pad", [(64, 64), (128, 32), (64, 48)])
def test_state_preserving_padding(S, pad):
    """Tokens with input gate -3e4 and forget gate +30 appended to a sequence change none of the
    custom backward's gradients of the original tokens (nor dc0), with the last-state gradient
    on: the padding the GPU backward uses for a ragged sequence (xlstm_hip.ops._PAD_I, _PAD_F)."""
    from xlstm_hip.ops import _PAD_F, _PAD_I
    B, NH, DQK, DV = 2, 1, 8, 8
    x, st = _inputs(B, NH, S, DQK, DV, seed=31 + pad, states=True)
    g = torch.Generator().manual_seed(3)
    dH = torch.randn(B, NH, S, DV, generator=g, dtype=F64)
    dCl = torch.randn(B, NH, DQK, DV, generator=g, dtype=F64)
    want = om.mlstm_chunkwise_bw(*x, dH, *st, matDeltaC_last=dCl, chunk_size=64)
    q, k, v, i, f = x
    padz = lambda t: torch.nn.functional.pad(t, (0, 0, 0, pad))
    xp = (padz(q), padz(k), padz(v), torch.nn.functional.pad(i, (0, pad), value=_PAD_I),
          torch.nn.functional.pad(f, (0, pad), value=_PAD_F))
    T = S + pad
    Lp = 64 if T % 64 == 0 else (32 if T % 32 == 0 else (16 if T % 16 == 0 else 1))
    if T % 16:
        pytest.skip("padded length must be a whole number of 16-token chunks")
    got = om.mlstm_chunkwise_bw(*xp, padz(dH), *st, matDeltaC_last=dCl, chunk_size=Lp)
    for nm, u, w in zip(["dq", "dk", "dv", "di", "df"], got[:5], want[:5]):
        _close(u[:, :, :S], w, nm, tol=1e-10)
    _close(got[5], want[5], "dc0", tol=1e-10)


def _round24(x):
    """The fused bf16 path's packed states (csrc/chunkwise_bwd.hip pack24): the upper 24 bits of
    each float32, rounded to nearest by adding half of the dropped byte."""
    a = x.to(torch.float32).contiguous().view(torch.int32)
    return ((a + 0x80) & -256).view(torch.float32).to(x.dtype)


def test_packed_state_rounding():
    """The GPU backward's fused path keeps the per-chunk C and dC as their upper 24 bits.  In
    float64 that moves every gradient by far less than the GPU tests' bar (2e-3 of the largest
    value beyond one output rounding), while bf16 states (8 significant bits) move dF past it:
    the packed format's precision is a measured choice, not a free one."""
    B, NH, S, DQK, DV, L = 1, 1, 512, 128, 128, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, NH, S, DQK, generator=g, dtype=F64)
    k = torch.randn(B, NH, S, DQK, generator=g, dtype=F64)
    v = torch.randn(B, NH, S, DV, generator=g, dtype=F64)
    i = torch.randn(B, NH, S, generator=g, dtype=F64)
    f = torch.randn(B, NH, S, generator=g, dtype=F64) + 3.0
    dH = torch.randn(B, NH, S, DV, generator=g, dtype=F64)
    want = om.mlstm_chunkwise_bw(q, k, v, i, f, dH, chunk_size=L)
    p24 = om.mlstm_chunkwise_bw(q, k, v, i, f, dH, chunk_size=L, state_round=_round24)
    bf16 = om.mlstm_chunkwise_bw(q, k, v, i, f, dH, chunk_size=L,
                                 state_round=lambda t: t.to(torch.bfloat16).to(t.dtype))
    rel = lambda a, b: float((a - b).abs().max() / b.abs().max())
    for nm, u, w in zip(["dq", "dk", "dv", "di", "df"], p24[:5], want[:5]):
        assert rel(u, w) <= 1e-4, f"{nm}: packed states move it by {rel(u, w):.2e} of its max"
    assert max(rel(u, w) for u, w in zip(bf16[:5], want[:5])) > 2e-3
