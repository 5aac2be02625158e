"""Pins the CPU oracle of the sLSTM layer's causal conv1d + SiLU and per-head GroupNorm (no GPU).

The reference has no tests of its own for these two modules; its CPU path is torch's
``nn.Conv1d`` after a left pad (``causal_conv1d.py:51-67``) and ``nn.GroupNorm``
(``slstm_output_cell.py:53,72-83``).  The oracle is numpy float64 code of its own; these
tests hold it to torch's CPU functions in float64, to the impulse response (a flipped tap
order fails it), to K = 1 (an affine map), to torch's own bf16 modules within one bf16 ulp,
and to the moments of the normalised output.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import slstm_layers as osl


def _torch_causal_conv(x_bsd, w_dk, b, act):
    """The reference module's CPU computation on [B, S, D]: permute, pad K - 1, depthwise conv."""
    D, K = w_dk.shape
    xc = F.pad(x_bsd.permute(0, 2, 1), (K - 1, 0))
    y = F.conv1d(xc, w_dk.reshape(D, 1, K), b, groups=D)
    if act:
        y = F.silu(y)
    return y.permute(0, 2, 1)


@pytest.mark.parametrize("B,S,D,K", [(2, 9, 5, 4), (1, 3, 7, 4), (3, 17, 4, 1), (1, 12, 6, 3), (2, 5, 3, 7)])
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("act", [None, "silu"])
def test_conv_matches_torch_conv1d_float64(B, S, D, K, with_bias, act):
    g = torch.Generator().manual_seed(B * 100 + S * 10 + K)
    x = torch.randn(B, S, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, K, generator=g, dtype=torch.float64)
    b = torch.randn(D, generator=g, dtype=torch.float64) if with_bias else None
    want = _torch_causal_conv(x, w, b, act == "silu").numpy()
    got = osl.causal_conv1d(x, w, b, activation=act)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_conv_impulse_response_fixes_tap_order():
    """A unit impulse at s = 0 comes out as the taps read backwards: y[s] = w[K - 1 - s]."""
    D, K, S = 3, 4, 7
    w = np.arange(1, D * K + 1, dtype=np.float64).reshape(D, K)
    x = np.zeros((1, S, D))
    x[0, 0, :] = 1.0
    y = osl.causal_conv1d(x, w)
    for s in range(S):
        want = w[:, K - 1 - s] if s < K else np.zeros(D)
        assert np.array_equal(y[0, s], want), (s, y[0, s], want)
    # a step at s = 2 leaves the first two outputs at the bias
    x2 = np.zeros((1, S, D))
    x2[0, 2:, :] = 1.0
    y2 = osl.causal_conv1d(x2, w, bias=np.full(D, 0.5))
    assert np.array_equal(y2[0, :2], np.full((2, D), 0.5))
    assert np.array_equal(y2[0, 2], w[:, K - 1] + 0.5)


def test_conv_k1_is_affine():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 6, 4, generator=g, dtype=torch.float64)
    w = torch.randn(4, 1, generator=g, dtype=torch.float64)
    b = torch.randn(4, generator=g, dtype=torch.float64)
    np.testing.assert_allclose(osl.causal_conv1d(x, w, b), (x * w[:, 0] + b).numpy(), rtol=0, atol=1e-15)


def test_silu_closed_form():
    vals = [-100.0, -20.0, -1.5, -1e-3, 0.0, 2e-3, 0.7, 3.0, 40.0]
    x = np.array(vals, dtype=np.float64).reshape(1, -1, 1)
    y = osl.causal_conv1d(x, np.ones((1, 1)), activation="silu")
    for v, got in zip(vals, y.reshape(-1)):
        assert math.isclose(got, v / (1.0 + math.exp(-v)), rel_tol=1e-14, abs_tol=1e-300)


@pytest.mark.parametrize("act", [None, "silu"])
def test_conv_bf16_semantics_match_torch_modules(act):
    """torch's CPU nn.Conv1d + nn.SiLU in bf16 (the reference run in bf16) agree with the oracle's
    rounding of the convolution before the SiLU to one bf16 ulp of the output."""
    g = torch.Generator().manual_seed(7)
    B, S, D, K = 2, 40, 24, 4
    x = torch.randn(B, S, D, generator=g).to(torch.bfloat16)
    w = (0.5 * torch.randn(D, K, generator=g)).to(torch.bfloat16)
    b = torch.randn(D, generator=g).to(torch.bfloat16)
    ref = _torch_causal_conv(x, w, b, act == "silu").to(torch.float64).numpy()
    got = osl.causal_conv1d(x, w, b, activation=act)
    got_bf16 = torch.from_numpy(got).to(torch.bfloat16).to(torch.float64).numpy()
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    assert np.all(np.abs(got_bf16 - ref) <= ulp + 1e-30)


@pytest.mark.parametrize("N,G,CG", [(5, 4, 8), (3, 1, 17), (7, 3, 64), (2, 8, 1)])
@pytest.mark.parametrize("affine", ["wb", "none", "w", "b"])
@pytest.mark.parametrize("eps", [1e-6, 1e-5])
def test_group_norm_matches_torch_float64(N, G, CG, affine, eps):
    g = torch.Generator().manual_seed(N * G + CG)
    x = 3 * torch.randn(N, G * CG, generator=g, dtype=torch.float64) + 1
    w = torch.randn(G * CG, generator=g, dtype=torch.float64) if "w" in affine else None
    b = torch.randn(G * CG, generator=g, dtype=torch.float64) if "b" in affine else None
    want = F.group_norm(x, G, w, b, eps).numpy()
    np.testing.assert_allclose(osl.group_norm(x, G, w, b, eps), want, rtol=1e-12, atol=1e-12)


def test_group_norm_moments_and_constant_groups():
    rng = np.random.default_rng(3)
    N, G, CG, eps = 4, 3, 50, 1e-6
    x = rng.normal(2.0, 5.0, size=(N, G * CG))
    y = osl.group_norm(x, G, eps=eps).reshape(N, G, CG)
    var = x.reshape(N, G, CG).var(axis=2)
    np.testing.assert_allclose(y.mean(axis=2), 0.0, atol=1e-13)
    np.testing.assert_allclose(y.var(axis=2), var / (var + eps), rtol=1e-12)
    # a constant group normalises to zero and comes out as the bias
    xc = np.full((1, G * CG), 4.25)
    w = rng.normal(size=G * CG)
    b = rng.normal(size=G * CG)
    assert np.array_equal(osl.group_norm(xc, G, w, b, eps)[0], b)
