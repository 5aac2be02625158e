"""Pins the CPU oracle of the mLSTM output cell's multi-head RMSNorm x sigmoid(o) (no GPU).

The reference has no tests of its own for these modules.  The oracle (numpy, float64) is held
to torch's CPU ``F.rms_norm`` in float64 (a library routine, not the formula retyped), to the
closed forms of a constant head and of the output's root mean square, to ``math.exp`` for the
gate, and to torch's bf16 type promotion of the reference's own expression (which fixes where
the 16-bit roundings fall) within one bf16 ulp.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mlstm_layers as oml


@pytest.mark.parametrize("B,NH,S,DH", [(2, 3, 5, 16), (1, 4, 7, 64), (1, 1, 3, 5)])
@pytest.mark.parametrize("eps", [1e-6, 1e-3])
def test_norm_matches_torch_rms_norm(B, NH, S, DH, eps):
    g = torch.Generator().manual_seed(B * NH + S + DH)
    h = torch.randn(B, NH, S, DH, generator=g, dtype=torch.float64) * 3
    want = F.rms_norm(h.permute(0, 2, 1, 3), (DH,), eps=eps).reshape(B, S, NH * DH).numpy()
    np.testing.assert_allclose(oml.mh_rmsnorm_gate(h, eps=eps), want, rtol=1e-12, atol=1e-14)
    # the same in the [B, S, NH, DH] layout
    got = oml.mh_rmsnorm_gate(h.permute(0, 2, 1, 3).contiguous(), eps=eps, heads_first=False)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-14)


def test_weight_and_gate_closed_forms():
    B, NH, S, DH = 1, 2, 3, 4
    h = np.full((B, NH, S, DH), -2.5)
    h[0, 1] = 0.75
    y = oml.mh_rmsnorm_gate(h, eps=0.0)
    assert np.array_equal(y[0, :, :DH], np.full((S, DH), -1.0)) and np.array_equal(y[0, :, DH:], np.ones((S, DH)))
    w = np.arange(1, NH * DH + 1, dtype=np.float64)
    o = np.linspace(-6, 6, B * S * NH * DH).reshape(B, S, NH * DH)
    yg = oml.mh_rmsnorm_gate(h, w, o, eps=0.0)
    for idx in np.ndindex(yg.shape):
        c = idx[2]
        sign = -1.0 if c < DH else 1.0
        assert math.isclose(yg[idx], sign * w[c] / (1.0 + math.exp(-o[idx])), rel_tol=1e-14)


def test_output_rms_with_eps():
    rng = np.random.default_rng(4)
    h = rng.normal(size=(2, 3, 6, 32))
    eps = 0.05
    y = oml.mh_rmsnorm_gate(h, eps=eps).reshape(2, 6, 3, 32)
    ms = (h.transpose(0, 2, 1, 3) ** 2).mean(axis=-1)
    np.testing.assert_allclose((y ** 2).mean(axis=-1), ms / (ms + eps), rtol=1e-12)


def test_bf16_roundings_match_torch_promotion():
    """The reference's expressions evaluated by torch in bf16 (its own promotion and rounding
    rules) agree with the oracle's explicit roundings within one bf16 ulp."""
    g = torch.Generator().manual_seed(9)
    B, NH, S, DH = 2, 2, 9, 32
    h = torch.randn(B, NH, S, DH, generator=g).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(NH * DH, generator=g)).to(torch.bfloat16)
    o = torch.randn(B, S, NH * DH, generator=g).to(torch.bfloat16)
    x = h.permute(0, 2, 1, 3)
    rms = torch.sqrt((x.float() ** 2).mean(dim=-1, keepdim=True) + 1e-6)
    ref = ((x / rms).type_as(x).reshape(B, S, -1) * w) * torch.sigmoid(o)
    got = torch.from_numpy(oml.mh_rmsnorm_gate(h, w, o)).to(torch.bfloat16).double()
    ref = ref.double()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    assert bool(((got - ref).abs() <= ulp).all())


def test_gate_proj_matches_torch_linear_and_tanh():
    """float64: the oracle is torch's F.linear followed by the soft-cap closed form with math.tanh."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(3, 5, 40, generator=g, dtype=torch.float64)
    w = torch.randn(6, 40, generator=g, dtype=torch.float64)
    b = torch.randn(6, generator=g, dtype=torch.float64)
    lin = F.linear(x, w, b).numpy()
    got = oml.gate_proj_softcap(x, w, b, 15.0)
    for idx in np.ndindex(got.shape):
        assert math.isclose(got[idx], 15.0 * math.tanh(lin[idx] / 15.0), rel_tol=1e-12, abs_tol=1e-15)
    np.testing.assert_allclose(oml.gate_proj_softcap(x, w, None, 0.0), F.linear(x, w).numpy(), rtol=1e-12)


def test_gate_proj_bf16_linear_rounding_matches_torch():
    """The Linear's output is rounded to bf16 before the soft-cap, as torch's bf16 F.linear returns it
    (within one bf16 ulp of torch, whose summation order differs)."""
    g = torch.Generator().manual_seed(22)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    w = (0.3 * torch.randn(8, 256, generator=g)).to(torch.bfloat16)
    b = torch.randn(8, generator=g).to(torch.bfloat16)
    lin = F.linear(x, w, b).double()
    got = torch.from_numpy(oml.gate_proj_softcap(x, w, b, 0.0))
    ulp = torch.exp2(torch.floor(torch.log2(lin.abs().clamp_min(1e-30))) - 7)
    assert bool(((got - lin).abs() <= ulp).all())


def test_gate_proj_softcap_in_dtype_matches_torch_bf16_expression():
    """cap_in_dtype: the sLSTM projection cell's ``cap * torch.tanh(x / cap)`` with cap a tensor of
    x's dtype (slstm_projection_cell.py:84-89), evaluated by torch on bf16 tensors, equals the
    oracle's per-operation roundings bit for bit except where torch's float32 tanh and the
    float64 one round to different bf16 neighbours (one ulp, rarely); and the three roundings are
    really there: the float64 soft-cap rounded once differs on many inputs."""
    g = torch.Generator().manual_seed(23)
    x = torch.eye(512, dtype=torch.bfloat16)
    w = (40 * torch.randn(512, 512, generator=g)).to(torch.bfloat16)  # outputs = the rows of w
    z = F.linear(x, w).double()
    got = torch.from_numpy(oml.gate_proj_softcap(x, w, None, 15.0, cap_in_dtype=True)).to(torch.bfloat16).double()
    cap_t = torch.tensor(15.0, dtype=torch.bfloat16)
    want = (cap_t * torch.tanh(F.linear(x, w) / cap_t)).double()
    ulp = torch.exp2(torch.floor(torch.log2(want.abs().clamp_min(1e-30))) - 7)
    diff = (got - want).abs()
    assert bool((diff <= ulp).all())
    assert float((diff > 0).double().mean()) < 0.01
    once = torch.from_numpy(oml.gate_proj_softcap(x, w, None, 15.0)).to(torch.bfloat16).double()
    assert float((once != want).double().mean()) > 0.05
    assert bool((z.abs() > 15).any())
