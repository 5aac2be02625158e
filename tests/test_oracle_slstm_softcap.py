"""Pins the CPU oracle of the sLSTM step and the soft-cap (no GPU).

* soft-cap: the known answers of the reference's
  ``kernel_development/soft_cap/mlx_fast_kernels/test_softcap.py:6-56`` and
  the input cases of ``tests/parity/test_numerical_parity.py:104-108``,
  stored in ``tests/golden/kat.json``; cap <= 0 is the identity
  (``softcap.py:27-28``).
* sLSTM step: scalar closed forms evaluated with ``math`` (independent of
  torch), on the shapes and seeds the reference's
  ``tests/test_slstm_metal_kernel.py:110-314`` uses (2,4,8 / zero state /
  gates at +-10 with states x100 / 5 chained steps).
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import slstm as osl

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _kat():
    with open(os.path.join(GOLDEN, "kat.json")) as fh:
        return json.load(fh)


def test_soft_cap_known_answers():
    for c in _kat()["soft_cap"]:
        y = osl.soft_cap(torch.tensor([c["x"]], dtype=torch.float32), c["cap"])
        assert abs(float(y[0]) - c["expect"]) < c["tol"], c


def test_soft_cap_cases():
    for c in _kat()["soft_cap_cases"]:
        y = osl.soft_cap(torch.tensor(c["x"], dtype=torch.float64), c["cap"])
        np.testing.assert_allclose(y.numpy(), c["expect"], rtol=1e-14, atol=1e-14)


def test_soft_cap_nonpositive_cap_is_identity():
    x = torch.randn(17)
    assert osl.soft_cap(x, 0.0) is x
    assert osl.soft_cap(x, -3.0) is x


def _lsig(x):
    return -math.log1p(math.exp(-x)) if x > -30 else x - math.log1p(math.exp(x))


def _scalar_step(z, i, f, o, c, n, m, eps):
    lsf = _lsig(f)
    m2 = max(m + lsf, i)
    ig = math.exp(i - m2)
    fg = math.exp(m + lsf - m2)
    og = 1.0 / (1.0 + math.exp(-o))
    c2 = [fg * cc + ig * math.tanh(zz) for cc, zz in zip(c, z)]
    n2 = [fg * nn + ig for nn in n]
    h = [og * cc / (abs(nn) + eps) for cc, nn in zip(c2, n2)]
    return h, c2, n2, m2


def _check_against_scalar(z, i, f, o, c, n, m, eps=1e-6, steps=1):
    B, NH, H = c.shape
    zt = z if steps > 1 else z[:, None]
    it = i if steps > 1 else i[:, None]
    ft = f if steps > 1 else f[:, None]
    ot = o if steps > 1 else o[:, None]
    hc, (cc, nc, mc) = osl.slstm_sequence(zt, it, ft, ot, state=(c, n, m), eps=eps)
    for b in range(B):
        for h in range(NH):
            cs, ns, ms = c[b, h].tolist(), n[b, h].tolist(), float(m[b, h])
            for t in range(zt.shape[1]):
                hs, cs, ns, ms = _scalar_step(zt[b, t, h].tolist(), float(it[b, t, h]), float(ft[b, t, h]),
                                              float(ot[b, t, h]), cs, ns, ms, eps)
                np.testing.assert_allclose(hc[b, t, h].numpy(), hs, rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(cc[b, h].numpy(), cs, rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(nc[b, h].numpy(), ns, rtol=1e-12, atol=1e-12)
            assert abs(float(mc[b, h]) - ms) < 1e-12


def test_slstm_step_random_state():
    g = torch.Generator().manual_seed(42)
    B, NH, H = 2, 4, 8
    z, = (torch.randn(B, NH, H, generator=g, dtype=torch.float64),)
    i, f, o = (torch.randn(B, NH, generator=g, dtype=torch.float64) for _ in range(3))
    c = torch.randn(B, NH, H, generator=g, dtype=torch.float64)
    n = torch.randn(B, NH, H, generator=g, dtype=torch.float64).abs()
    m = torch.randn(B, NH, generator=g, dtype=torch.float64)
    _check_against_scalar(z, i, f, o, c, n, m)


def test_slstm_step_zero_state():
    g = torch.Generator().manual_seed(123)
    B, NH, H = 1, 2, 4
    z = torch.randn(B, NH, H, generator=g, dtype=torch.float64)
    i, f, o = (torch.randn(B, NH, generator=g, dtype=torch.float64) for _ in range(3))
    zero = torch.zeros(B, NH, H, dtype=torch.float64)
    _check_against_scalar(z, i, f, o, zero, zero.clone(), torch.zeros(B, NH, dtype=torch.float64))
    # closed form from zero state: h = sigmoid(o) tanh(z) ig / (ig + eps)
    h, c2, n2, m2 = osl.slstm_step(z, i, f, o, zero, zero, torch.zeros(B, NH, dtype=torch.float64))
    ig = torch.exp(i - m2)
    torch.testing.assert_close(n2, ig[..., None].expand_as(n2))
    torch.testing.assert_close(h, torch.sigmoid(o)[..., None] * torch.tanh(z) * ig[..., None] / (ig[..., None] + 1e-6))


@pytest.mark.parametrize("gate", [10.0, -10.0])
def test_slstm_step_extreme_gates(gate):
    g = torch.Generator().manual_seed(7)
    B, NH, H = 2, 4, 8
    z = torch.randn(B, NH, H, generator=g, dtype=torch.float64)
    full = torch.full((B, NH), gate, dtype=torch.float64)
    c = 100 * torch.randn(B, NH, H, generator=g, dtype=torch.float64)
    n = 100 * torch.randn(B, NH, H, generator=g, dtype=torch.float64).abs()
    m = torch.randn(B, NH, generator=g, dtype=torch.float64)
    _check_against_scalar(z, full, full, full, c, n, m)


def test_slstm_five_steps():
    g = torch.Generator().manual_seed(5)
    B, NH, H, S = 2, 4, 8, 5
    z = torch.randn(B, S, NH, H, generator=g, dtype=torch.float64)
    i, f, o = (torch.randn(B, S, NH, generator=g, dtype=torch.float64) for _ in range(3))
    zero = torch.zeros(B, NH, H, dtype=torch.float64)
    _check_against_scalar(z, i, f, o, zero, zero.clone(), torch.zeros(B, NH, dtype=torch.float64), steps=S)
