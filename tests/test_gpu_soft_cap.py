"""soft_cap on the GPU vs the CPU oracle, the reference's known answers, and
torch float32 at full size (cfg3 logits, 50304 x 2048)."""

import json
import os

import pytest
import torch

from helpers import assert_parity, dev
from oracle import slstm as osl

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_known_answers(gpu_case):
    import xlstm_hip
    kat = json.load(open(os.path.join(GOLDEN, "kat.json")))
    for c in kat["soft_cap"]:
        y = xlstm_hip.soft_cap(torch.tensor([c["x"]], device=dev()), c["cap"]).cpu()
        assert abs(float(y[0]) - c["expect"]) < c["tol"], c
    for c in kat["soft_cap_cases"]:
        y = xlstm_hip.soft_cap(torch.tensor(c["x"], device=dev()), c["cap"]).cpu()
        torch.testing.assert_close(y.double(), torch.tensor(c["expect"], dtype=torch.float64), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("numel", [1, 7, 8, 4099, 1 << 20])
def test_vs_oracle(gpu_case, dtype, numel):
    import xlstm_hip
    g = torch.Generator().manual_seed(numel)
    x = (torch.randn(numel, generator=g) * 20).to(dtype)
    for cap in (15.0, 30.0):
        y = xlstm_hip.soft_cap(x.to(dev()), cap).cpu()
        want = osl.soft_cap(x.float(), cap)
        if dtype == torch.float32:
            assert_parity(y, want, dtype, f"soft_cap fp32 n={numel}")
        else:  # 16-bit output: within one rounding of the fp32 result
            tol = (want.abs() * (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11)).clamp_min(1e-6)
            assert bool(((y.float() - want).abs() <= tol).all())


def test_identity_and_offset_views(gpu_case):
    import xlstm_hip
    x = torch.randn(1000, device=dev())
    assert xlstm_hip.soft_cap(x, 0.0) is x
    v = x[3:]  # misaligned view is handled
    torch.testing.assert_close(xlstm_hip.soft_cap(v, 5.0), 5.0 * torch.tanh(v / 5.0), rtol=1e-5, atol=1e-6)
    cell = xlstm_hip.SoftCapCell(15.0)
    torch.testing.assert_close(cell(x), 15.0 * torch.tanh(x / 15.0), rtol=1e-5, atol=1e-6)


def test_full_size_logits_bf16(gpu_case):
    import xlstm_hip
    g = torch.Generator(device=dev()).manual_seed(3)
    x = (torch.randn(2048, 50304, device=dev(), generator=g) * 40).to(torch.bfloat16)
    y = xlstm_hip.soft_cap(x, 30.0)
    want = (30.0 * torch.tanh(x.float() / 30.0))
    err = ((y.float() - want).abs() - want.abs() * 2.0 ** -8).max().item()
    assert err <= 1e-6
    assert float(y.float().abs().max()) <= 30.0
