"""Logit projection + soft-cap kernel (lm_head_softcap) on the GPU.

The reference computes soft_cap(lm_head(x), 30) (xlstm_metal/torch_native/models/
wired_xlstm.py:176, generate.py:131): the Linear's output in the model dtype, then
30 tanh(z / 30).  The expected values here are F.linear in float64 and the soft-cap in float64:

* exact form: y64 = cap tanh(z64 / cap), no rounding at all;
* reference form: yr = bf16(cap tanh(bf16(z64) / cap)), the reference's two roundings.

Bars (16-bit output): |y - yr| <= ulp(yr) + ulp(z64) sech^2((|z64| - ulp(z64)) / cap) + cap 1e-6:
the output's own rounding on both sides (half an ulp each), the change one flipped rounding of z
makes after the soft-cap (float32 accumulation against float64 can land z on the other side of a
rounding boundary; sech^2 taken at the smaller end of that ulp), and the kernel's tanh, formed
from the hardware exp2 and reciprocal, within 5e-7 absolute (so cap 5e-7 on y); the same bound
against the exact form y64.

Shapes: config 3's decode step (1 token, D 4096, vocab 50304; 4 tokens), config 4's (8 tokens, D 2048),
the most token rows the kernel stages (16 at D 4096: 131 KB of LDS), a vocabulary that is not a
multiple of 16 or of a workgroup's 128 rows, D not a multiple of 32 (200) and below one k-step
(8), fewer vocabulary rows than the row form has waves (7), f16, no cap (cap 0: the plain Linear), and weights scaled so that z reaches far into the
cap's saturation.  More than 16 rows take the Linear + soft_cap path, under the same bar.
"""

import pytest
import torch

from helpers import dev

pytestmark = pytest.mark.gpu


def _ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    mant = 7 if dtype == torch.bfloat16 else 10
    return torch.exp2(torch.floor(torch.log2(x.abs().clamp_min(1e-30))) - mant)


def _inputs(M, D, V, dtype, w_std, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).to(dtype)  # RMS-normalised rows
    w = (w_std * torch.randn(V, D, generator=g)).to(dtype)
    return x, w


def _check(y, x, w, cap, what):
    z64 = x.double() @ w.double().t()
    yd = y.double().cpu()
    if cap > 0:
        y64 = cap * torch.tanh(z64 / cap)
        yr = (cap * torch.tanh(z64.to(y.dtype).double() / cap)).to(y.dtype).double()
        uz = _ulp(z64, y.dtype)
        flip = uz / torch.cosh((z64.abs() - uz).clamp_min(0) / cap) ** 2
        slack = cap * 1e-6
    else:
        y64, yr, flip, slack = z64, z64.to(y.dtype).double(), _ulp(z64, y.dtype), 1e-6
    ex_ref = float((((yd - yr).abs()) - _ulp(yr, y.dtype) - flip).max())
    ex_exact = float((((yd - y64).abs()) - _ulp(y64, y.dtype) - flip).max())
    assert ex_ref <= slack, f"{what}: {ex_ref:.3e} beyond the bar against the reference's roundings"
    assert ex_exact <= slack, f"{what}: {ex_exact:.3e} beyond the bar against float64"
    if cap > 0:
        assert float(yd.abs().max()) <= cap


@pytest.mark.parametrize("M,D,V,w_std", [(1, 4096, 50304, 0.02), (8, 2048, 50304, 0.02), (1, 4096, 50304, 0.6),
                                         (16, 4096, 50304, 0.3), (13, 512, 4099, 0.3), (3, 200, 1000, 1.0),
                                         (16, 1024, 2048, 0.5), (5, 8, 37, 4.0), (2, 2048, 3001, 0.3),
                                         (4, 4096, 50304, 0.02), (1, 1024, 7, 0.5)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_vs_float64(gpu_case, M, D, V, w_std, dtype):
    import xlstm_hip
    x, w = _inputs(M, D, V, dtype, w_std, seed=M * 7 + D + V)
    y = xlstm_hip.lm_head_softcap(x.to(dev()), w.to(dev()), 30.0)
    assert y.shape == (M, V) and y.dtype == dtype
    _check(y, x, w, 30.0, f"M{M} D{D} V{V} std{w_std} {dtype}")


def test_no_cap_is_the_linear(gpu_case):
    import xlstm_hip
    x, w = _inputs(3, 256, 300, torch.bfloat16, 1.0, seed=5)
    y = xlstm_hip.lm_head_softcap(x.to(dev()), w.to(dev()), 0.0)
    _check(y, x, w, 0.0, "cap 0")
    assert float(y.float().abs().max()) > 30  # not capped


def test_leading_dims_and_the_unfused_path(gpu_case):
    """[B, 1, D] rows as the decode step passes them; more than 16 rows take the Linear + soft_cap
    path, which the same bar covers."""
    import xlstm_hip
    x, w = _inputs(8, 512, 1024, torch.bfloat16, 0.5, seed=6)
    y = xlstm_hip.lm_head_softcap(x.view(8, 1, 512).to(dev()), w.to(dev()), 30.0)
    assert y.shape == (8, 1, 1024)
    _check(y.view(8, 1024), x, w, 30.0, "[8, 1, D]")
    for rows in (17, 70):
        x2, _ = _inputs(rows, 512, 1, torch.bfloat16, 1.0, seed=rows)
        y2 = xlstm_hip.lm_head_softcap(x2.to(dev()), w.to(dev()), 30.0)
        _check(y2, x2, w, 30.0, f"{rows} rows (Linear + soft_cap)")


def test_stack_logits_fused_vs_linear(gpu_case):
    """The config-3 stack's lm_head: the fused kernel against torch's Linear then soft_cap on the
    same normalised rows (both within the bar of the float64 form above, so within two of it of
    each other)."""
    from xlstm_hip.stack import CFG3_STACK, xLSTMStack
    import dataclasses
    cfg = dataclasses.replace(CFG3_STACK, num_blocks=1)
    model = xLSTMStack.random(cfg, dev(), seed=3)
    g = torch.Generator(device=dev()).manual_seed(4)
    xb = torch.randn(1, 1, cfg.d_model, generator=g, device=dev()).to(cfg.dtype)
    with torch.no_grad():
        fused = model.logits(xb)
        model.fused_lm_head = False
        plain = model.logits(xb)
        xn = model.out_norm(xb).view(1, -1).cpu()
    w = model.lm_head.weight.detach().cpu()
    _check(fused.view(1, -1), xn, w, cfg.logit_soft_cap, "fused")
    _check(plain.view(1, -1), xn, w, cfg.logit_soft_cap, "Linear")


def test_rejects(gpu_case):
    import xlstm_hip
    from xlstm_hip import ops
    x = torch.randn(17, 64, device=dev(), dtype=torch.bfloat16)
    w = torch.randn(128, 64, device=dev(), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="at most 16"):
        ops.lm_head_softcap_op(x, w, 30.0)
    with pytest.raises(ValueError):
        xlstm_hip.lm_head_softcap(x[:4], w[:, :32], 30.0)
