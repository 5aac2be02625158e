"""Gate projection + soft-cap kernel on the GPU vs the CPU oracle, and the projection cells using it.

Shapes cover one to four 16-column output tiles (G 1 .. 64, ragged), D a multiple of 32 and not
(40), M not a multiple of 16, config 4's sLSTM i/f gates (D 2048, G 8) and the 7B mLSTM cell's
(D 4096, G 16); the row-streaming form (D a multiple of 512, G x D / 512 x 4 registers of weight
slices at most 128) takes D 2048 with G 8 and 4, D 512 with G 16 and D 1024 with G 2 (fewer rows
than it has waves).  Bar: 16-bit max-abs 2e-2 beyond two roundings of the output (its own and the
Linear's output rounding before the soft-cap, which the reference applies and a different
summation order can move by one ulp); with the sLSTM cell's soft-cap in the dtype, beyond four
(z / cap and tanh are rounded too).
"""

import pytest
import torch

from helpers import assert_parity, dev, relerr
from oracle import mlstm_layers as oml
from oracle import slstm as osl_cell
from oracle import slstm_layers as osl

pytestmark = pytest.mark.gpu


def _inputs(M, D, G, dtype, seed, with_bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).to(dtype)
    w = (4 * torch.randn(G, D, generator=g) / D ** 0.5).to(dtype)  # outputs ~N(0, 16): across the cap
    b = torch.randn(G, generator=g).to(dtype) if with_bias else None
    return x, w, b


@pytest.mark.parametrize("M,D,G", [(1000, 2048, 8), (300, 2048, 4), (77, 4096, 16), (5, 64, 3), (33, 40, 64),
                                   (1, 8, 1), (129, 512, 17), (64, 1024, 48), (100, 512, 16), (3, 1024, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cap,in_dtype", [(15.0, False), (15.0, True), (0.0, False)])
def test_vs_oracle(gpu_case, M, D, G, dtype, cap, in_dtype):
    """in_dtype (the sLSTM cell's soft-cap, each operation rounded): the bar counts the two more
    16-bit roundings (z / cap and tanh) that a different tanh or summation order can flip."""
    import xlstm_hip
    x, w, b = _inputs(M, D, G, dtype, seed=M + D + G, with_bias=(M % 2 == 0))
    y = xlstm_hip.gate_proj_softcap(x.to(dev()), w.to(dev()), None if b is None else b.to(dev()), cap,
                                    cap_in_dtype=in_dtype)
    want = torch.from_numpy(oml.gate_proj_softcap(x, w, b, cap, cap_in_dtype=in_dtype))
    assert y.shape == (M, G) and y.dtype == dtype
    assert_parity(y.cpu(), want, dtype, f"gate_proj {M, D, G} {dtype} cap={cap} in_dtype={in_dtype}",
                  roundings=4 if in_dtype else 2)


def test_rejections(gpu_case):
    from xlstm_hip.ops import gate_proj_softcap_op
    x = torch.randn(4, 64, device=dev())
    with pytest.raises(NotImplementedError, match="float32"):
        gate_proj_softcap_op(x, torch.randn(4, 64, device=dev()), None, 15.0)
    xb = x.to(torch.bfloat16)
    with pytest.raises(NotImplementedError, match="at most 64"):
        gate_proj_softcap_op(xb, torch.randn(65, 64, device=dev()).to(torch.bfloat16), None, 15.0)
    with pytest.raises(NotImplementedError, match="multiple of 8"):
        gate_proj_softcap_op(xb[:, :12].contiguous(), torch.randn(4, 12, device=dev()).to(torch.bfloat16), None, 0.0)


def test_mlstm_projection_cell_bf16(gpu_case):
    """mLSTMProjectionCell (7B-like gates: D 4096 -> 2 x NH 8) in bf16: q, k, v are its Linear layers,
    the gates match the oracle on the stacked gate weights; fp32 matches torch's composition."""
    import xlstm_hip
    torch.manual_seed(1)
    B, S, D, NH = 2, 50, 4096, 8
    cell = xlstm_hip.mLSTMProjectionCell(D, NH, 64, 128, gate_soft_cap=15.0)
    with torch.no_grad():
        for lin in (cell.igate_proj, cell.fgate_proj):
            lin.weight.mul_(40.0)  # gate pre-activations across the cap
    x = torch.randn(B, S, D)
    cell_b = cell.to(torch.bfloat16).to(dev())
    q, k, v, i, f = cell_b(x.to(torch.bfloat16).to(dev()))
    assert q.shape == (B, NH, S, 64) and v.shape == (B, NH, S, 128) and i.shape == (B, NH, S)
    xb = x.to(torch.bfloat16)
    for got, lin in ((i, cell_b.igate_proj), (f, cell_b.fgate_proj)):
        want = oml.gate_proj_softcap(xb, lin.weight.cpu(), lin.bias.cpu(), 15.0)
        assert_parity(got.permute(0, 2, 1).cpu(), torch.from_numpy(want), torch.bfloat16, "mLSTM gate", roundings=2)
    cell_f = cell.float()
    with torch.no_grad():
        i32 = cell_f(x.to(dev()))[3].cpu()
        ref = osl_cell.soft_cap(torch.nn.functional.linear(x, cell_f.igate_proj.weight.cpu(),
                                                           cell_f.igate_proj.bias.cpu()), 15.0).permute(0, 2, 1)
    assert relerr(i32, ref) <= 1e-4


def test_slstm_projection_cell_bf16(gpu_case):
    """sLSTMProjectionCell at config 4's widths (d_model 2048, NH 4) in bf16: i and f from the conv
    output and o from the input, each against the oracle (conv + SiLU oracle rounded to bf16, then
    the gate oracle)."""
    import xlstm_hip
    torch.manual_seed(2)
    B, S, D, NH = 2, 64, 2048, 4
    cell = xlstm_hip.sLSTMProjectionCell(D, NH, 512)
    with torch.no_grad():
        for lin in (cell.igate_proj, cell.fgate_proj, cell.ogate_proj):
            lin.weight.mul_(40.0)
    cell = cell.to(torch.bfloat16).to(dev())
    x = torch.randn(B, S, D).to(torch.bfloat16)
    z, i, f, o, xc = cell(x.to(dev()))
    xc_want = osl.causal_conv1d(x, cell.conv1d.conv.weight.cpu(), cell.conv1d.conv.bias.cpu(), activation="silu")
    assert_parity(xc.cpu(), torch.from_numpy(xc_want), torch.bfloat16, "x_conv")
    for got, lin, src in ((i, cell.igate_proj, xc.cpu()), (f, cell.fgate_proj, xc.cpu()), (o, cell.ogate_proj, x)):
        # the reference soft-caps with bf16 torch ops (slstm_projection_cell.py:84-89)
        want = oml.gate_proj_softcap(src, lin.weight.cpu(), lin.bias.cpu(), 15.0, cap_in_dtype=True)
        assert got.shape == (B, S, NH)
        assert_parity(got.cpu(), torch.from_numpy(want), torch.bfloat16, "sLSTM gate", roundings=4)
