"""sLSTM layer stages on the GPU vs the CPU oracle: causal conv1d (+ SiLU) and per-head GroupNorm.

Shapes cover both access paths of each kernel (16-byte vectors when the channel count allows,
scalar otherwise), sequences shorter than the kernel and than one 16-step tile, every kernel
size 1..8, groups held in registers and groups streamed three times, and config 4's sLSTM
layer (d_model 2048, conv K = 4; NH 4 x H 512) on two of its eight batch rows.  Bars: float32
rel-err 1e-4; 16-bit max-abs 2e-2 beyond the output's own rounding, and for the conv no more
than one rounding (of the output, or of the pre-activation the kernel rounds before the SiLU as
the oracle does) from the oracle.
"""

import pytest
import torch

from helpers import assert_parity, dev, half_ulp, relerr
from oracle import slstm as osl_cell
from oracle import slstm_layers as osl

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _conv_inputs(B, S, D, K, dtype, seed, with_bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, D, generator=g).to(dtype)
    w = (0.5 * torch.randn(D, 1, K, generator=g)).to(dtype)
    b = torch.randn(D, generator=g).to(dtype) if with_bias else None
    return x, w, b


def _check_conv(y, x, w, b, act, dtype, what):
    want = torch.from_numpy(osl.causal_conv1d(x, w, b, activation=act, dtype=dtype))
    assert y.dtype == dtype and y.shape == x.shape
    assert_parity(y.cpu(), want, dtype, what)
    if dtype != torch.float32:
        # the same roundings as the oracle: the output within one ulp of it, plus one ulp of the
        # pre-activation rounding carried through the SiLU (slope <= 1.1) where the float32 sum of
        # the taps lands on the other side of a rounding boundary, plus 1e-6 for that sum (and for
        # results near zero, where float16 subnormals are 6e-8 apart)
        d = (y.cpu().double() - want).abs()
        tol = 3 * half_ulp(want, dtype) + 1e-6
        if act == "silu":
            a = torch.from_numpy(osl.causal_conv1d(x, w, b))
            tol = tol + 2.2 * half_ulp(a, dtype)
        assert bool((d <= tol).all()), f"{what}: more than one rounding from the oracle"


@pytest.mark.parametrize("B,S,D,K", [(2, 37, 96, 4), (1, 3, 40, 4), (3, 100, 2048, 4), (2, 50, 100, 4),
                                     (1, 19, 7, 3), (2, 33, 64, 1), (1, 40, 24, 8), (4, 16, 256, 5),
                                     (1, 1, 16, 2), (2, 29, 12, 6), (1, 23, 8, 7)])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("act", [None, "silu"])
def test_conv_vs_oracle(gpu_case, B, S, D, K, dtype, act):
    import xlstm_hip
    x, w, b = _conv_inputs(B, S, D, K, dtype, seed=B * S + D + K)
    y = xlstm_hip.causal_conv1d(x.to(dev()), w.to(dev()), b.to(dev()), activation=act)
    _check_conv(y, x, w, b, act, dtype, f"conv {B, S, D, K} {dtype} {act}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_conv_without_bias(gpu_case, dtype):
    import xlstm_hip
    x, w, _ = _conv_inputs(2, 45, 48, 4, dtype, seed=9, with_bias=False)
    y = xlstm_hip.causal_conv1d(x.to(dev()), w.to(dev()), None, activation="silu")
    _check_conv(y, x, w, None, "silu", dtype, f"conv no bias {dtype}")


def test_conv_cfg4_layer_rows(gpu_case):
    """Config 4's sLSTM projection conv (d_model 2048, K 4, bf16, SiLU) over S = 4096 for 2 batch rows."""
    import xlstm_hip
    x, w, b = _conv_inputs(2, 4096, 2048, 4, torch.bfloat16, seed=4)
    y = xlstm_hip.causal_conv1d(x.to(dev()), w.to(dev()), b.to(dev()), activation="silu")
    _check_conv(y, x, w, b, "silu", torch.bfloat16, "cfg4 conv")


def test_conv_module_layouts(gpu_case):
    """CausalConv1d.forward on [B, C, S]: a permuted view of channels-last memory and a contiguous
    [B, C, S] tensor both match the channels-last kernel call, and nn.Conv1d on the CPU."""
    import xlstm_hip
    torch.manual_seed(0)
    m = xlstm_hip.CausalConv1d(64, 64, 4, groups=64)
    x_bsd = torch.randn(3, 50, 64)
    want = osl.causal_conv1d(x_bsd, m.conv.weight, m.conv.bias)
    ref_cpu = m.conv(torch.nn.functional.pad(x_bsd.permute(0, 2, 1), (3, 0))).permute(0, 2, 1)
    assert relerr(ref_cpu, torch.from_numpy(want)) < 1e-6
    md = m.to(dev())
    y_view = md(x_bsd.to(dev()).permute(0, 2, 1))
    y_contig = md(x_bsd.permute(0, 2, 1).contiguous().to(dev()))
    assert y_view.shape == (3, 64, 50)
    assert torch.equal(y_view, y_contig)
    assert relerr(y_view.permute(0, 2, 1), torch.from_numpy(want)) <= 1e-4


def test_conv_rejections(gpu_case):
    import xlstm_hip
    from xlstm_hip import _lib
    x = torch.randn(1, 8, 16, device=dev())
    w = torch.randn(16, 9, device=dev())
    with pytest.raises(NotImplementedError, match="kernel size 9"):
        xlstm_hip.causal_conv1d(x, w)
    with pytest.raises(ValueError, match="share a dtype"):
        xlstm_hip.causal_conv1d(x, w[:, :4].to(torch.bfloat16))
    with pytest.raises(NotImplementedError, match="depthwise"):
        xlstm_hip.CausalConv1d(16, 16, 4, groups=1).to(dev())(x.permute(0, 2, 1))
    lib = _lib.load()
    w4 = torch.randn(16, 4, device=dev())
    rc = lib.xl_causal_conv1d_fwd(x.data_ptr(), w4.data_ptr(), None, x.data_ptr(), 1, 8, 16, 4, 1, 0, None)
    assert rc == -1 and b"alias" in lib.xl_last_error()


@pytest.mark.parametrize("N,G,CG", [(5, 4, 512), (7, 3, 64), (4, 2, 100), (3, 2, 4096), (2, 1, 16384),
                                    (1000, 8, 16), (6, 5, 3), (9, 4, 8)])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("affine", ["wb", "none", "w", "b"])
def test_group_norm_vs_oracle(gpu_case, N, G, CG, dtype, affine):
    import xlstm_hip
    g = torch.Generator().manual_seed(N + G + CG)
    x = (2 * torch.randn(N, G * CG, generator=g) + 3).to(dtype)
    w = torch.randn(G * CG, generator=g).to(dtype) if "w" in affine else None
    b = torch.randn(G * CG, generator=g).to(dtype) if "b" in affine else None
    y = xlstm_hip.group_norm(x.to(dev()), G, None if w is None else w.to(dev()), None if b is None else b.to(dev()),
                             1e-6)
    want = torch.from_numpy(osl.group_norm(x, G, w, b, 1e-6))
    assert y.dtype == dtype
    assert_parity(y.cpu(), want, dtype, f"group_norm {N, G, CG} {dtype} affine={affine}")


def test_group_norm_offset_and_constant_groups(gpu_case):
    """A mean far from zero (the variance is taken about the mean, not as E[x^2] - E[x]^2) and
    groups that are constant (normalised to zero: the output is the bias)."""
    import xlstm_hip
    g = torch.Generator().manual_seed(2)
    x = 100 + 0.1 * torch.randn(6, 4 * 256, generator=g)
    x[2, 256:512] = 7.0
    w, b = torch.randn(1024, generator=g), torch.randn(1024, generator=g)
    y = xlstm_hip.group_norm(x.to(dev()), 4, w.to(dev()), b.to(dev()), 1e-6).cpu()
    want = torch.from_numpy(osl.group_norm(x, 4, w, b, 1e-6))
    # float32 sums of 256 values near 100 leave ~1e-5 in the mean, ~1e-4 of the 0.1 spread; the
    # E[x^2] - E[x]^2 form would lose ~6e-4 of the 1e-2 variance (a few percent of every output)
    assert float((y.double() - want).abs().max()) <= 5e-3
    assert torch.equal(y[2, 256:512], b[256:512])


def test_group_norm_in_place(gpu_case):
    from xlstm_hip import _lib
    g = torch.Generator().manual_seed(3)
    x = torch.randn(10, 2 * 512, generator=g).to(torch.bfloat16).to(dev())
    w, b = (torch.randn(1024, generator=g).to(torch.bfloat16).to(dev()) for _ in range(2))
    lib = _lib.load()
    y = torch.empty_like(x)
    for out in (y, x):  # out of place, then in place
        rc = lib.xl_group_norm_fwd(x.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(), 10, 2, 512, 1e-6, 1,
                                   None)
        assert rc == 0
    assert torch.equal(x, y)


def test_output_cell_cfg4_layer_rows(gpu_case):
    """sLSTMOutputCell.normalize on config 4's kernel output shape (NH 4, H 512), 2 batch rows, bf16."""
    import xlstm_hip
    g = torch.Generator().manual_seed(5)
    h = torch.randn(2, 4096, 4, 512, generator=g).to(torch.bfloat16)
    cell = xlstm_hip.sLSTMOutputCell(2048, 4, 512)
    with torch.no_grad():
        cell.group_norm.weight.copy_(torch.randn(2048, generator=g))
        cell.group_norm.bias.copy_(torch.randn(2048, generator=g))
    cell = cell.to(torch.bfloat16).to(dev())
    y = cell.normalize(h.to(dev()))
    want = osl.group_norm(h.reshape(-1, 2048), 4, cell.group_norm.weight.cpu(), cell.group_norm.bias.cpu(), 1e-6)
    assert_parity(y.reshape(-1, 2048).cpu(), torch.from_numpy(want), torch.bfloat16, "cfg4 group norm")


def test_projection_and_output_cells_fp32(gpu_case):
    """The cells end to end in float32 against the oracle's conv / soft-cap / GroupNorm with the
    same nn.Linear weights on the CPU."""
    import xlstm_hip
    torch.manual_seed(11)
    B, S, D, NH, H = 2, 70, 96, 4, 24
    proj = xlstm_hip.sLSTMProjectionCell(D, NH, H)
    outc = xlstm_hip.sLSTMOutputCell(D, NH, H)
    with torch.no_grad():
        outc.group_norm.weight.normal_()
        outc.group_norm.bias.normal_()
    x = torch.randn(B, S, D)
    hk = torch.randn(B, S, NH, H)
    # CPU composition: oracle conv + SiLU, torch Linear, oracle soft-cap, oracle GroupNorm
    xc = torch.from_numpy(osl.causal_conv1d(x, proj.conv1d.conv.weight.detach(), proj.conv1d.conv.bias.detach(),
                                            activation="silu")).float()
    with torch.no_grad():
        want = (proj.z_proj(x).view(B, S, NH, H), osl_cell.soft_cap(proj.igate_proj(xc), 15.0),
                osl_cell.soft_cap(proj.fgate_proj(xc), 15.0), osl_cell.soft_cap(proj.ogate_proj(x), 15.0), xc)
        gn = torch.from_numpy(osl.group_norm(hk.reshape(B * S, NH * H), NH, outc.group_norm.weight,
                                             outc.group_norm.bias, 1e-6)).float().view(B, S, NH * H)
        want_out = outc.out_proj(gn)
        got = proj.to(dev())(x.to(dev()))
        got_out = outc.to(dev())(hk.to(dev()))
    for g_, w_, name in zip(got, want, ("z", "i", "f", "o", "x_conv")):
        assert g_.shape == w_.shape, name
        assert relerr(g_, w_) <= 1e-4, name
    assert relerr(got_out, want_out) <= 1e-4
