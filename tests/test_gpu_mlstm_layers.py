"""mLSTM output cell stage on the GPU vs the CPU oracle: multi-head RMSNorm x weight x sigmoid(o).

Head dims cover a full-wave team (DH 512 bf16), smaller teams (256, 64), the scalar path (DH
not a multiple of the 16-byte vector), eight vectors per lane (DH 4096 bf16) and sixteen with one
group per team (DH 8192 bf16, 4096 float32); h in the
chunkwise layout [B, NH, S, DH] and in [B, S, NH, DH]; with and without the weight and the gate;
and config 2's kernel output for one batch row (NH 8, S 8192, DH 512).  Bars: float32 rel-err
1e-4; 16-bit max-abs 2e-2 beyond the output's own rounding.
"""

import pytest
import torch

from helpers import assert_parity, dev, relerr
from oracle import mlstm_layers as oml

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _inputs(B, NH, S, DH, dtype, seed, heads_first=True):
    g = torch.Generator().manual_seed(seed)
    shape = (B, NH, S, DH) if heads_first else (B, S, NH, DH)
    h = (3 * torch.randn(shape, generator=g)).to(dtype)
    w = (1 + 0.5 * torch.randn(NH * DH, generator=g)).to(dtype)
    o = (2 * torch.randn(B, S, NH * DH, generator=g)).to(dtype)
    return h, w, o


@pytest.mark.parametrize("B,NH,S,DH", [(2, 4, 37, 512), (1, 8, 64, 256), (2, 3, 10, 100), (1, 2, 5, 4096),
                                       (1, 2, 9, 7), (3, 1, 4, 64), (1, 1, 3, 8192)])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("heads_first", [True, False])
@pytest.mark.parametrize("use_w,use_o", [(True, True), (False, False), (True, False)])
def test_vs_oracle(gpu_case, B, NH, S, DH, dtype, heads_first, use_w, use_o):
    import xlstm_hip
    h, w, o = _inputs(B, NH, S, DH, dtype, seed=B + NH + S + DH, heads_first=heads_first)
    w, o = (w if use_w else None), (o if use_o else None)
    if dtype == torch.float32 and DH > 4096:  # 32 float32 vectors per lane: above the documented limit
        with pytest.raises(NotImplementedError, match="head dim"):
            xlstm_hip.mh_rmsnorm_gate(h.to(dev()), heads_first=heads_first)
        return
    y = xlstm_hip.mh_rmsnorm_gate(h.to(dev()), None if w is None else w.to(dev()), None if o is None else o.to(dev()),
                                  1e-6, heads_first=heads_first)
    want = torch.from_numpy(oml.mh_rmsnorm_gate(h, w, o, 1e-6, heads_first=heads_first))
    assert y.shape == (B, S, NH * DH) and y.dtype == dtype
    assert_parity(y.cpu(), want, dtype, f"{B, NH, S, DH} {dtype} hf={heads_first} w={use_w} o={use_o}")


def test_cfg2_kernel_output_row(gpu_case):
    """Config 2's chunkwise output for one batch row (NH 8, S 8192, DH 512, bf16), gated."""
    import xlstm_hip
    h, w, o = _inputs(1, 8, 8192, 512, torch.bfloat16, seed=2)
    y = xlstm_hip.mh_rmsnorm_gate(h.to(dev()), w.to(dev()), o.to(dev()), 1e-6)
    assert_parity(y.cpu(), torch.from_numpy(oml.mh_rmsnorm_gate(h, w, o, 1e-6)), torch.bfloat16, "cfg2 row")


def test_modules_fp32(gpu_case):
    """MultiHeadRMSNorm and mLSTMOutputCell end to end in float32 against the oracle with the same
    nn.Linear weights on the CPU."""
    import xlstm_hip
    torch.manual_seed(3)
    B, NH, S, DH, D = 2, 4, 33, 64, 96
    cell = xlstm_hip.mLSTMOutputCell(D, NH, DH)
    with torch.no_grad():
        cell.norm.weight.normal_()
    h = torch.randn(B, NH, S, DH)
    x = torch.randn(B, S, D)
    with torch.no_grad():
        want = cell.out_proj(torch.from_numpy(oml.mh_rmsnorm_gate(h, cell.norm.weight, cell.ogate_proj(x))).float())
        want_norm = oml.mh_rmsnorm_gate(h.permute(0, 2, 1, 3), cell.norm.weight, heads_first=False)
        cell = cell.to(dev())
        got = cell(h.to(dev()), x.to(dev()))
        got_norm = cell.norm(h.permute(0, 2, 1, 3).to(dev()))
    assert relerr(got, want) <= 1e-4
    assert relerr(got_norm, torch.from_numpy(want_norm)) <= 1e-4


def test_rejections(gpu_case):
    import xlstm_hip
    from xlstm_hip import _lib
    h = torch.randn(1, 2, 4, 16384, device=dev()).to(torch.bfloat16)
    with pytest.raises(NotImplementedError, match="head dim"):
        xlstm_hip.mh_rmsnorm_gate(h)
    with pytest.raises(ValueError, match="dtype"):
        xlstm_hip.mh_rmsnorm_gate(h[..., :64].contiguous(), torch.ones(128, device=dev()))
    lib = _lib.load()
    x = torch.randn(1, 2, 4, 64, device=dev())
    rc = lib.xl_mh_rmsnorm_gate_fwd(x.data_ptr(), None, None, x.data_ptr(), 1, 2, 4, 64, 1, 1e-6, 0, None)
    assert rc == -1 and b"alias" in lib.xl_last_error()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("use_bias", [False, True])
def test_multihead_layernorm(gpu_case, dtype, use_bias):
    """MultiHeadLayerNorm (per-head LayerNorm, weight and optional bias) on the GroupNorm kernel."""
    import xlstm_hip
    from oracle import slstm_layers as osl
    torch.manual_seed(6)
    B, S, NH, DH = 2, 40, 4, 128
    m = xlstm_hip.MultiHeadLayerNorm(NH, DH, use_bias=use_bias)
    with torch.no_grad():
        m.weight.normal_()
        if use_bias:
            m.bias.normal_()
    m = m.to(dtype)
    x = (2 * torch.randn(B, S, NH, DH) + 1).to(dtype)
    want = osl.group_norm(x.reshape(B * S, NH * DH), NH, m.weight, m.bias, 1e-6).reshape(B, S, NH * DH)
    y = m.to(dev())(x.to(dev()))
    assert y.shape == (B, S, NH * DH)
    assert_parity(y.cpu(), torch.from_numpy(want), dtype, f"MultiHeadLayerNorm {dtype} bias={use_bias}")
