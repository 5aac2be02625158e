"""mLSTM decode step and sequence kernels vs the CPU oracle.

cfg1 (B16 NH8 DQK256 DV512, bf16 q/k/v, float32 states, gates soft-capped at
15) is checked at full size: the oracle step finishes in well under a second
on the CPU.  For a 16-bit q the oracle follows the reference's own dtype
semantics (native_step.py:78-96) on the identical inputs, so the bar is the
north-star max-abs 2e-2 plus a tight agreement check; the float32 path is
held to rel-err 1e-4.
"""

import ctypes

import pytest
import torch

from helpers import FP32_REL, assert_parity, dev, maxabs, print_margins, relerr
from oracle import mlstm as om

pytestmark = pytest.mark.gpu


def _rand_step(B, NH, DQK, DV, dtype, gate_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, NH, DQK, generator=g).to(dtype)
    k = torch.randn(B, NH, DQK, generator=g).to(dtype)
    v = torch.randn(B, NH, DV, generator=g).to(dtype)
    i = (15 * torch.tanh(torch.randn(B, NH, 1, generator=g) / 15)).to(gate_dtype)
    f = (15 * torch.tanh((torch.randn(B, NH, 1, generator=g) + 3) / 15)).to(gate_dtype)
    C = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n = torch.randn(B, NH, DQK, generator=g).abs()
    m = torch.randn(B, NH, 1, generator=g)
    return q, k, v, i, f, C, n, m


def _to(ts):
    return [t.to(dev()) for t in ts]


def test_cfg1_decode_step_bf16(gpu_case):
    import xlstm_hip
    from xlstm_hip.workloads import CFG1, step_inputs
    cpu = step_inputs(CFG1)
    h, (C, n, m) = xlstm_hip.mlstm_recurrent_step__native(*_to(cpu))
    hr, (Cr, nr, mr) = om.mlstm_recurrent_step(*cpu)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        e = assert_parity(got, want, torch.bfloat16, name)
        print(f"cfg1 {name}: max-abs {e:.3e}")
    # the kernel reproduces the reference's bf16 roundings: near-exact agreement
    assert maxabs(h, hr) <= 2 * 2.0 ** -8 * float(hr.float().abs().max())
    assert relerr(C, Cr) <= 1e-6 and relerr(n, nr) <= 1e-6


@pytest.mark.parametrize("shape", [(2, 3, 64, 64), (1, 1, 48, 72), (3, 2, 512, 260), (1, 4, 16, 4),
                                   # 256-column tiles (DV a multiple of 256, >= 256 workgroups, DQK <= 256)
                                   (32, 8, 64, 256), (64, 4, 128, 256), (16, 16, 200, 512)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_step_shapes_dtypes(gpu_case, shape, dtype):
    import xlstm_hip
    B, NH, DQK, DV = shape
    cpu = _rand_step(B, NH, DQK, DV, dtype, torch.float32, seed=DQK + DV)
    h, (C, n, m) = xlstm_hip.mlstm_recurrent_step__native(*_to(cpu))
    hr, (Cr, nr, mr) = om.mlstm_recurrent_step(*cpu)
    assert h.dtype == dtype and C.dtype == torch.float32 and m.shape == (B, NH, 1)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, dtype, f"{shape} {dtype} {name}")


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float16])
def test_step_lowp_gates(gpu_case, gate_dtype):
    import xlstm_hip
    cpu = _rand_step(2, 2, 64, 128, torch.bfloat16, gate_dtype, seed=5)
    h, (C, n, m) = xlstm_hip.mlstm_recurrent_step__native(*_to(cpu))
    hr, (Cr, nr, mr) = om.mlstm_recurrent_step(*cpu)
    for got, want in ((h, hr), (C, Cr), (n, nr), (m, mr)):
        assert_parity(got, want, torch.bfloat16)


def test_step_inplace_matches_functional(gpu_case):
    import xlstm_hip
    cpu = _rand_step(4, 8, 256, 512, torch.bfloat16, torch.float32, seed=11)
    q, k, v, i, f, C, n, m = _to(cpu)
    h1, (C1, n1, m1) = xlstm_hip.mlstm_recurrent_step__native(q, k, v, i, f, C, n, m)
    C2 = C.clone()
    h2, (C2b, n2, m2) = xlstm_hip.mlstm_recurrent_step_(q, k, v, i, f, C2, n, m)
    assert C2b is C2
    assert torch.equal(h1, h2) and torch.equal(C1, C2) and torch.equal(n1, n2) and torch.equal(m1, m2)


def test_chained_steps_match_sequence_oracle(gpu_case):
    import xlstm_hip
    B, NH, S, DQK, DV = 2, 4, 24, 128, 256
    g = torch.Generator().manual_seed(21)
    q, k = (torch.randn(B, NH, S, DQK, generator=g) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    hr, (Cr, nr, mr) = om.mlstm_recurrent_sequence(q, k, v, i, f, return_last_states=True)
    C = torch.zeros(B, NH, DQK, DV, device=dev())
    n = torch.zeros(B, NH, DQK, device=dev())
    m = torch.zeros(B, NH, 1, device=dev())
    hs = []
    qd, kd, vd, idv, fd = _to((q, k, v, i, f))
    for t in range(S):
        h, (C, n, m) = xlstm_hip.mlstm_recurrent_step__native(qd[:, :, t], kd[:, :, t], vd[:, :, t],
                                                              idv[:, :, t, None], fd[:, :, t, None], C, n, m)
        hs.append(h)
    H = torch.stack(hs, dim=2)
    for got, want in ((H, hr), (C, Cr), (n, nr), (m, mr)):
        assert relerr(got, want) <= FP32_REL


@pytest.mark.parametrize("S", [1, 5, 15, 64, 65, 130, 200])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sequence_kernel(gpu_case, S, dtype):
    import xlstm_hip
    B, NH, DQK, DV = 2, 3, 256, 192
    g = torch.Generator().manual_seed(S)
    q, k = (torch.randn(B, NH, S, DQK, generator=g).to(dtype) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g).to(dtype)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    C0 = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n0 = torch.randn(B, NH, DQK, generator=g).abs()
    m0 = torch.randn(B, NH, 1, generator=g)
    h, (C, n, m) = xlstm_hip.mlstm_recurrent_sequence__native_fw(*_to((q, k, v, i, f, C0, n0, m0)),
                                                                return_last_states=True)
    hr, (Cr, nr, mr) = om.mlstm_recurrent_sequence(q, k, v, i, f, C0, n0, m0, return_last_states=True)
    # With a 16-bit q the reference rounds q C' and q n' to q's dtype before dividing one by
    # the other and rounds h once more (native_step.py:83-96).  The GPU's and the CPU's
    # float32 exponentials differ by up to one ulp, which can flip the first two roundings:
    # tests/test_oracle_bf16_sensitivity.py shows the oracle alone, under seeded 1-ulp
    # changes of its gate exponentials, moving its own h beyond 2e-2 past one rounding (at
    # this test's S = 130 inputs) and never beyond 2e-2 past three.  The kernel's measured
    # excess (printed as "[margin]") stays within 2e-2 past two roundings at every S here
    # (worst 1.6e-2 at S = 200), so h is held to 2e-2 beyond two of the reference's roundings.
    rnd = 2
    if dtype != torch.float32:
        print_margins(h, hr, f"sequence h S={S}")
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, dtype, f"S={S} {dtype} {name}", roundings=rnd if name == "h" else 1)
    h0 = xlstm_hip.mlstm_recurrent_sequence__native_fw(*_to((q, k, v, i, f)))
    h0r = om.mlstm_recurrent_sequence(q, k, v, i, f)
    if dtype != torch.float32:
        print_margins(h0, h0r, f"sequence h S={S} zero state")
    assert_parity(h0, h0r, dtype, "zero state", roundings=rnd)


def test_step_alias_rejected(gpu_case):
    from xlstm_hip import _lib
    lib = _lib.load()
    cpu = _rand_step(1, 2, 64, 64, torch.float32, torch.float32, seed=1)
    q, k, v, i, f, C, n, m = _to(cpu)
    h = torch.empty(1, 2, 64, device=dev())
    rc = lib.xl_mlstm_step_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(), C.data_ptr(),
                               n.data_ptr(), m.data_ptr(), h.data_ptr(), C.data_ptr(), n.data_ptr(),
                               torch.empty_like(m).data_ptr(), 1, 2, 64, 64, 0.125, 1e-6, 0, 0, None)
    assert rc == -1 and b"alias" in lib.xl_last_error()


@pytest.mark.parametrize("B,NH,DQK,DV", [(16, 8, 256, 512), (2, 3, 256, 192), (1, 2, 512, 516), (4, 8, 64, 256)])
@pytest.mark.parametrize("in_place", [True, False])
def test_step_copy_ceiling(gpu_case, B, NH, DQK, DV, in_place):
    """xl_mlstm_step_copy_ceiling (the decode step's access pattern without its arithmetic) moves
    every element of C unchanged, in place and out of place, on the wide tiles (config 1) and the
    64-column tiles (ragged last tile, 8 rows per thread)."""
    from xlstm_hip import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev()).manual_seed(DQK + DV)
    C = torch.randn(B, NH, DQK, DV, generator=g, device=dev())
    want = C.clone()
    out = C if in_place else torch.full_like(C, float("nan"))
    rc = lib.xl_mlstm_step_copy_ceiling(C.data_ptr(), out.data_ptr(), B, NH, DQK, DV, None)
    _lib.check(rc, "copy ceiling")
    torch.cuda.synchronize()
    assert torch.equal(out, want)


@pytest.mark.parametrize("DQK,DV", [(64, 64), (128, 256), (512, 128)])
@pytest.mark.parametrize("S", [63, 150])
def test_sequence_kernel_heads_and_strong_gates(gpu_case, DQK, DV, S):
    """Head sizes of every row-per-thread variant (DQK 64 .. 512) and gates spanning +-15, so the
    stabiliser resets to i_t often and the 64-step gate chunks carry m across their boundary."""
    import xlstm_hip
    B, NH = 1, 2
    g = torch.Generator().manual_seed(DQK + S)
    q, k = (torch.randn(B, NH, S, DQK, generator=g) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g)
    i = 15 * torch.tanh(4 * torch.randn(B, NH, S, generator=g) / 15)
    f = 15 * torch.tanh(6 * torch.randn(B, NH, S, generator=g) / 15)
    C0 = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n0 = torch.randn(B, NH, DQK, generator=g).abs()
    m0 = torch.randn(B, NH, 1, generator=g)
    h, (C, n, m) = xlstm_hip.mlstm_recurrent_sequence__native_fw(*_to((q, k, v, i, f, C0, n0, m0)),
                                                                return_last_states=True)
    hr, (Cr, nr, mr) = om.mlstm_recurrent_sequence(q, k, v, i, f, C0, n0, m0, return_last_states=True)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, torch.float32, f"DQK={DQK} DV={DV} S={S} {name}")


@pytest.mark.parametrize("S,with_state", [(1, True), (1, False), (7, True), (70, False)])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16])
def test_recurrent_kernel_cell(gpu_case, S, with_state, in_dtype):
    """mLSTMRecurrentKernelCell (the model-level decode caller, float32 compute and states by
    default): one token with a state runs the step kernel, the rest the sequence kernel; both
    against the cell's own restatement (mlstm_recurrent_kernel_cell.py:53-161) on the inputs cast
    to float32, as the cell casts them."""
    import xlstm_hip
    B, NH, DQK, DV = 2, 4, 256, 512
    g = torch.Generator().manual_seed(S + 100 * with_state)
    q, k = (torch.randn(B, NH, S, DQK, generator=g).to(in_dtype) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g).to(in_dtype)
    i = (15 * torch.tanh(torch.randn(B, NH, S, generator=g) / 15)).to(in_dtype)
    f = (15 * torch.tanh((torch.randn(B, NH, S, generator=g) + 3) / 15)).to(in_dtype)
    state = None
    if with_state:
        state = (0.1 * torch.randn(B, NH, DQK, DV, generator=g), torch.randn(B, NH, DQK, generator=g).abs(),
                 torch.randn(B, NH, generator=g))
    cell = xlstm_hip.mLSTMRecurrentKernelCell(NH, DQK, DV)
    h, (C, n, m) = cell(*_to((q, k, v, i, f)), None if state is None else tuple(_to(state)))
    hr, (Cr, nr, mr) = om.mlstm_recurrent_kernel_cell(*(t.float() for t in (q, k, v, i, f)), state)
    assert h.shape == (B, NH, S, DV) and h.dtype == torch.float32 and m.shape == (B, NH)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert relerr(got, want) <= FP32_REL, f"S={S} state={with_state} {in_dtype} {name}"
