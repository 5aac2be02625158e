"""sLSTM step/sequence and the arbitrary-length backend on the GPU vs the CPU oracle.

sLSTM cases reuse the shapes and seeds of the reference's
tests/test_slstm_metal_kernel.py:110-314 (2,4,8 / zero state / gates +-10 with
states x100 / 5 chained steps) plus cfg4's sLSTM shape (B8 NH4 H512).
"""

import pytest
import torch

from helpers import FP32_REL, assert_parity, dev, relerr
from oracle import mlstm as om
from oracle import slstm as osl

pytestmark = pytest.mark.gpu


def _to(ts):
    return [None if t is None else t.to(dev()) for t in ts]


@pytest.mark.parametrize("case", ["random", "zero", "extreme_pos", "extreme_neg"])
def test_slstm_step_cases(gpu_case, case):
    import xlstm_hip
    g = torch.Generator().manual_seed(42)
    B, NH, H = 2, 4, 8
    z = torch.randn(B, NH, H, generator=g)
    i, f, o = (torch.randn(B, NH, generator=g) for _ in range(3))
    c = torch.randn(B, NH, H, generator=g)
    n = torch.randn(B, NH, H, generator=g).abs()
    m = torch.randn(B, NH, generator=g)
    if case == "zero":
        c, n, m = torch.zeros_like(c), torch.zeros_like(n), torch.zeros_like(m)
    elif case.startswith("extreme"):
        val = 10.0 if case.endswith("pos") else -10.0
        i = f = o = torch.full((B, NH), val)
        c, n = 100 * c, 100 * n
    got = xlstm_hip.slstm_step(*_to((z, i, f, o, c, n, m)))
    want = osl.slstm_step(z, i, f, o, c, n, m)
    for a, b in zip(got, want):
        assert relerr(a, b) <= FP32_REL


def test_slstm_cell_five_steps(gpu_case):
    import xlstm_hip
    g = torch.Generator().manual_seed(5)
    B, NH, H, S = 2, 4, 8, 5
    z = torch.randn(B, S, NH, H, generator=g)
    i, f, o = (torch.randn(B, S, NH, generator=g) for _ in range(3))
    cell = xlstm_hip.sLSTMStepwiseKernelCell(NH, H)
    state = None
    hs = []
    zd, idv, fd, od = _to((z, i, f, o))
    for t in range(S):
        h, state = cell(zd[:, t], idv[:, t], fd[:, t], od[:, t], state)
        hs.append(h)
    hr, (cr, nr, mr) = osl.slstm_sequence(z, i, f, o)
    assert relerr(torch.stack(hs, 1), hr) <= FP32_REL
    for a, b in zip(state, (cr, nr, mr)):
        assert relerr(a, b) <= FP32_REL


@pytest.mark.parametrize("with_state", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 7, 4, 8), (8, 256, 4, 512), (1, 33, 3, 100), (2, 1100, 2, 64),
                                   (1, 4096, 2, 128), (1, 2000, 1, 200), (2, 1025, 2, 64), (1, 3000, 1, 64)])
def test_slstm_sequence(gpu_case, dtype, shape, with_state):
    """With an initial state every element carries its own n; without one n is the same for
    every d of a head and the kernel forms h = c * og / (|n| + eps) with one scale per step."""
    import xlstm_hip
    B, S, NH, H = shape
    g = torch.Generator().manual_seed(S)
    z = torch.randn(B, S, NH, H, generator=g).to(dtype)
    i, f, o = ((15 * torch.tanh(torch.randn(B, S, NH, generator=g) / 15)).to(dtype) for _ in range(3))
    st = (torch.randn(B, NH, H, generator=g), torch.randn(B, NH, H, generator=g).abs(), torch.randn(B, NH, generator=g))
    st = st if with_state else None
    h, (c, n, m) = xlstm_hip.slstm_sequence(*_to((z, i, f, o)), state=tuple(_to(st)) if st else None)
    hr, (cr, nr, mr) = osl.slstm_sequence(z.float(), i.float(), f.float(), o.float(), state=st)
    for a, b, name in ((h, hr, "h"), (c, cr, "c"), (n, nr, "n"), (m, mr, "m")):
        if dtype == torch.float32 or with_state:
            # float32 outputs (with a float32 state the outputs are float32 for bf16 inputs too)
            assert a.dtype == torch.float32 and relerr(a, b) <= FP32_REL, name
        else:  # no state: outputs in the inputs' 16-bit dtype
            assert a.dtype == dtype
            assert_parity(a, b, dtype, f"{shape} {name}")


@pytest.mark.parametrize("with_state", [True, False])
@pytest.mark.parametrize("shape", [(2, 300, 2, 64), (1, 1500, 1, 200)])
def test_slstm_sequence_strong_gates(gpu_case, shape, with_state):
    """Gate pre-activations spread over +-15: i resets the stabiliser often and the forget
    products of a 64-step chunk underflow, so the chunk weights of the first pass see both."""
    import xlstm_hip
    B, S, NH, H = shape
    g = torch.Generator().manual_seed(7 * S)
    z = 2 * torch.randn(B, S, NH, H, generator=g)
    i, f, o = (15 * torch.tanh(6 * torch.randn(B, S, NH, generator=g) / 15) for _ in range(3))
    st = (torch.randn(B, NH, H, generator=g), torch.randn(B, NH, H, generator=g).abs(), torch.randn(B, NH, generator=g))
    st = st if with_state else None
    h, (c, n, m) = xlstm_hip.slstm_sequence(*_to((z, i, f, o)), state=tuple(_to(st)) if st else None)
    hr, (cr, nr, mr) = osl.slstm_sequence(z, i, f, o, state=st)
    for a, b, name in ((h, hr, "h"), (c, cr, "c"), (n, nr, "n"), (m, mr, "m")):
        assert relerr(a, b) <= FP32_REL, f"{shape} state={with_state} {name}"


@pytest.mark.parametrize("S", [768, 700])
def test_slstm_sequence_tanh_every_bf16(gpu_case, S):
    """tanh z of the sequence kernel over every bf16 value of z, against float64 tanh.

    Gates that make each step its own (f = -inf: fg = 0; i = 0: ig = 1; o = +inf: og = 1;
    eps = 0, fp32 h) give h_t = tanh z_t.  S = 768 runs the whole-segment pass (12 waves x 64
    steps), S = 700 the short-segment one.  Every finite and infinite bf16 value appears in
    steps 0 .. S-2; NaN in the last step, where it cannot reach another step.  Bound: the
    kernel's tanh, 1 - 2 / (1 + e^{2z}), within 2e-7 absolute of tanh z, and +-1 exactly for
    |z| >= 9.5 (where tanh z rounds to +-1 in fp32)."""
    import xlstm_hip
    H = 128
    bits = torch.arange(65536, dtype=torch.int32)
    nan = ((bits & 0x7F80) == 0x7F80) & ((bits & 0x7F) != 0)
    finite = bits[~nan]
    n_body = (S - 1) * H
    body = finite.repeat((n_body + finite.numel() - 1) // finite.numel())[:n_body]
    last = bits[nan][:H]
    allb = torch.cat([body, last]).to(torch.int16)
    z = allb.view(torch.bfloat16).view(1, S, 1, H)
    i = torch.zeros(1, S, 1)
    f = torch.full((1, S, 1), -float("inf"))
    o = torch.full((1, S, 1), float("inf"))
    h, _ = xlstm_hip.slstm_sequence(*_to((z, i, f, o)), eps=0.0)
    assert h.dtype == torch.float32
    h = h.cpu().double().view(S, H)
    ref = torch.tanh(z.double().view(S, H))
    err = (h[:-1] - ref[:-1]).abs()
    print(f"S={S}: max |h - tanh z| {err.max().item():.3e} (bound 2e-7)")
    assert err.max().item() < 2e-7
    big = z.double().view(S, H)[:-1].abs() >= 9.5
    assert torch.equal(h[:-1][big], torch.sign(ref[:-1][big]))
    assert torch.isnan(h[-1]).all()


@pytest.mark.parametrize("S", [1, 5, 16, 37, 100, 129, 200])
def test_arbitrary_length_inference(gpu_case, S):
    import xlstm_hip
    B, NH, DQK, DV = 1, 2, 64, 64
    g = torch.Generator().manual_seed(S)
    q, k = (torch.randn(B, NH, S, DQK, generator=g) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    backend = xlstm_hip.mLSTMBackend(xlstm_hip.mLSTMBackendConfig(mode="inference", chunk_size=64))
    h, (C, n, m) = backend(*_to((q, k, v, i, f)))
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, chunk_size=64)
    for a, b, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert relerr(a, b) <= FP32_REL, f"S={S} {name}"


def test_backend_train_modes(gpu_case):
    import xlstm_hip
    B, NH, S, D = 1, 2, 100, 32
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, NH, S, D, generator=g) for _ in range(3))
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    pad = xlstm_hip.mLSTMBackend(xlstm_hip.mLSTMBackendConfig(mode="train_with_padding", return_last_states=False))
    h = pad(*_to((q, k, v, i, f)))
    Sp = 128
    padded = [torch.nn.functional.pad(t, (0, 0, 0, Sp - S)) for t in (q, k, v)] + \
             [torch.nn.functional.pad(t, (0, Sp - S)) for t in (i, f)]
    hr = om.mlstm_chunkwise(*padded)[:, :, :S]
    assert relerr(h, hr) <= FP32_REL
    train = xlstm_hip.mLSTMBackend(xlstm_hip.mLSTMBackendConfig(mode="train", chunk_size=64))
    x = [t[:, :, :64] for t in (q, k, v)] + [t[:, :, :64] for t in (i, f)]
    h, (C, n, m) = train(*_to(x))
    hr, (Cr, nr, mr) = om.mlstm_chunkwise(*x, return_last_states=True)
    assert relerr(h, hr) <= FP32_REL and relerr(C, Cr) <= FP32_REL
