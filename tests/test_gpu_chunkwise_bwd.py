"""Chunkwise backward on the GPU (xl_mlstm_chunkwise_bwd through torch.autograd) against the oracle's
restatement of the reference's custom backward (oracle.mlstm.mlstm_chunkwise_bw, itself pinned to
torch.autograd in tests/test_oracle_chunkwise_bw.py), run in float64 on the same inputs.

Bars, per gradient, relative to the largest magnitude of the expected tensor:
* float32 inputs (two-pass float32 forward, float32 backward): |got - want| <= 1e-4 max|want|;
* bf16 inputs (the gradients come back in bf16): |got - want| <= 2^-8 |want| + 2e-3 max|want|
  (the output's own rounding, one ulp, plus float32 accumulation over the chunk).

Cases: with and without initial states, the last-state gradient, chunk sizes 16 / 32 / 64 / 128
(128 runs as 64-token chunks), DQK and DV that are not multiples of the 64-wide tiles, several heads
and chunks, bf16 and f16 inputs, ragged sequences from the single-pass forward (padded to whole
chunks with state-preserving tokens), and the registry form mlstm_chunkwise__native_custbw.
"""

import pytest
import torch

from helpers import dev
from oracle import mlstm as om

pytestmark = pytest.mark.gpu


def _inputs(B, NH, S, DQK, DV, seed, states):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, NH, S, DQK, generator=g)
    k = torch.randn(B, NH, S, DQK, generator=g)
    v = torch.randn(B, NH, S, DV, generator=g)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3.0
    st = None
    if states:
        st = (0.3 * torch.randn(B, NH, DQK, DV, generator=g), torch.rand(B, NH, DQK, generator=g) + 0.5,
              0.5 * torch.randn(B, NH, 1, generator=g))
    dh = torch.randn(B, NH, S, DV, generator=g)
    dcl = torch.randn(B, NH, DQK, DV, generator=g)
    return (q, k, v, i, f), st, dh, dcl


def _check(got, want, dtype, what, scale=None):
    got, want = got.detach().double().cpu(), want.detach().double().cpu()
    scale = float(want.abs().max()) if scale is None else scale
    if dtype == torch.float32:
        err = float((got - want).abs().max()) / scale
        assert err <= 1e-4, f"{what}: rel-err {err:.3e}"
    else:
        excess = float(((got - want).abs() - 2.0 ** -8 * want.abs()).max()) / scale
        assert excess <= 2e-3, f"{what}: {excess:.3e} of max beyond one rounding"


def _run(B, NH, S, DQK, DV, L, dtype, states, last, seed, algo="auto"):
    import xlstm_hip
    x, st, dh, dcl = _inputs(B, NH, S, DQK, DV, seed, states)
    xd = [t.to(dtype).to(dev()).requires_grad_(True) for t in x]
    std = [t.to(dev()).requires_grad_(True) for t in st] if states else [None, None, None]
    out = xlstm_hip.mlstm_chunkwise(*xd, *std, return_last_states=last, chunk_size=L, algo=algo)
    h, (C, _, _) = out if last else (out, (None, None, None))
    loss = (h.float() * dh.to(dev())).sum()
    if last:
        loss = loss + (C * dcl.to(dev())).sum()
    loss.backward()
    # oracle on the same (rounded) inputs in float64; h is in q's dtype, so the gradient reaching it
    # is dh rounded to that dtype
    x64 = [t.to(dtype).double() for t in x]
    st64 = [t.double() for t in st] if states else [None, None, None]
    want = om.mlstm_chunkwise_bw(*x64, dh.to(dtype).double(), *st64, matDeltaC_last=dcl.double() if last else None,
                                 chunk_size=L)
    for nm, t, w in zip(["dq", "dk", "dv", "di", "df"], xd, want[:5]):
        assert t.grad.dtype == dtype
        _check(t.grad, w, dtype, f"{nm} B{B} NH{NH} S{S} DQK{DQK} DV{DV} L{L} {dtype} states={states} last={last}")
    if states:
        _check(std[0].grad, want[5], torch.float32, "dc0")
        assert float(std[1].grad.abs().max()) == 0.0 and float(std[2].grad.abs().max()) == 0.0


@pytest.mark.parametrize("B,NH,S,DQK,DV,L", [(1, 2, 128, 64, 64, 64), (2, 3, 96, 48, 80, 32), (1, 1, 64, 16, 16, 16),
                                             (1, 2, 192, 128, 96, 64), (2, 2, 128, 200, 72, 16)])
@pytest.mark.parametrize("states,last", [(False, False), (True, True), (True, False), (False, True)])
def test_fp32_vs_oracle(gpu_case, B, NH, S, DQK, DV, L, states, last):
    _run(B, NH, S, DQK, DV, L, torch.float32, states, last, seed=B * 100 + S + DQK + L + 2 * states + last)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,NH,S,DQK,DV", [(1, 2, 256, 128, 128), (2, 2, 128, 256, 64)])
def test_lowp_vs_oracle(gpu_case, dtype, B, NH, S, DQK, DV):
    _run(B, NH, S, DQK, DV, 64, dtype, True, True, seed=7 + S)


@pytest.mark.parametrize("B,NH,S,DQK,DV,L", [(1, 2, 512, 256, 512, 64), (1, 1, 192, 128, 192, 64),
                                             (1, 2, 128, 64, 128, 32), (2, 1, 96, 256, 64, 32),
                                             (1, 2, 96, 128, 64, 16)])
def test_bf16_block_counts(gpu_case, B, NH, S, DQK, DV, L):
    """bf16 at config 2's head shape (8 DV blocks in the dQ/dK loop, 4 DQK blocks in dV), an odd
    number of DV blocks (3), 32-token chunks (the bf16 chunk scans with one 32-token step) and
    16-token chunks (float32-MFMA scans, FMA tile passes)."""
    _run(B, NH, S, DQK, DV, L, torch.bfloat16, True, True, seed=11 + S + DV)


@pytest.mark.parametrize("B,NH,S,DQK,DV", [(1, 2, 256, 64, 256), (2, 1, 192, 128, 512), (1, 1, 128, 256, 256),
                                          (1, 3, 64, 128, 256)])
@pytest.mark.parametrize("states,last", [(True, True), (False, False)])
def test_bf16_fused_pass_shapes(gpu_case, B, NH, S, DQK, DV, states, last):
    """bf16 with DV 256 / 512 (dV, dQ and dK in one pass per (head, chunk)) at every DQK the pass
    is built for (1, 2 and 4 d-tiles, 4 and 8 v-blocks), an odd chunk count and a single chunk."""
    _run(B, NH, S, DQK, DV, 64, torch.bfloat16, states, last, seed=23 + S + DQK + DV + states)


def test_bf16_config2_heads_full_length(gpu_case):
    """Two heads of config 2 over its whole sequence (S 8192, 128 chunks of the state and dC
    recurrences; DQK 256, DV 512, bf16), with initial and last states."""
    _run(1, 2, 8192, 256, 512, 64, torch.bfloat16, True, True, seed=8192)


def test_larger_fp32(gpu_case):
    _run(2, 4, 512, 128, 256, 64, torch.float32, True, True, seed=77)


def test_registry_form_and_gate_dtypes(gpu_case):
    """mlstm_chunkwise__native_custbw with bf16 q/k/v and float32 gates: the gate gradients come back
    in float32, dq/dk/dv in bf16, all within the bars above."""
    import xlstm_hip
    B, NH, S, DQK, DV = 1, 2, 128, 64, 64
    x, st, dh, _ = _inputs(B, NH, S, DQK, DV, 5, False)
    q, k, v = (t.bfloat16().to(dev()).requires_grad_(True) for t in x[:3])
    i, f = (t.to(dev()).requires_grad_(True) for t in x[3:])
    h = xlstm_hip.mlstm_chunkwise__native_custbw(q, k, v, i, f)
    (h.float() * dh.to(dev())).sum().backward()
    want = om.mlstm_chunkwise_bw(*(t.bfloat16().double() for t in x[:3]), x[3].double(), x[4].double(),
                                 dh.bfloat16().double())
    for nm, t, w, dt in (("dq", q, want[0], torch.bfloat16), ("dk", k, want[1], torch.bfloat16),
                         ("dv", v, want[2], torch.bfloat16), ("di", i, want[3], torch.float32),
                         ("df", f, want[4], torch.float32)):
        assert t.grad.dtype == dt
        _check(t.grad, w, dt if dt == torch.float32 else torch.bfloat16, nm)


@pytest.mark.parametrize("dtype,states,last", [(torch.bfloat16, True, True), (torch.float32, False, True),
                                              (torch.bfloat16, False, False)])
def test_chunk_size_128(gpu_case, dtype, states, last):
    """Training with chunk_size=128: the backward runs at 64-token chunks (the custom backward's
    gradients do not depend on the chunk size), against the oracle's backward at 128."""
    _run(1, 2, 256, 128, 128, 128, dtype, states, last, seed=128 + 2 * states + last)


@pytest.mark.parametrize("S", [1, 37, 100, 200, 1000])
@pytest.mark.parametrize("states,last", [(True, True), (False, False)])
@pytest.mark.parametrize("algo", ["pipelined", "fused"])
def test_ragged_sequence_backward(gpu_case, S, states, last, algo):
    """A sequence the single-pass forward ran with a ragged last chunk (bf16, S % 64 != 0) is
    differentiable: the backward pads it to whole 64-token chunks with state-preserving tokens
    (input gate -3e4, forget gate +30; tests/test_oracle_chunkwise_bw.py::test_state_preserving_padding
    shows they change no gradient of the original tokens) and drops their gradients.  Against
    the oracle's backward on the same padded sequence."""
    import xlstm_hip
    from xlstm_hip.ops import _PAD_F, _PAD_I
    B, NH, DQK, DV, dtype = 1, 2, 128, 128, torch.bfloat16
    x, st, dh, dcl = _inputs(B, NH, S, DQK, DV, 300 + S, states)
    xd = [t.to(dtype).to(dev()).requires_grad_(True) for t in x]
    std = [t.to(dev()).requires_grad_(True) for t in st] if states else [None, None, None]
    out = xlstm_hip.mlstm_chunkwise(*xd, *std, return_last_states=last, chunk_size=64, algo=algo)
    h, (C, _, _) = out if last else (out, (None, None, None))
    loss = (h.float() * dh.to(dev())).sum()
    if last:
        loss = loss + (C * dcl.to(dev())).sum()
    loss.backward()
    pad = (-S) % 64
    padz = lambda t: torch.nn.functional.pad(t, (0, 0, 0, pad))
    q, k, v, i, f = (t.to(dtype).double() for t in x)
    xp = (padz(q), padz(k), padz(v), torch.nn.functional.pad(i, (0, pad), value=_PAD_I),
          torch.nn.functional.pad(f, (0, pad), value=_PAD_F))
    st64 = [t.double() for t in st] if states else [None, None, None]
    want = om.mlstm_chunkwise_bw(*xp, padz(dh.to(dtype).double()), *st64,
                                 matDeltaC_last=dcl.double() if last else None, chunk_size=64)
    # the gate gradients against the larger of the two: with one token and no states df is a sum
    # of terms that cancel exactly (the oracle's float64 leaves ~1e-12 of them)
    gate_scale = max(float(want[3][:, :, :S].abs().max()), float(want[4][:, :, :S].abs().max()))
    for nm, t, w in zip(["dq", "dk", "dv", "di", "df"], xd, want[:5]):
        assert t.grad.shape == t.shape
        _check(t.grad, w[:, :, :S], dtype, f"ragged {nm} S{S} {algo} states={states} last={last}",
               scale=gate_scale if nm in ("di", "df") else None)
    if states:
        _check(std[0].grad, want[5], torch.float32, "ragged dc0")


def test_native_autograd_name_warns_on_custom_gradients(gpu_case):
    """Under the reference's __native_autograd name the gradients are the custom backward's: a
    call that returns the last states with inputs that require grad says so (a RuntimeWarning,
    once per process); one that returns h only does not."""
    import warnings

    import xlstm_hip
    from xlstm_hip import chunkwise
    x, _, _, _ = _inputs(1, 2, 64, 64, 64, 9, False)
    xd = [t.to(dev()).requires_grad_(True) for t in x]
    chunkwise._autograd_warned = False
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        xlstm_hip.mlstm_chunkwise__native_autograd(*xd)  # h only: no warning
    with pytest.warns(RuntimeWarning, match="custom backward"):
        xlstm_hip.mlstm_chunkwise__native_autograd(*xd, return_last_states=True)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        xlstm_hip.mlstm_chunkwise__native_autograd(*xd, return_last_states=True)  # once only
