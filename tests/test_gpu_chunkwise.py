"""Chunkwise mLSTM forward on the GPU vs the CPU oracle.

* cfg0 at full size (float32, B1 NH8 S256 DQK256 DV512 L64): rel-err <= 1e-4
  on h and the final C, n, m;
* every chunk size, initial states, ragged head dims, 16-bit inputs against the
  float32 oracle on the upcast inputs (max-abs <= 2e-2);
* cfg2 at full size (bf16, B4 NH8 S8192, L 64 and 128) against the oracle on
  the whole batch, plus the causal prefix property (tokens < S' depend only
  on inputs < S'), chunk-size invariance and agreement with the other
  algorithm;
* the fused kernel works on 64-token chunks for every chunk_size (the forward
  is chunk-size invariant): chunk sizes 16, 32, 128 against the oracle at that
  chunk size;
* algo="fused" with any S (ragged last chunk) and the any-S backend's one-call
  bf16 path against the oracle's any-S driver;
* every single-pass case runs on both single-pass kernels: "fused" and
  "pipelined" (the two-phase state/output-wave schedule of the same chunk
  algorithm), each against the oracle;
* float16 q/k/v on the pipelined kernel (f16 MFMA operands): any S, initial
  states, the sequence split, and inputs where f16's range matters.
"""

import pytest
import torch

from helpers import FP32_REL, LOWP_ABS, assert_parity, dev, half_ulp, lowp_excess, maxabs, relerr
from oracle import mlstm as om

pytestmark = pytest.mark.gpu


def _inputs(B, NH, S, DQK, DV, dtype, seed, with_state=False):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, NH, S, DQK, generator=g) / DQK ** 0.5).to(dtype)
    k = torch.randn(B, NH, S, DQK, generator=g).to(dtype)
    v = torch.randn(B, NH, S, DV, generator=g).to(dtype)
    i = torch.randn(B, NH, S, generator=g).to(dtype)
    f = (torch.randn(B, NH, S, generator=g) + 3).to(dtype)
    st = (None, None, None)
    if with_state:
        st = (0.1 * torch.randn(B, NH, DQK, DV, generator=g), torch.randn(B, NH, DQK, generator=g).abs(),
              torch.randn(B, NH, 1, generator=g))
    return (q, k, v, i, f), st


def _gpu(ts):
    return [None if t is None else t.to(dev()) for t in ts]


SINGLE_PASS = ["fused", "pipelined"]
_cfg2_oracle = {}


def _oracle(x, st, L):
    return om.mlstm_chunkwise(*(t.float() for t in x), *st, return_last_states=True, chunk_size=L)


def test_cfg0_fp32_full_size(gpu_case):
    import xlstm_hip
    from xlstm_hip.workloads import CFG0, chunkwise_inputs
    x = chunkwise_inputs(CFG0)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), return_last_states=True, chunk_size=CFG0.L)
    hr, (Cr, nr, mr) = _oracle(x, (None, None, None), CFG0.L)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        e = relerr(got, want)
        print(f"cfg0 {name}: rel-err {e:.3e}")
        assert e <= FP32_REL, name


@pytest.mark.parametrize("L", [16, 32, 64, 128])
@pytest.mark.parametrize("with_state", [False, True])
def test_fp32_chunk_sizes(gpu_case, L, with_state):
    import xlstm_hip
    x, st = _inputs(2, 3, 256, 64, 96, torch.float32, seed=L, with_state=with_state)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=L)
    hr, (Cr, nr, mr) = _oracle(x, st, L)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert relerr(got, want) <= FP32_REL, name


@pytest.mark.parametrize("shape,with_state,last", [((2, 2, 256, 64, 128), True, True), ((1, 2, 320, 128, 64), True, True),
                                              ((2, 1, 192, 256, 192), False, True), ((1, 2, 128, 128, 128), True, False)])
def test_fp32_matrix_core_two_pass(gpu_case, shape, with_state, last):
    """float32 q/k/v with 64-token chunks and whole 64-wide tiles: the states pass on float32 MFMA and
    the output pass in the three-product bf16 form, at each DQK the output kernel instantiates, with
    and without initial states and last states."""
    import xlstm_hip
    B, NH, S, DQK, DV = shape
    x, st = _inputs(B, NH, S, DQK, DV, torch.float32, seed=S + DQK + DV, with_state=with_state)
    out = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=last, chunk_size=64)
    hr, (Cr, nr, mr) = _oracle(x, st, 64)
    if not last:
        assert relerr(out, hr) <= FP32_REL, "h"
        return
    h, (C, n, m) = out
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert relerr(got, want) <= FP32_REL, f"{shape} {name}"


@pytest.mark.parametrize("shape", [(1, 1, 64, 32, 16), (2, 2, 128, 80, 72), (1, 2, 192, 256, 512)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("algo", ["auto", "two_pass"])
def test_lowp_inputs(gpu_case, shape, dtype, algo):
    import xlstm_hip
    B, NH, S, DQK, DV = shape
    x, st = _inputs(B, NH, S, DQK, DV, dtype, seed=S + DQK, with_state=True)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=64,
                                             algo=algo)
    hr, (Cr, nr, mr) = _oracle(x, st, 64)
    assert h.dtype == dtype
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, dtype, f"{shape} {dtype} {algo} {name}")


def test_no_last_states_and_defaults(gpu_case):
    import xlstm_hip
    x, _ = _inputs(1, 2, 128, 32, 32, torch.float32, seed=3)
    h = xlstm_hip.mlstm_chunkwise(*_gpu(x))
    assert isinstance(h, torch.Tensor)
    assert relerr(h, om.mlstm_chunkwise(*x)) <= FP32_REL
    h2 = xlstm_hip.mlstm_chunkwise__native_autograd(*_gpu(x), chunk_size=32,
                                                    autocast_kernel_dtype=torch.bfloat16)
    assert relerr(h2, om.mlstm_chunkwise(*x, chunk_size=32)) <= FP32_REL


def test_errors(gpu_case):
    import xlstm_hip
    x, _ = _inputs(1, 2, 100, 32, 32, torch.float32, seed=3)
    with pytest.raises(AssertionError, match="not divisible"):
        xlstm_hip.mlstm_chunkwise(*_gpu(x), chunk_size=64)
    x, _ = _inputs(1, 2, 96, 32, 32, torch.float32, seed=3)
    with pytest.raises(NotImplementedError):
        xlstm_hip.mlstm_chunkwise(*_gpu(x), chunk_size=48)


@pytest.mark.parametrize("L", [64, 128])
def test_cfg2_full_size_prefix_and_invariance(gpu_case, L):
    import xlstm_hip
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    x = chunkwise_inputs(CFG2)
    xd = _gpu(x)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*xd, return_last_states=True, chunk_size=L)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(h).all()) and bool(torch.isfinite(C).all())
    # causal prefix: the first 512 tokens of heads (0,0) and (3,7) against the oracle
    P = 512
    for b, hh in ((0, 0), (3, 7)):
        xs = tuple(t[b:b + 1, hh:hh + 1, :P] for t in x)
        hr = om.mlstm_chunkwise(*(t.float() for t in xs), chunk_size=L)
        e = lowp_excess(h[b:b + 1, hh:hh + 1, :P], hr)
        print(f"cfg2 L={L} prefix head ({b},{hh}): max-abs beyond rounding {e:.3e}")
        assert e <= LOWP_ABS
    # final states: the two algorithms and the two chunk sizes agree
    h2, (C2, n2, m2) = xlstm_hip.mlstm_chunkwise(*xd, return_last_states=True, chunk_size=L, algo="two_pass")
    h3, (C3, n3, m3) = xlstm_hip.mlstm_chunkwise(*xd, return_last_states=True, chunk_size=192 - L)
    # two 16-bit outputs may each be half an ulp off the exact value: allow a full ulp between them
    for a, b_ in ((h, h2), (h, h3)):
        d = (a.double().cpu() - b_.double().cpu()).abs()
        assert float((d - 2 * half_ulp(b_.double(), torch.bfloat16)).max()) <= LOWP_ABS
    for a, b_, c in ((C, C2, C3), (n, n2, n3), (m, m2, m3)):
        assert maxabs(a, b_) <= LOWP_ABS and maxabs(a, c) <= LOWP_ABS


@pytest.mark.parametrize("shape", [(1, 2, 128, 256, 64), (2, 2, 256, 128, 128), (1, 3, 512, 256, 192),
                                   (1, 1, 64, 128, 64)])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("algo", SINGLE_PASS)
def test_fused_vs_oracle(gpu_case, shape, with_state, gate_dtype, algo):
    import xlstm_hip
    B, NH, S, DQK, DV = shape
    x, st = _inputs(B, NH, S, DQK, DV, torch.bfloat16, seed=S + DV, with_state=with_state)
    x = x[:3] + tuple(t.to(gate_dtype) for t in x[3:])
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=64,
                                             algo=algo)
    hr, (Cr, nr, mr) = _oracle(x, st, 64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        e = lowp_excess(got, want)
        print(f"{algo} {shape} state={with_state} {gate_dtype} {name}: max-abs {maxabs(got, want):.3e}, "
              f"beyond output rounding {e:.3e}")
        assert e <= LOWP_ABS, name


@pytest.mark.parametrize("algo", SINGLE_PASS)
def test_fused_strong_forget_gates(gpu_case, algo):
    """Strongly negative forget gates and large input gates: the stabiliser path."""
    import xlstm_hip
    B, NH, S, DQK, DV = 1, 2, 256, 256, 64
    x, _ = _inputs(B, NH, S, DQK, DV, torch.bfloat16, seed=99)
    g = torch.Generator().manual_seed(100)
    i = (15 * torch.tanh(4 * torch.randn(B, NH, S, generator=g) / 15)).to(torch.bfloat16)
    f = (15 * torch.tanh(6 * torch.randn(B, NH, S, generator=g) / 15)).to(torch.bfloat16)
    x = x[:3] + (i, f)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), return_last_states=True, algo=algo)
    hr, (Cr, nr, mr) = _oracle(x, (None, None, None), 64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        e = lowp_excess(got, want)
        print(f"{algo} strong gates {name}: max-abs {maxabs(got, want):.3e}, beyond output rounding {e:.3e}")
        assert e <= LOWP_ABS, name


@pytest.mark.parametrize("L", [64, 128])
@pytest.mark.parametrize("algo", SINGLE_PASS)
def test_cfg2_full_size_vs_oracle(gpu_case, L, algo):
    """cfg2 at full size, fused path, against the oracle at the same chunk size on the whole batch
    (h and final states).  chunk_size=128 runs on the fused kernel's 64-token chunks: the forward is
    chunk-size invariant, so only rounding separates it from the oracle's 128-token chunks."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    x = chunkwise_inputs(CFG2)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), return_last_states=True, chunk_size=L, algo=algo)
    if L not in _cfg2_oracle:
        _cfg2_oracle[L] = _oracle(x, (None, None, None), L)
    hr, (Cr, nr, mr) = _cfg2_oracle[L]
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        e = lowp_excess(got, want)
        print(f"cfg2 full {algo} L={L} {name}: max-abs {maxabs(got, want):.3e}, beyond output rounding {e:.3e}, "
              f"rel {relerr(got, want):.3e}")
        assert e <= LOWP_ABS, name


@pytest.mark.parametrize("L", [16, 32, 128])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("algo", SINGLE_PASS)
def test_fused_other_chunk_sizes(gpu_case, L, with_state, algo):
    """chunk_size 16, 32 and 128 on the fused kernel (S a multiple of 64) against the oracle at that chunk size."""
    import xlstm_hip
    B, NH, S, DQK, DV = 1, 2, 256, 256, 128
    x, st = _inputs(B, NH, S, DQK, DV, torch.bfloat16, seed=L + with_state, with_state=with_state)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=L,
                                             algo=algo)
    hr, (Cr, nr, mr) = _oracle(x, st, L)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, torch.bfloat16, f"{algo} L={L} state={with_state} {name}")


@pytest.mark.parametrize("S", [1, 5, 63, 65, 100, 200, 1000])
@pytest.mark.parametrize("DQK,DV", [(256, 64), (128, 128)])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("algo", SINGLE_PASS)
def test_fused_ragged_length(gpu_case, S, DQK, DV, with_state, algo):
    """algo="fused" takes any S (64-token chunks, ragged last chunk), against the oracle's any-S
    driver (chunkwise pieces of 64/32/16 tokens, then the recurrent tail) on the same inputs."""
    import xlstm_hip
    x, st = _inputs(1, 2, S, DQK, DV, torch.bfloat16, seed=S + DQK, with_state=with_state)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=64,
                                             algo=algo)
    q, k, v, i, f = (t.float() for t in x)
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, *st, chunk_size=64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, torch.bfloat16, f"{algo} ragged S={S} DQK={DQK} DV={DV} state={with_state} {name}")
    # auto and two_pass keep the reference's contract
    if S % 64:
        with pytest.raises(AssertionError, match="not divisible"):
            xlstm_hip.mlstm_chunkwise(*_gpu(x), chunk_size=64)


@pytest.mark.parametrize("S", [37, 100, 8255])
def test_backend_any_length_bf16(gpu_case, S):
    """mLSTMBackend inference on bf16 inputs: one fused call for any S (the any-S wrapper's fast
    path), against the oracle's any-S driver; S = 8255 is config 2's heads of one batch row with
    the worst tail (32 + 16 + 15 tokens after 8192)."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    if S == 8255:
        x = chunkwise_inputs(CFG2, S=S, B=1)
    else:
        x, _ = _inputs(1, 2, S, 256, 128, torch.bfloat16, seed=S)
    backend = xlstm_hip.mLSTMBackend(xlstm_hip.mLSTMBackendConfig(mode="inference", chunk_size=64))
    h, (C, n, m) = backend(*_gpu(x))
    q, k, v, i, f = (t.float() for t in x)
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, chunk_size=64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got, want, torch.bfloat16, f"backend any-S bf16 S={S} {name}")


def test_auto_fallback_warns_once(gpu_case):
    """algo="auto" with a head shape the single-pass kernels do not take (DV 48) runs the two-pass
    kernels and says so once (a RuntimeWarning naming the reason), still within the parity bar."""
    import warnings

    import xlstm_hip
    from xlstm_hip import ops
    ops._fallback_warned.clear()
    x, st = _inputs(1, 2, 128, 64, 48, torch.float16, seed=77)
    with pytest.warns(RuntimeWarning, match="two-pass"):
        h = xlstm_hip.mlstm_chunkwise(*_gpu(x))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        xlstm_hip.mlstm_chunkwise(*_gpu(x))  # the same reason is not repeated
    assert_parity(h.cpu(), _oracle(x, st, 64)[0], torch.float16, "f16 two-pass h")


@pytest.mark.parametrize("B,NH,S,DQK,DV,with_state", [
    (1, 2, 2048, 256, 128, False),   # 4 (head, tile) pairs: 8 segments of 4 chunks
    (1, 2, 2048, 256, 128, True),
    (2, 1, 1000, 128, 64, True),     # ragged last chunk inside the last segment
    (1, 8, 2048, 256, 512, True),    # config 3's heads: 4 segments of 8 chunks
    (1, 1, 300, 256, 64, False),     # 5 chunks: too short to split
])
@pytest.mark.parametrize("algo", SINGLE_PASS)
def test_fused_sequence_split(gpu_case, B, NH, S, DQK, DV, with_state, algo):
    """Few heads: the fused kernel splits the sequence into segments (a states-only pass, the
    segment combine, then all segments at once from their start states).  h and the last C, n, m
    against the oracle's any-S driver, and the workspace grows by the per-segment states."""
    import xlstm_hip
    from xlstm_hip.ops import chunkwise_workspace_bytes
    x, st = _inputs(B, NH, S, DQK, DV, torch.bfloat16, seed=S + NH, with_state=with_state)
    ws = chunkwise_workspace_bytes(B, NH, S, DQK, DV, 64, torch.bfloat16, algo=algo)
    prep = ((B * NH * ((S + 63) // 64) * 1280 + 255) // 256) * 256
    assert (ws > prep) == (B * NH * DV // 64 < 256 and (S + 63) // 64 >= 8)
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, algo=algo)
    q, k, v, i, f = (t.float() for t in x)
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, *st, chunk_size=64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got.cpu(), want, torch.bfloat16, f"{algo} split B{B} NH{NH} S{S} DQK{DQK} DV{DV} {name}")


@pytest.mark.parametrize("B,NH,S,DQK,DV,with_state", [
    (1, 2, 256, 256, 128, False), (1, 2, 256, 256, 128, True), (2, 2, 320, 128, 64, True),
    (1, 1, 100, 256, 64, True),     # ragged last chunk
    (1, 2, 1000, 128, 128, False),
    (1, 1, 5, 256, 64, True),
    (1, 8, 2048, 256, 512, True),   # config 3's heads: the sequence split into 4 segments
])
def test_f16_pipelined(gpu_case, B, NH, S, DQK, DV, with_state):
    """float16 q/k/v run the pipelined kernel (f16 MFMA operands, float32 operands as f16 hi + lo
    pairs, the stored state renormalised at every chunk instead of the deferred rescale): h and
    the last C, n, m against the oracle's any-S driver on the same f16 inputs, any S, with and
    without initial states and with the sequence split."""
    import xlstm_hip
    x, st = _inputs(B, NH, S, DQK, DV, torch.float16, seed=S + DQK + 1, with_state=with_state)
    if S % 64 == 0:
        assert xlstm_hip.chunkwise_algorithm(B, NH, S, DQK, DV, 64, torch.float16) == "pipelined"
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=64,
                                             algo="pipelined")
    assert h.dtype == torch.float16
    q, k, v, i, f = (t.float() for t in x)
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, *st, chunk_size=64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got.cpu(), want, torch.float16, f"f16 B{B} NH{NH} S{S} DQK{DQK} DV{DV} state={with_state} {name}")


@pytest.mark.parametrize("case", ["wide_values", "strong_forget", "weak_forget"])
def test_f16_pipelined_ranges(gpu_case, case):
    """The f16 kernel where its range matters: q, k, v scaled up (|v| ~ 8, |k| ~ 2: the state and
    alpha' V far from 1), forget gates near 0 (every chunk renormalises a large decay) and near
    saturation (the state keeps its whole history)."""
    import xlstm_hip
    B, NH, S, DQK, DV = 1, 2, 640, 256, 128
    g = torch.Generator().manual_seed(99)
    q = torch.randn(B, NH, S, DQK, generator=g) / DQK ** 0.5
    k = torch.randn(B, NH, S, DQK, generator=g)
    v = torch.randn(B, NH, S, DV, generator=g)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    if case == "wide_values":
        k, v = 2 * k, 8 * v
    elif case == "strong_forget":
        f = torch.randn(B, NH, S, generator=g) - 2
    else:
        f = torch.randn(B, NH, S, generator=g) + 8
    x = [t.to(torch.float16) for t in (q, k, v, i, f)]
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), return_last_states=True, chunk_size=64, algo="pipelined")
    assert bool(torch.isfinite(h).all()) and bool(torch.isfinite(C).all())
    hr, (Cr, nr, mr) = _oracle(x, (None, None, None), 64)
    scale = max(1.0, float(hr.abs().max()) / 16)  # wide values: the bar relative to |h| ~ 16
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        e = lowp_excess(got.cpu(), want) / (scale if name in ("h", "C") else 1.0)
        assert e <= LOWP_ABS, f"f16 {case} {name}: {e:.3e}"


def test_f16_fused_schedule_rejected(gpu_case):
    """The fused schedule is bf16 only: algo="fused" with f16 inputs names the pipelined one."""
    import xlstm_hip
    x, _ = _inputs(1, 2, 128, 256, 64, torch.float16, seed=5)
    with pytest.raises(Exception, match="pipelined"):
        xlstm_hip.mlstm_chunkwise(*_gpu(x), algo="fused")


@pytest.mark.parametrize("S", [37, 100, 1000])
def test_backend_any_length_f16(gpu_case, S):
    """mLSTMBackend inference on f16 inputs: one pipelined call for any S, against the oracle's
    any-S driver on the same f16 inputs."""
    import xlstm_hip
    x, _ = _inputs(1, 2, S, 256, 128, torch.float16, seed=S + 7)
    backend = xlstm_hip.mLSTMBackend(xlstm_hip.mLSTMBackendConfig(mode="inference", chunk_size=64))
    h, (C, n, m) = backend(*_gpu(x))
    assert h.dtype == torch.float16
    q, k, v, i, f = (t.float() for t in x)
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, chunk_size=64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got.cpu(), want, torch.float16, f"backend any-S f16 S={S} {name}")


@pytest.mark.parametrize("B,NH,S,DQK,DV,with_state", [
    (1, 2, 256, 64, 128, True), (2, 2, 320, 32, 64, False), (1, 2, 1000, 96, 128, True),
    (1, 1, 100, 192, 64, True), (1, 2, 37, 64, 64, False),
    (1, 4, 2048, 96, 192, True),   # the sequence split (16 column tiles x 4 heads < 256)
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pipelined_narrow_heads(gpu_case, B, NH, S, DQK, DV, with_state, dtype):
    """Head widths below the pipelined kernel's 128 / 256-row tile (32, 64, 96 in the 128 tile,
    192 in the 256 tile): the tile's rows and columns past DQK stay zero, the state waves past it
    idle.  h and the last states against the oracle's any-S driver, any S, initial states, the
    sequence split, bf16 and f16."""
    import xlstm_hip
    x, st = _inputs(B, NH, S, DQK, DV, dtype, seed=S + DQK + 3, with_state=with_state)
    if S % 64 == 0:
        assert xlstm_hip.chunkwise_algorithm(B, NH, S, DQK, DV, 64, dtype) == "pipelined"
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(*_gpu(x), *_gpu(st), return_last_states=True, chunk_size=64,
                                             algo="pipelined")
    q, k, v, i, f = (t.float() for t in x)
    hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, *st, chunk_size=64)
    for got, want, name in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got.cpu(), want, dtype, f"narrow B{B} NH{NH} S{S} DQK{DQK} DV{DV} {dtype} {name}")
