"""Pins the CPU oracle of the mLSTM kernels (no GPU).

Each check is chosen so that a plausible mistake in the oracle (a dropped
gate term, a sign, an off-by-one in the cumulative forget sum, a transposed
operand, a wrong stabiliser) fails at least one of them:

* chunkwise == recurrent loop (float64, with and without initial states);
* chunk-size invariance;
* chunkwise == quadratic parallel form at eps = 0 (the stabiliser cancels);
* chunkwise == the stabiliser-free brute-force closed form;
* torch recurrent step == the independent numpy restatement
  (``oracle.canonical_np``, after ``tests/parity/canonical_reference.py``);
* single-token and q = 0 closed forms;
* the gate and denominator known answers of the reference's
  ``tests/test_mlx_torch_numerical_parity.py:8-73``;
* committed float64 fixtures (``tests/golden/mlstm_small.npz``).
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import canonical_np as cn
from oracle import mlstm as om

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _inputs(B, NH, S, DK, DV, seed, dtype=torch.float64, fmean=3.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, NH, S, DK, generator=g, dtype=dtype)
    k = torch.randn(B, NH, S, DK, generator=g, dtype=dtype)
    v = torch.randn(B, NH, S, DV, generator=g, dtype=dtype)
    i = torch.randn(B, NH, S, generator=g, dtype=dtype)
    f = torch.randn(B, NH, S, generator=g, dtype=dtype) + fmean
    return q, k, v, i, f


def _states(B, NH, DK, DV, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed + 1000)
    C = 0.1 * torch.randn(B, NH, DK, DV, generator=g, dtype=dtype)
    n = torch.randn(B, NH, DK, generator=g, dtype=dtype).abs()
    m = torch.randn(B, NH, 1, generator=g, dtype=dtype)
    return C, n, m


@pytest.mark.parametrize("L", [16, 32, 64])
@pytest.mark.parametrize("with_state", [False, True])
def test_chunkwise_equals_recurrent_loop(L, with_state):
    B, NH, S, DK, DV = 2, 2, 128, 16, 24
    q, k, v, i, f = _inputs(B, NH, S, DK, DV, seed=L)
    st = _states(B, NH, DK, DV, seed=L) if with_state else (None, None, None)
    h1, (C1, n1, m1) = om.mlstm_chunkwise(q, k, v, i, f, *st, return_last_states=True, chunk_size=L)
    h2, (C2, n2, m2) = om.mlstm_recurrent_sequence(q, k, v, i, f, *st, return_last_states=True,
                                                    dtype_state=torch.float64)
    torch.testing.assert_close(h1, h2, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(C1, C2, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(n1, n2, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(m1, m2, rtol=0, atol=1e-12)


def test_chunk_size_invariance():
    B, NH, S, DK, DV = 1, 3, 256, 32, 16
    q, k, v, i, f = _inputs(B, NH, S, DK, DV, seed=7)
    C0, n0, m0 = _states(B, NH, DK, DV, seed=7)
    ref = om.mlstm_chunkwise(q, k, v, i, f, C0, n0, m0, return_last_states=True, chunk_size=16)
    for L in (32, 64, 128, 256):
        out = om.mlstm_chunkwise(q, k, v, i, f, C0, n0, m0, return_last_states=True, chunk_size=L)
        torch.testing.assert_close(out[0], ref[0], rtol=1e-9, atol=1e-10)
        for a, b in zip(out[1], ref[1]):
            torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-10)


def test_chunkwise_equals_parallel_form_at_zero_eps():
    q, k, v, i, f = _inputs(2, 2, 128, 16, 16, seed=3, fmean=1.0)
    hp, _, _ = om.mlstm_parallel_fw(q, k, v, i, f, eps=0.0)
    hc = om.mlstm_chunkwise(q, k, v, i, f, chunk_size=32, eps=0.0)
    torch.testing.assert_close(hc, hp, rtol=1e-9, atol=1e-10)


@pytest.mark.parametrize("eps", [0.0, 1e-6, 1e-2])
def test_chunkwise_equals_brute_force_closed_form(eps):
    q, k, v, i, f = _inputs(1, 2, 64, 8, 8, seed=11)
    hb = cn.brute_force_h(q.numpy(), k.numpy(), v.numpy(), i.numpy(), f.numpy(), eps)
    hc = om.mlstm_chunkwise(q, k, v, i, f, chunk_size=16, eps=eps)
    np.testing.assert_allclose(hc.numpy(), hb, rtol=1e-9, atol=1e-11)


def test_recurrent_step_matches_numpy_restatement():
    B, NH, S, DK, DV = 2, 3, 20, 16, 8
    q, k, v, i, f = _inputs(B, NH, S, DK, DV, seed=5)
    C0, n0, m0 = _states(B, NH, DK, DV, seed=5)
    h1, (C1, n1, m1) = om.mlstm_recurrent_sequence(q, k, v, i, f, C0, n0, m0, return_last_states=True,
                                                    dtype_state=torch.float64)
    h2, (C2, n2, m2) = cn.recurrent_sequence(q.numpy(), k.numpy(), v.numpy(), i.numpy(), f.numpy(), 1e-6,
                                             state=(C0.numpy(), n0.numpy(), m0.numpy()))
    np.testing.assert_allclose(h1.numpy(), h2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(C1.numpy(), C2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(n1.numpy(), n2, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(m1.numpy(), m2, rtol=0, atol=1e-12)


def test_single_token_closed_form():
    q, k, v, i, f = _inputs(1, 1, 1, 16, 4, seed=9)
    eps = 1e-6
    h = om.mlstm_chunkwise(q, k, v, i, f, chunk_size=1, eps=eps)
    lsf = -math.log1p(math.exp(-float(f[0, 0, 0])))
    m = max(lsf, float(i[0, 0, 0]))
    ia = math.exp(float(i[0, 0, 0]) - m)
    qk = float(q[0, 0, 0] @ k[0, 0, 0]) / 4.0
    expect = ia * qk * v[0, 0, 0].numpy() / (max(abs(ia * qk), math.exp(-m)) + eps)
    np.testing.assert_allclose(h[0, 0, 0].numpy(), expect, rtol=1e-12, atol=1e-14)


def test_zero_query_gives_zero_output():
    q, k, v, i, f = _inputs(1, 2, 64, 8, 8, seed=4)
    C0, n0, m0 = _states(1, 2, 8, 8, seed=4)
    h = om.mlstm_chunkwise(torch.zeros_like(q), k, v, i, f, C0, n0, m0, chunk_size=16)
    assert torch.count_nonzero(h) == 0


def test_gate_known_answers():
    # Points and formulas of tests/test_mlx_torch_numerical_parity.py:8-46.
    x = torch.tensor([-50.0, -10.0, -1.0, 0.0, 1.0, 10.0, 50.0], dtype=torch.float64)
    expect = [-math.log1p(math.exp(-float(t))) if t > -30 else float(t) - math.log1p(math.exp(float(t)))
              for t in x]
    np.testing.assert_allclose(torch.nn.functional.logsigmoid(x).numpy(), expect, rtol=1e-14)
    iv = torch.tensor([[-10.0], [0.0], [10.0]], dtype=torch.float64)
    fv = torch.tensor([[-10.0], [0.0], [10.0]], dtype=torch.float64)
    mv = torch.tensor([[0.0], [5.0], [-5.0]], dtype=torch.float64)
    # one step with zero C/n: the oracle's new m must be max(logsig f + m, i)
    _, (_, _, m_new) = om.mlstm_recurrent_step(
        torch.zeros(3, 1, 4, dtype=torch.float64), torch.zeros(3, 1, 4, dtype=torch.float64),
        torch.zeros(3, 1, 2, dtype=torch.float64), iv[:, None], fv[:, None],
        torch.zeros(3, 1, 4, 2, dtype=torch.float64), torch.zeros(3, 1, 4, dtype=torch.float64),
        mv[:, None], dtype_state=torch.float64)
    lsf = [-math.log1p(math.exp(10.0)), -math.log(2.0), -math.log1p(math.exp(-10.0))]
    expect_m = [max(lsf[0] + 0.0, -10.0), max(lsf[1] + 5.0, 0.0), max(lsf[2] - 5.0, 10.0)]
    np.testing.assert_allclose(m_new.reshape(-1).numpy(), expect_m, rtol=1e-14)


def test_denominator_floor_known_answer():
    # tests/test_mlx_torch_numerical_parity.py:49-73: tiny q.n, m = 10 -> floor exp(-10) + eps.
    B, NH, DK, DV = 1, 1, 3, 2
    q = torch.full((B, NH, DK), 1e-8, dtype=torch.float64) * math.sqrt(DK)  # q_scaled = 1e-8
    n = torch.tensor([[[1e-8, -1e-8, 0.0]]], dtype=torch.float64)
    m = torch.tensor([[[10.0]]], dtype=torch.float64)
    # f -> +inf keeps m' = m and n' = n, i -> -inf adds nothing
    h, (_, n_new, m_new) = om.mlstm_recurrent_step(
        q, torch.zeros_like(q), torch.ones(B, NH, DV, dtype=torch.float64),
        torch.tensor([[[-1e4]]], dtype=torch.float64), torch.tensor([[[1e4]]], dtype=torch.float64),
        torch.ones(B, NH, DK, DV, dtype=torch.float64), n, m, dtype_state=torch.float64)
    assert float(m_new) == 10.0
    qn = float((q / math.sqrt(DK) * n_new).sum())
    denom = max(abs(qn), math.exp(-10.0)) + 1e-6
    np.testing.assert_allclose(h.reshape(-1).numpy(), [3e-8 / denom] * DV, rtol=1e-12)


def test_arbitrary_length_matches_sequence_loop():
    for S in (1, 5, 16, 37, 64, 100, 129):
        q, k, v, i, f = _inputs(1, 2, S, 8, 8, seed=S)
        C0, n0, m0 = _states(1, 2, 8, 8, seed=S)
        h1, st1 = om.arbitrary_length(q, k, v, f, i, C0, n0, m0, chunk_size=64, dtype_state=torch.float64)
        h2, st2 = om.mlstm_recurrent_sequence(q, k, v, i, f, C0, n0, m0, return_last_states=True,
                                              dtype_state=torch.float64)
        torch.testing.assert_close(h1, h2.to(h1.dtype), rtol=1e-9, atol=1e-10)
        for a, b in zip(st1, st2):
            torch.testing.assert_close(a, b.to(a.dtype), rtol=1e-9, atol=1e-10)


def test_golden_fixture_small():
    path = os.path.join(GOLDEN, "mlstm_small.npz")
    z = np.load(path)
    for name in ("a", "b"):
        q, k, v, i, f = (torch.from_numpy(z[f"{name}_{t}"]) for t in ("q", "k", "v", "i", "f"))
        st = tuple(torch.from_numpy(z[f"{name}_{t}"]) for t in ("c0", "n0", "m0"))
        L = int(z[f"{name}_L"])
        h, (C, n, m) = om.mlstm_chunkwise(q, k, v, i, f, *st, return_last_states=True, chunk_size=L)
        np.testing.assert_allclose(h.numpy(), z[f"{name}_h"], rtol=1e-9, atol=1e-11)
        np.testing.assert_allclose(C.numpy(), z[f"{name}_C"], rtol=1e-9, atol=1e-11)
        np.testing.assert_allclose(n.numpy(), z[f"{name}_n"], rtol=1e-9, atol=1e-11)
        np.testing.assert_allclose(m.numpy(), z[f"{name}_m"], rtol=0, atol=1e-12)


@pytest.mark.parametrize("with_state", [False, True])
def test_recurrent_kernel_cell_equals_sequence(with_state):
    """mLSTMRecurrentKernelCell (mlstm_recurrent_kernel_cell.py:53-161) and native_sequence.py are the
    same recurrence: the two restatements agree in float64 (m carried as [B, NH] vs [B, NH, 1])."""
    g = torch.Generator().manual_seed(17)
    B, NH, S, DQK, DV = 2, 3, 11, 16, 8
    dt = torch.float64
    q, k = (torch.randn(B, NH, S, DQK, generator=g, dtype=dt) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g, dtype=dt)
    i = 3 * torch.randn(B, NH, S, generator=g, dtype=dt)
    f = 3 * torch.randn(B, NH, S, generator=g, dtype=dt) + 1
    state = None
    if with_state:
        state = (0.3 * torch.randn(B, NH, DQK, DV, generator=g, dtype=dt),
                 torch.randn(B, NH, DQK, generator=g, dtype=dt).abs(), torch.randn(B, NH, generator=g, dtype=dt))
    h, (C, n, m) = om.mlstm_recurrent_kernel_cell(q, k, v, i, f, state)
    init = (None, None, None) if state is None else (state[0], state[1], state[2][:, :, None])
    hr, (Cr, nr, mr) = om.mlstm_recurrent_sequence(q, k, v, i, f, *init, return_last_states=True, dtype_state=dt)
    for a, b in ((h, hr), (C, Cr), (n, nr), (m, mr[:, :, 0])):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
