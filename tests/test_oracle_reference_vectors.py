"""The oracle against vectors the reference's own code produced (tests/golden/reference_vectors.npz).

The vectors were written in the build container by tests/golden/make_reference_fixtures.py,
which loads the reference's torch-native files by path (REC/native_step.py,
REC/native_sequence.py, VTN/fw.py, TNS/stepwise/slstm_metal_kernel.py) and runs them on small
seeded inputs.  These tests pin what the closed forms and invariants leave open:

* the bf16 semantics of the decode step and the sequence (the casts of C' and n' to q's
  dtype and the bf16 products, native_step.py:78-96) — the oracle reproduces the reference's
  bf16 h bit for bit;
* the float32 chunkwise forward at chunk sizes 16 and 64 with initial and last states
  (fw.py:29-412), to float32 rounding (batched-GEMM accumulation order is the only freedom);
* the float32 sLSTM step over five chained steps with +-10 gates (slstm_metal_kernel.py:14-65).
"""

import os

import numpy as np
import pytest
import torch

from oracle import mlstm as om
from oracle import slstm as osl

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = np.load(os.path.join(HERE, "golden", "reference_vectors.npz"))


def _t(key, dtype=torch.float32):
    return torch.from_numpy(VEC[key]).to(dtype)


def test_vectors_name_their_sources():
    assert set(VEC["_source"].tolist()) == {"REC/native_step.py", "REC/native_sequence.py", "VTN/fw.py",
                                             "TNS/stepwise/slstm_metal_kernel.py"}


def test_bf16_step_bit_exact():
    p = "step_bf16_"
    q, k, v = (_t(p + x, torch.bfloat16) for x in "qkv")
    h, (C, n, m) = om.mlstm_recurrent_step(q, k, v, _t(p + "i"), _t(p + "f"), _t(p + "c"), _t(p + "n"), _t(p + "m"))
    assert h.dtype == torch.bfloat16
    assert torch.equal(h.float(), _t(p + "h"))
    for got, key in ((C, "c_new"), (n, "n_new"), (m, "m_new")):
        assert torch.equal(got, _t(p + key)), key


def test_bf16_sequence_bit_exact():
    p = "seq_bf16_"
    q, k, v = (_t(p + x, torch.bfloat16) for x in "qkv")
    h, (C, n, m) = om.mlstm_recurrent_sequence(q, k, v, _t(p + "i"), _t(p + "f"), _t(p + "c"), _t(p + "n"),
                                               _t(p + "m"), return_last_states=True)
    assert torch.equal(h.float(), _t(p + "h"))
    for got, key in ((C, "c_last"), (n, "n_last"), (m, "m_last")):
        assert torch.equal(got, _t(p + key)), key


@pytest.mark.parametrize("L", [16, 64])
def test_fp32_chunkwise(L):
    x = [_t("cw_" + s) for s in ("q", "k", "v", "i", "f", "c", "n", "m")]
    h, (C, n, m) = om.mlstm_chunkwise(*x, return_last_states=True, chunk_size=L)
    for got, key in ((h, "h"), (C, "c_last"), (n, "n_last"), (m, "m_last")):
        want = _t(f"cw{L}_{key}")
        err = float((got - want).abs().max() / want.abs().max())
        assert err <= 1e-6, f"L={L} {key}: rel-err {err:.2e}"


def test_fp32_chunkwise_differs_from_a_dropped_initial_state():
    # the fixture is sensitive to the initial states: dropping them moves h far beyond 1e-6
    x = [_t("cw_" + s) for s in ("q", "k", "v", "i", "f")]
    h = om.mlstm_chunkwise(*x, chunk_size=64)
    assert float((h - _t("cw64_h")).abs().max()) > 1e-2


def test_fp32_slstm_five_steps():
    z, i, f, o = (_t("slstm_" + s) for s in "zifo")
    T, B, NH, H = z.shape
    c, n, m = torch.zeros(B, NH, H), torch.zeros(B, NH, H), torch.zeros(B, NH)
    hs = []
    for t in range(T):
        h, c, n, m = osl.slstm_step(z[t], i[t], f[t], o[t], c, n, m)
        hs.append(h)
    for got, key in ((torch.stack(hs), "h"), (c, "c_last"), (n, "n_last"), (m, "m_last")):
        want = _t("slstm_" + key)
        err = float((got - want).abs().max() / want.abs().max())
        assert err <= 1e-6, f"sLSTM {key}: rel-err {err:.2e}"
