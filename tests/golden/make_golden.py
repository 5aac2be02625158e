"""Writes the float64 fixtures under tests/golden/ (run from the repo root).

The mLSTM vectors come from ``oracle.canonical_np`` (the numpy restatement
after the reference's ``tests/parity/canonical_reference.py:59-111``), not
from the torch oracle they are used to check.  The soft-cap and gate known
answers are the values the reference's own tests hold:
``kernel_development/soft_cap/mlx_fast_kernels/test_softcap.py:6-56`` and the
input cases of ``tests/parity/test_numerical_parity.py:104-108`` /
``tests/parity/test_parity_simple.py:70-75``; their expected outputs are the
closed form ``cap * tanh(x / cap)`` evaluated with ``math.tanh``.

    python tests/golden/make_golden.py
"""

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import canonical_np as cn  # noqa: E402


def _case(rng, B, NH, S, DK, DV, with_state):
    q = rng.standard_normal((B, NH, S, DK))
    k = rng.standard_normal((B, NH, S, DK))
    v = rng.standard_normal((B, NH, S, DV))
    i = rng.standard_normal((B, NH, S))
    f = rng.standard_normal((B, NH, S)) + 3.0
    if with_state:
        c0 = 0.1 * rng.standard_normal((B, NH, DK, DV))
        n0 = np.abs(rng.standard_normal((B, NH, DK)))
        m0 = rng.standard_normal((B, NH, 1))
    else:
        c0 = np.zeros((B, NH, DK, DV))
        n0 = np.zeros((B, NH, DK))
        m0 = np.zeros((B, NH, 1))
    h, (C, n, m) = cn.recurrent_sequence(q, k, v, i, f, 1e-6, state=(c0, n0, m0))
    return dict(q=q, k=k, v=v, i=i, f=f, c0=c0, n0=n0, m0=m0, h=h, C=C, n=n, m=m)


def main():
    rng = np.random.default_rng(20261201)
    out = {}
    for name, (B, NH, S, DK, DV, L, st) in {
        "a": (1, 2, 48, 8, 8, 16, False),
        "b": (2, 2, 64, 16, 8, 32, True),
    }.items():
        for key, val in _case(rng, B, NH, S, DK, DV, st).items():
            out[f"{name}_{key}"] = val
        out[f"{name}_L"] = np.array(L)
    np.savez_compressed(os.path.join(HERE, "mlstm_small.npz"), **out)

    kat = {
        "soft_cap": [
            # test_softcap.py:6-56 (cap, x, expected, tolerance used there)
            {"cap": 5.0, "x": 0.0, "expect": 0.0, "tol": 1e-5},
            {"cap": 5.0, "x": 5.0, "expect": 3.808, "tol": 0.01},
            {"cap": 5.0, "x": 50.0, "expect": 5.0, "tol": 0.01},
            {"cap": 5.0, "x": -50.0, "expect": -5.0, "tol": 0.01},
            {"cap": 5.0, "x": 0.1, "expect": 0.1, "tol": 0.01},
            {"cap": 2.0, "x": 2.0, "expect": 1.523, "tol": 0.01},
        ],
        "soft_cap_cases": [
            # test_numerical_parity.py:104-108 / test_parity_simple.py:70-75 inputs
            {"cap": 15.0, "x": [-0.5, 0.0, 0.5, 1.0]},
            {"cap": 15.0, "x": [-50.0, -20.0, 20.0, 50.0]},
            {"cap": 30.0, "x": [-100.0, 0.0, 100.0]},
            {"cap": 15.0, "x": [-1.0, 0.0, 1.0, 5.0]},
        ],
    }
    for case in kat["soft_cap_cases"]:
        case["expect"] = [case["cap"] * math.tanh(x / case["cap"]) for x in case["x"]]
    with open(os.path.join(HERE, "kat.json"), "w") as fh:
        json.dump(kat, fh, indent=1)


if __name__ == "__main__":
    main()
