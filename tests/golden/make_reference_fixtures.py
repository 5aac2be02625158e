"""Writes tests/golden/reference_vectors.npz from the reference's own torch-native code.

Run from the repository root in the build container, where /root/reference is mounted:

    python tests/golden/make_reference_fixtures.py [/root/reference]

Each reference file is loaded by its path (importlib), never through its package: the
packages pull in MLX, Metal extensions or torch.compile at import time.  Files loaded:

* kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent/native_step.py
* kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent/native_sequence.py
  (its relative import of native_step is served from the module loaded above; its optional
  Triton imports fail and are skipped by its own try/except)
* kernel_development/xlstm/mlstm_block/mlstm_chunkwise/vendored/torch/native/fw.py
* xlstm_metal/torch_native/blocks/slstm/slstm_layers/stepwise/slstm_metal_kernel.py

Vectors (small, seeded; 16-bit tensors are stored as their exact float32 values with the
dtype recorded, so the file holds plain arrays only):

* ``step_bf16_*``: one decode step with bf16 q/k/v and float32 gates and states
  (mlstm_recurrent_step__native, native_step.py:105-133): the reference's bf16 roundings;
* ``seq_bf16_*``: a 20-token bf16 sequence from initial states
  (mlstm_recurrent_sequence__native_fw, native_sequence.py:131-170);
* ``cw{16,64}_*``: the float32 chunkwise forward at chunk sizes 16 and 64 with initial
  states and the last states (mlstm_chunkwise, fw.py:372-412);
* ``slstm_*``: five chained float32 sLSTM steps from the zero state with +-10 gates
  (slstm_step_pytorch, slstm_metal_kernel.py:14-65).

Nothing from the reference travels further: the .npz holds inputs and outputs only.
"""

from __future__ import annotations

import importlib.util
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "reference_vectors.npz")

REC = "kernel_development/xlstm/mlstm_block/mlstm_recurrent/recurrent"
VTN = "kernel_development/xlstm/mlstm_block/mlstm_chunkwise/vendored/torch/native"
SLSTM = "xlstm_metal/torch_native/blocks/slstm/slstm_layers/stepwise/slstm_metal_kernel.py"


def _load(name: str, path: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_reference(root: str):
    # a stand-in parent package for native_sequence's relative import (no search path: only
    # modules registered here resolve)
    pkg = types.ModuleType("xlref_rec")
    pkg.__path__ = []
    sys.modules["xlref_rec"] = pkg
    step = _load("xlref_rec.native_step", os.path.join(root, REC, "native_step.py"))
    seq = _load("xlref_rec.native_sequence", os.path.join(root, REC, "native_sequence.py"))
    fw = _load("xlref_vtn_fw", os.path.join(root, VTN, "fw.py"))
    sl = _load("xlref_slstm_step", os.path.join(root, SLSTM))
    return step, seq, fw, sl


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def main(root: str) -> None:
    step, seq, fw, sl = load_reference(root)
    out: dict[str, np.ndarray] = {}

    # one bf16 decode step
    g = torch.Generator().manual_seed(101)
    B, NH, DQK, DV = 2, 2, 32, 32
    q, k = (torch.randn(B, NH, DQK, generator=g).to(torch.bfloat16) for _ in range(2))
    v = torch.randn(B, NH, DV, generator=g).to(torch.bfloat16)
    i = torch.randn(B, NH, 1, generator=g)
    f = torch.randn(B, NH, 1, generator=g) + 3
    c = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n = torch.randn(B, NH, DQK, generator=g).abs()
    m = torch.randn(B, NH, 1, generator=g)
    h, (c1, n1, m1) = step.mlstm_recurrent_step__native(q, k, v, i, f, c, n, m)
    assert h.dtype == torch.bfloat16
    for key, t in dict(q=q, k=k, v=v, i=i, f=f, c=c, n=n, m=m, h=h, c_new=c1, n_new=n1, m_new=m1).items():
        out[f"step_bf16_{key}"] = _f32(t)

    # a 20-token bf16 sequence from initial states
    g = torch.Generator().manual_seed(102)
    B, NH, S, DQK, DV = 1, 2, 20, 32, 32
    q, k = (torch.randn(B, NH, S, DQK, generator=g).to(torch.bfloat16) for _ in range(2))
    v = torch.randn(B, NH, S, DV, generator=g).to(torch.bfloat16)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    c = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n = torch.randn(B, NH, DQK, generator=g).abs()
    m = torch.randn(B, NH, 1, generator=g)
    h, (c1, n1, m1) = seq.mlstm_recurrent_sequence__native_fw(q, k, v, i, f, c, n, m, return_last_states=True)
    for key, t in dict(q=q, k=k, v=v, i=i, f=f, c=c, n=n, m=m, h=h, c_last=c1, n_last=n1, m_last=m1).items():
        out[f"seq_bf16_{key}"] = _f32(t)

    # float32 chunkwise at chunk sizes 16 and 64, with initial and last states
    g = torch.Generator().manual_seed(103)
    B, NH, S, DQK, DV = 1, 2, 128, 32, 32
    q = torch.randn(B, NH, S, DQK, generator=g) / DQK ** 0.5
    k = torch.randn(B, NH, S, DQK, generator=g)
    v = torch.randn(B, NH, S, DV, generator=g)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3
    c = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n = torch.randn(B, NH, DQK, generator=g).abs()
    m = torch.randn(B, NH, 1, generator=g)
    for key, t in dict(q=q, k=k, v=v, i=i, f=f, c=c, n=n, m=m).items():
        out[f"cw_{key}"] = _f32(t)
    for L in (16, 64):
        h, (c1, n1, m1) = fw.mlstm_chunkwise(q, k, v, i, f, c, n, m, return_last_states=True, chunk_size=L)
        for key, t in dict(h=h, c_last=c1, n_last=n1, m_last=m1).items():
            out[f"cw{L}_{key}"] = _f32(t)

    # five chained float32 sLSTM steps from the zero state, gates within +-10
    g = torch.Generator().manual_seed(42)
    B, NH, H, T = 2, 4, 8, 5
    z = torch.randn(T, B, NH, H, generator=g)
    ig, fg, og = (10 * torch.tanh(2 * torch.randn(T, B, NH, generator=g)) for _ in range(3))
    cs, ns, ms = torch.zeros(B, NH, H), torch.zeros(B, NH, H), torch.zeros(B, NH)
    hs = []
    for t in range(T):
        # per-head scalar gates [B, NH], broadcast over H inside the step (slstm_metal_kernel.py:53-56)
        hh, cs, ns, ms = sl.slstm_step_pytorch(z[t], ig[t], fg[t], og[t], cs, ns, ms)
        hs.append(hh)
    for key, t in dict(z=z, i=ig, f=fg, o=og, h=torch.stack(hs), c_last=cs, n_last=ns, m_last=ms).items():
        out[f"slstm_{key}"] = _f32(t)

    out["_source"] = np.array(["REC/native_step.py", "REC/native_sequence.py", "VTN/fw.py",
                               "TNS/stepwise/slstm_metal_kernel.py"])
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
