"""C-ABI boundary checks that need no GPU.

* libxlstm_hip.so loads and exports every entry point include/xlstm_hip.h
  declares, with the ABI version the header states;
* argument validation fails with the documented error codes and messages
  before any GPU call (null pointers, bad shapes, aliasing, S % L != 0,
  unsupported chunk sizes) — the failure paths the reference raises for
  (fw.py:303-305, native_step.py:49-67);
* the Python ops refuse CPU tensors (there is no CPU fallback) and the
  registry names mirror the reference's backend names.
"""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "xlstm_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xl_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from xlstm_hip import _lib
    return _lib.load()


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("xl_abi_version", "xl_last_error", "xl_soft_cap_fwd", "xl_mlstm_step_fwd", "xl_mlstm_chunkwise_fwd",
              "xl_mlstm_chunkwise_workspace_size", "xl_mlstm_sequence_fwd", "xl_slstm_step_fwd", "xl_slstm_seq_fwd",
              "xl_causal_conv1d_fwd", "xl_group_norm_fwd", "xl_mh_rmsnorm_gate_fwd", "xl_gate_proj_softcap_fwd"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(lib._name)
    for name in _declared():
        assert hasattr(raw, name), f"{name} declared in include/xlstm_hip.h but not exported"


def test_python_signatures_cover_header(lib):
    from xlstm_hip import _lib
    assert sorted(_lib.SIGNATURES) == _declared()


def test_abi_version_matches_header(lib):
    m = re.search(r"#define XL_ABI_VERSION (\d+)", open(HEADER).read())
    assert lib.xl_abi_version() == int(m.group(1))


def test_soft_cap_rejects_bad_args(lib):
    assert lib.xl_soft_cap_fwd(None, None, -1, 1.0, 0, None) == -1
    assert b"numel" in lib.xl_last_error()
    assert lib.xl_soft_cap_fwd(None, None, 4, 1.0, 7, None) == -1
    assert b"dtype" in lib.xl_last_error()
    assert lib.xl_soft_cap_fwd(None, None, 4, 1.0, 0, None) == -1
    assert b"null" in lib.xl_last_error()
    assert lib.xl_soft_cap_fwd(None, None, 0, 1.0, 0, None) == 0  # empty input is a no-op


def test_step_rejects_bad_args(lib):
    f = lib.xl_mlstm_step_fwd
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    assert f(p, p, p, p, p, p, p, p, p, p, p, p, 0, 8, 256, 512, 0.0625, 1e-6, 1, 0, None) == -1
    assert b"positive" in lib.xl_last_error()
    assert f(p, p, p, p, p, p, p, p, p, p, p, p, 2, 8, 256, 514, 0.0625, 1e-6, 1, 0, None) == -2
    assert f(p, p, p, p, p, p, p, p, p, p, p, p, 2, 8, 1024, 512, 0.0625, 1e-6, 1, 0, None) == -2
    assert f(p, p, p, p, p, None, p, p, p, p, p, p, 2, 8, 256, 512, 0.0625, 1e-6, 1, 0, None) == -1
    assert b"null" in lib.xl_last_error()
    a, b = ctypes.c_void_p(512), ctypes.c_void_p(1024)
    assert f(p, p, p, p, p, a, b, p, p, a, b, ctypes.c_void_p(2048), 2, 8, 256, 512, 0.0625, 1e-6, 1, 0, None) == -1
    assert b"alias" in lib.xl_last_error()
    # the step's copy ceiling (a measurement aid): the step's shape checks, null and alignment
    g = lib.xl_mlstm_step_copy_ceiling
    assert g(p, p, 0, 8, 256, 512, None) == -1
    assert g(p, p, 2, 8, 256, 514, None) == -2
    assert g(None, p, 2, 8, 256, 512, None) == -1 and b"null" in lib.xl_last_error()
    assert g(ctypes.c_void_p(260), p, 2, 8, 256, 512, None) == -1 and b"aligned" in lib.xl_last_error()


def test_chunkwise_rejects_bad_args(lib):
    f = lib.xl_mlstm_chunkwise_fwd
    p = ctypes.c_void_p(256)
    args = lambda S, L, algo=0, c0=None: (p, p, p, p, p, c0, None, None, p, None, None, None, 1, 8, S, 256, 512, L,
                                           0.0625, 1e-6, 1, 1, algo, None, 0, None)
    assert f(*args(250, 64)) == -1
    assert b"not divisible" in lib.xl_last_error()
    assert f(*args(240, 48)) == -2
    assert f(*args(256, 64, algo=9)) == -1
    assert f(*args(256, 64, c0=p)) == -1
    assert b"together" in lib.xl_last_error()
    mis = ctypes.c_void_p(264)  # 8-byte aligned only
    assert f(mis, p, p, p, p, None, None, None, p, None, None, None, 1, 8, 256, 256, 512, 64, 0.0625, 1e-6, 1, 1, 0,
             None, 0, None) == -1
    assert b"16-byte aligned" in lib.xl_last_error()
    assert f(*args(256, 64, algo=1)) == -3  # two-pass without workspace
    assert b"workspace" in lib.xl_last_error()
    # two-pass: per chunk of every head the entering C, n, m and the states pass's 196-float gate prefix
    assert lib.xl_mlstm_chunkwise_workspace_size(1, 8, 256, 256, 512, 64, 0, 1) == (4 * 8 * (256 * 512 + 256 + 1 + 196) * 4 + 255) // 256 * 256
    assert lib.xl_mlstm_chunkwise_workspace_size(1, 8, 250, 256, 512, 64, 0, 1) == 0


def test_chunkwise_bwd_rejects_bad_args(lib):
    f = lib.xl_mlstm_chunkwise_bwd
    p, mis = ctypes.c_void_p(256), ctypes.c_void_p(264)

    def call(q=p, dq=p, L=64, S=256):
        return f(q, p, p, p, p, None, None, None, p, None, dq, p, p, p, p, None, 1, 2, S, 64, 64, L, 0.125, 1e-6, 1,
                 1, None, 0, None)

    assert call(L=128) == -2 and b"chunk_size" in lib.xl_last_error()
    assert call(S=100) == -1 and b"not divisible" in lib.xl_last_error()
    assert call(q=mis) == -1 and b"16-byte aligned" in lib.xl_last_error()
    assert call(dq=mis) == -1 and b"16-byte aligned" in lib.xl_last_error()
    assert call() == -3 and b"workspace" in lib.xl_last_error()


def test_slstm_rejects_bad_args(lib):
    p = ctypes.c_void_p(256)
    assert lib.xl_slstm_step_fwd(p, p, p, p, p, p, p, p, p, p, p, 1, 4, 0, 1e-6, 0, 0, 0, None) == -1
    assert lib.xl_slstm_step_fwd(p, p, p, p, p, p, p, p, p, p, p, 1, 4, 8, 1e-6, 0, 0, 0, None) == -1  # m alias
    assert b"alias" in lib.xl_last_error()
    assert lib.xl_slstm_seq_fwd(p, p, p, p, p, None, None, p, None, None, None, 1, 3, 4, 8, 1e-6, 0, 0, 0, None) == -1


def test_conv1d_and_group_norm_reject_bad_args(lib):
    conv, gn = lib.xl_causal_conv1d_fwd, lib.xl_group_norm_fwd
    p, q = ctypes.c_void_p(256), ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    assert conv(p, p, None, q, 1, -8, 16, 4, 1, 1, None) == -1
    assert b"negative" in lib.xl_last_error()
    assert conv(p, p, None, q, 1, 8, 16, 9, 1, 1, None) == -2
    assert b"kernel size" in lib.xl_last_error()
    assert conv(p, p, None, q, 1, 8, 16, 4, 2, 1, None) == -1
    assert conv(p, p, None, q, 1, 8, 16, 4, 1, 5, None) == -1
    assert conv(p, None, None, q, 1, 8, 16, 4, 1, 1, None) == -1
    assert b"null" in lib.xl_last_error()
    assert conv(p, p, None, ctypes.c_void_p(256 + 64), 1, 8, 16, 4, 1, 1, None) == -1  # y overlaps x
    assert b"alias" in lib.xl_last_error()
    assert conv(None, None, None, None, 0, 8, 16, 4, 1, 1, None) == 0  # empty input is a no-op
    assert gn(p, None, None, q, 4, 0, 16, 1e-6, 1, None) == -1
    assert gn(p, p, None, q, 4, 2, -16, 1e-6, 1, None) == -1
    assert b"bad size" in lib.xl_last_error()
    assert gn(p, None, None, q, 4, 2, 16, -1.0, 1, None) == -1
    assert b"eps" in lib.xl_last_error()
    assert gn(p, None, None, q, 4, 2, 16, 1e-6, 9, None) == -1
    assert gn(None, None, None, None, 4, 2, 16, 1e-6, 1, None) == -1
    assert gn(None, None, None, None, 0, 2, 16, 1e-6, 1, None) == 0
    rn = lib.xl_mh_rmsnorm_gate_fwd
    assert rn(p, None, None, q, 1, -2, 4, 64, 1, 1e-6, 1, None) == -1
    assert rn(p, None, None, q, 1, 2, 4, 64, 2, 1e-6, 1, None) == -1
    assert b"h_layout" in lib.xl_last_error()
    assert rn(p, None, None, q, 1, 2, 4, 64, 1, -1.0, 1, None) == -1
    assert rn(p, None, None, ctypes.c_void_p(256 + 128), 1, 2, 4, 64, 1, 1e-6, 1, None) == -1
    assert b"alias" in lib.xl_last_error()
    assert rn(p, None, None, q, 1, 2, 4, 16384, 1, 1e-6, 1, None) == -2  # 32 vectors per lane
    assert rn(None, None, None, None, 0, 2, 4, 64, 1, 1e-6, 1, None) == 0
    gp = lib.xl_gate_proj_softcap_fwd
    assert gp(p, p, None, q, 4, 64, 8, 15.0, 0, 0, None) == -2  # float32
    assert gp(p, p, None, q, 4, 64, 65, 15.0, 0, 1, None) == -2
    assert gp(p, p, None, q, 4, 12, 8, 15.0, 0, 1, None) == -2
    assert gp(p, p, None, q, -4, 64, 8, 15.0, 0, 1, None) == -1
    assert gp(p, p, None, q, 4, 64, 8, 15.0, 2, 1, None) == -1  # cap_rounding 0 or 1
    assert b"cap_rounding" in lib.xl_last_error()
    assert gp(ctypes.c_void_p(264), p, None, q, 4, 64, 8, 15.0, 0, 1, None) == -1  # misaligned x
    assert b"aligned" in lib.xl_last_error()
    assert gp(None, None, None, None, 0, 64, 8, 15.0, 0, 1, None) == 0


def test_ops_refuse_cpu_tensors():
    import xlstm_hip
    x = torch.randn(8)
    with pytest.raises(RuntimeError, match="GPU"):
        xlstm_hip.soft_cap(x, 5.0)
    q = torch.randn(1, 2, 64, 16)
    i = torch.randn(1, 2, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        xlstm_hip.mlstm_chunkwise(q, q, q, i, i)
    assert xlstm_hip.soft_cap(x, 0.0) is x  # cap <= 0: identity without touching the device


def test_registry_names():
    import xlstm_hip
    assert xlstm_hip.get_mlstm_kernel("chunkwise--native_autograd") is xlstm_hip.mlstm_chunkwise__native_autograd
    assert xlstm_hip.get_mlstm_step_kernel("native") is xlstm_hip.mlstm_recurrent_step__native
    assert xlstm_hip.get_mlstm_sequence_kernel("native_sequence__native") is \
        xlstm_hip.mlstm_recurrent_sequence__native_fw
    with pytest.raises(NotImplementedError):
        xlstm_hip.get_mlstm_kernel("chunkwise--triton_xl_chunk")
    with pytest.raises(ValueError):
        xlstm_hip.mLSTMBackendConfig(chunkwise_kernel="parallel--native_autograd", return_last_states=True)


def test_ops_registered_with_torch_library():
    import xlstm_hip  # noqa: F401
    for name in ("soft_cap", "mlstm_step", "mlstm_step_", "mlstm_chunkwise", "mlstm_sequence", "slstm_step",
                 "slstm_sequence", "causal_conv1d", "group_norm", "mh_rmsnorm_gate", "gate_proj_softcap"):
        assert hasattr(torch.ops.xlstm_hip, name)


def test_fake_tensor_shapes():
    import xlstm_hip  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(2, 4, 128, 32, dtype=torch.bfloat16, device="cuda")
        v = torch.empty(2, 4, 128, 48, dtype=torch.bfloat16, device="cuda")
        g = torch.empty(2, 4, 128, dtype=torch.bfloat16, device="cuda")
        h, c, n, m = torch.ops.xlstm_hip.mlstm_chunkwise(q, q, v, g, g, None, None, None, 0.1, 64, 1e-6, True, 0)
        assert h.shape == (2, 4, 128, 48) and h.dtype == torch.bfloat16
        assert c.shape == (2, 4, 32, 48) and n.shape == (2, 4, 32) and m.shape == (2, 4, 1)
        x = torch.empty(2, 100, 64, dtype=torch.bfloat16, device="cuda")
        w = torch.empty(64, 1, 4, dtype=torch.bfloat16, device="cuda")
        y = torch.ops.xlstm_hip.causal_conv1d(x, w, None, 1)
        assert y.shape == x.shape and y.dtype == x.dtype
        y = torch.ops.xlstm_hip.group_norm(x.view(200, 64), 4, None, None, 1e-6)
        assert y.shape == (200, 64)
        h = torch.empty(2, 4, 100, 16, dtype=torch.bfloat16, device="cuda")
        y = torch.ops.xlstm_hip.mh_rmsnorm_gate(h, None, None, True, 1e-6)
        assert y.shape == (2, 100, 64) and y.dtype == torch.bfloat16
        y = torch.ops.xlstm_hip.gate_proj_softcap(x, torch.empty(8, 64, dtype=torch.bfloat16, device="cuda"), None,
                                                  15.0)
        assert y.shape == (2, 100, 8)


def test_chunkwise_algorithm_query(lib):
    """xl_mlstm_chunkwise_algo names the algorithm auto picks and why it left the fused one."""
    from xlstm_hip import chunkwise_algorithm
    assert chunkwise_algorithm(4, 8, 8192, 256, 512, 64, torch.bfloat16) == "pipelined"
    assert chunkwise_algorithm(4, 8, 8192, 256, 512, 128, torch.bfloat16) == "pipelined"
    assert chunkwise_algorithm(1, 8, 256, 256, 512, 64, torch.float32) == "two_pass"
    assert chunkwise_algorithm(4, 8, 8192, 256, 512, 64, torch.bfloat16, algo="two_pass") == "two_pass"
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 256, 512, 64, 2, 0) == 3  # float16 q/k/v: pipelined
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 256, 512, 64, 2, 2) == -2  # the fused schedule is bf16 only
    assert b"bfloat16" in lib.xl_last_error() and b"pipelined" in lib.xl_last_error()
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 256, 512, 64, 0, 0) == 1  # float32 q/k/v
    assert b"bfloat16 or float16" in lib.xl_last_error()
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 96, 512, 64, 1, 0) == 3  # DQK 96: pipelined, padded tile
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 80, 512, 64, 1, 0) == 1  # DQK 80
    assert b"DQK" in lib.xl_last_error()
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 160, 512, 64, 1, 0) == 1  # DQK 160: not whole 64-row blocks
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 100, 256, 512, 64, 1, 0) == -1  # S % L
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 100, 256, 512, 64, 1, 2) == 2  # fused takes any S
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 256, 512, 48, 1, 0) == -2
    assert lib.xl_mlstm_chunkwise_algo(1, 2, 128, 96, 512, 64, 1, 2) == -2
