"""ctypes binding of libxlstm_hip.so (the C-ABI declared in include/xlstm_hip.h).

The library is loaded from ``xlstm_hip/lib/`` (built in-tree by
``xlstm-metal_amd/build.py``).  There is no fallback: if it is missing, every
op raises ``RuntimeError`` telling how to build it.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libxlstm_hip.so")

XL_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
XL_ERRORS = {-1: "invalid argument", -2: "unsupported", -3: "workspace", -4: "launch"}

ALGO = {"auto": 0, "two_pass": 1, "fused": 2, "pipelined": 3}

_vp, _fp, _i, _f, _sz, _i64 = ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_int64

# name -> (restype, argtypes); must match include/xlstm_hip.h
SIGNATURES = {
    "xl_abi_version": (_i, []),
    "xl_last_error": (ctypes.c_char_p, []),
    "xl_soft_cap_fwd": (_i, [_vp, _vp, _i64, _f, _i, _vp]),
    "xl_mlstm_step_fwd": (_i, [_vp] * 5 + [_fp] * 3 + [_vp] + [_fp] * 3 + [_i] * 4 + [_f, _f] + [_i, _i, _vp]),
    "xl_mlstm_step_copy_ceiling": (_i, [_fp, _fp] + [_i] * 4 + [_vp]),
    "xl_mlstm_chunkwise_workspace_size": (_sz, [_i] * 8),
    "xl_mlstm_chunkwise_algo": (_i, [_i] * 8),
    "xl_mlstm_chunkwise_fwd": (_i, [_vp] * 5 + [_fp] * 3 + [_vp] + [_fp] * 3 + [_i] * 6 + [_f, _f] + [_i] * 3
                               + [_vp, _sz, _vp]),
    "xl_mlstm_chunkwise_bwd_workspace_size": (_sz, [_i] * 6),
    "xl_mlstm_chunkwise_bwd": (_i, [_vp] * 5 + [_fp] * 3 + [_vp, _fp] + [_vp] * 5 + [_fp] + [_i] * 6 + [_f, _f]
                               + [_i, _i, _vp, _sz, _vp]),
    "xl_mlstm_chunkwise_noalloc_max_bytes": (_sz, []),
    "xl_mlstm_chunkwise_fwd_noalloc": (_i, [_vp] * 5 + [_fp] * 3 + [_vp] + [_fp] * 3 + [_i] * 6 + [_f, _f] + [_i] * 2
                                       + [_vp]),
    "xl_mlstm_sequence_fwd": (_i, [_vp] * 5 + [_fp] * 3 + [_vp] + [_fp] * 3 + [_i] * 5 + [_f, _f] + [_i, _i, _vp]),
    "xl_slstm_step_fwd": (_i, [_vp] * 4 + [_fp] * 3 + [_vp] + [_fp] * 3 + [_i] * 3 + [_f] + [_i] * 3 + [_vp]),
    "xl_slstm_seq_fwd": (_i, [_vp] * 4 + [_fp] * 3 + [_vp] + [_fp] * 3 + [_i] * 4 + [_f] + [_i] * 3 + [_vp]),
    "xl_causal_conv1d_fwd": (_i, [_vp] * 4 + [_i] * 6 + [_vp]),
    "xl_group_norm_fwd": (_i, [_vp] * 4 + [_i64, _i, _i, _f, _i, _vp]),
    "xl_mh_rmsnorm_gate_fwd": (_i, [_vp] * 4 + [_i] * 5 + [_f, _i, _vp]),
    "xl_gate_proj_softcap_fwd": (_i, [_vp] * 4 + [_i] * 3 + [_f, _i, _i, _vp]),
    "xl_lm_head_softcap_fwd": (_i, [_vp] * 3 + [_i] * 3 + [_f, _i, _vp]),
}

ABI_VERSION = 2

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads the library once and declares every signature; raises if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"xlstm_hip: HIP library not found at {path}; build it with "
                "`python xlstm-metal_amd/build.py` (there is no CPU fallback)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.xl_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"xlstm_hip: library ABI {ver} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raises ``RuntimeError(xl_last_error())`` for a non-zero status."""
    if rc != 0:
        msg = load().xl_last_error().decode(errors="replace")
        kind = XL_ERRORS.get(rc, f"code {rc}")
        if rc == -1:
            raise ValueError(f"{what}: {msg} ({kind})")
        if rc == -2:
            raise NotImplementedError(f"{what}: {msg} ({kind})")
        raise RuntimeError(f"{what}: {msg} ({kind})")


def dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return XL_DTYPE[t.dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {t.dtype} (float32, bfloat16, float16)") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor | None, what: str) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{what}: tensors must be on the GPU (got {t.device}); there is no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} vs {t.device})")
