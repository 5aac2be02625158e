"""``torch.library`` operators ``xlstm_hip::*`` backed by libxlstm_hip.so.

Each op validates shapes and dtypes in Python, allocates its outputs with
torch's caching allocator (the library itself never allocates), passes raw
pointers and the current HIP stream through the C-ABI and returns without
synchronising.  Fake (meta) implementations make the ops traceable.  There is
no CPU path: CPU tensors raise.
"""

from __future__ import annotations

import warnings
from typing import Optional

import torch
from torch import Tensor

from . import _lib

__all__ = [
    "soft_cap_op", "mlstm_step_op", "mlstm_step_inplace_op", "mlstm_chunkwise_op", "mlstm_chunkwise_bwd_op", "mlstm_sequence_op",
    "slstm_step_op", "slstm_sequence_op", "causal_conv1d_op", "group_norm_op", "mh_rmsnorm_gate_op",
    "gate_proj_softcap_op", "lm_head_softcap_op", "chunkwise_workspace_bytes", "chunkwise_algorithm",
]

_EMPTY_SHAPE = (0,)


def _prep(t: Tensor, align: int = 16) -> Tensor:
    t = t.contiguous()
    if t.data_ptr() % align:
        t = t.clone()
    return t


def _f32(t: Optional[Tensor]) -> Optional[Tensor]:
    if t is None:
        return None
    return _prep(t if t.dtype == torch.float32 else t.to(torch.float32))


def _check(cond: bool, what: str, msg: str) -> None:
    if not cond:
        raise ValueError(f"{what}: {msg}")


# --------------------------------------------------------------------- soft_cap
@torch.library.custom_op("xlstm_hip::soft_cap", mutates_args=())
def soft_cap_op(x: Tensor, cap: float) -> Tensor:
    _lib.require_gpu(x, what="soft_cap")
    x = _prep(x)
    y = torch.empty_like(x)
    rc = _lib.load().xl_soft_cap_fwd(x.data_ptr(), y.data_ptr(), x.numel(), float(cap),
                                      _lib.dtype_code(x, "soft_cap"), _lib.stream_of(x))
    _lib.check(rc, "soft_cap")
    return y


@soft_cap_op.register_fake
def _(x, cap):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


# ---------------------------------------------------------------- mLSTM step
def _step_shapes(q, k, v, i, f, c, n, m, what):
    _check(q.dim() == 3, what, f"q must be (B, NH, DHQK), got {tuple(q.shape)}")
    B, NH, DQK = q.shape
    DV = v.shape[-1]
    _check(k.shape == q.shape, what, "q and k must have the same shape")
    _check(v.dim() == 3 and v.shape[:2] == (B, NH), what, f"v must be (B, NH, DHV), got {tuple(v.shape)}")
    _check(q.dtype == k.dtype == v.dtype, what, "q, k, v must share a dtype")
    _check(c.shape == (B, NH, DQK, DV), what, f"matC_old has wrong shape, got {tuple(c.shape)}")
    _check(n.shape == (B, NH, DQK), what, f"vecN_old has wrong shape, got {tuple(n.shape)}")
    _check(m.numel() == B * NH, what, f"scaM_old has wrong shape, got {tuple(m.shape)}")
    _check(i.numel() == B * NH, what, f"scaI has wrong shape, got {tuple(i.shape)}")
    _check(f.numel() == B * NH, what, f"scaF has wrong shape, got {tuple(f.shape)}")
    _check(i.dtype == f.dtype, what, "i and f must share a dtype")
    return B, NH, DQK, DV


def _launch_step(q, k, v, i, f, c, n, m, h, c_new, n_new, m_new, B, NH, DQK, DV, qk_scale, eps, what):
    rc = _lib.load().xl_mlstm_step_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(),
        c.data_ptr(), n.data_ptr(), m.data_ptr(), h.data_ptr(), c_new.data_ptr(), n_new.data_ptr(),
        m_new.data_ptr(), B, NH, DQK, DV, float(qk_scale), float(eps),
        _lib.dtype_code(q, what), _lib.dtype_code(i, what), _lib.stream_of(q))
    _lib.check(rc, what)


@torch.library.custom_op("xlstm_hip::mlstm_step", mutates_args=())
def mlstm_step_op(q: Tensor, k: Tensor, v: Tensor, i: Tensor, f: Tensor, c: Tensor, n: Tensor, m: Tensor,
                  eps: float, qk_scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    what = "mlstm_step"
    _lib.require_gpu(q, k, v, i, f, c, n, m, what=what)
    B, NH, DQK, DV = _step_shapes(q, k, v, i, f, c, n, m, what)
    q, k, v, i, f = (_prep(t) for t in (q, k, v, i, f))
    c, n, m = _f32(c), _f32(n), _f32(m)
    h = torch.empty((B, NH, DV), dtype=q.dtype, device=q.device)
    c_new = torch.empty((B, NH, DQK, DV), dtype=torch.float32, device=q.device)
    n_new = torch.empty((B, NH, DQK), dtype=torch.float32, device=q.device)
    m_new = torch.empty((B, NH, 1), dtype=torch.float32, device=q.device)
    _launch_step(q, k, v, i, f, c, n, m, h, c_new, n_new, m_new, B, NH, DQK, DV, qk_scale, eps, what)
    return h, c_new, n_new, m_new


@mlstm_step_op.register_fake
def _(q, k, v, i, f, c, n, m, eps, qk_scale):
    B, NH, DQK = q.shape
    DV = v.shape[-1]
    return (q.new_empty((B, NH, DV)), q.new_empty((B, NH, DQK, DV), dtype=torch.float32),
            q.new_empty((B, NH, DQK), dtype=torch.float32), q.new_empty((B, NH, 1), dtype=torch.float32))


@torch.library.custom_op("xlstm_hip::mlstm_step_", mutates_args=("c",))
def mlstm_step_inplace_op(q: Tensor, k: Tensor, v: Tensor, i: Tensor, f: Tensor, c: Tensor, n: Tensor, m: Tensor,
                          eps: float, qk_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    """Decode step updating the float32 C state in place; returns (h, n', m')."""
    what = "mlstm_step_"
    _lib.require_gpu(q, k, v, i, f, c, n, m, what=what)
    B, NH, DQK, DV = _step_shapes(q, k, v, i, f, c, n, m, what)
    _check(c.dtype == torch.float32 and c.is_contiguous() and c.data_ptr() % 16 == 0, what,
           "in-place C must be a contiguous, 16-byte aligned float32 tensor")
    q, k, v, i, f = (_prep(t) for t in (q, k, v, i, f))
    n, m = _f32(n), _f32(m)
    h = torch.empty((B, NH, DV), dtype=q.dtype, device=q.device)
    n_new = torch.empty((B, NH, DQK), dtype=torch.float32, device=q.device)
    m_new = torch.empty((B, NH, 1), dtype=torch.float32, device=q.device)
    _launch_step(q, k, v, i, f, c, n, m, h, c, n_new, m_new, B, NH, DQK, DV, qk_scale, eps, what)
    return h, n_new, m_new


@mlstm_step_inplace_op.register_fake
def _(q, k, v, i, f, c, n, m, eps, qk_scale):
    B, NH, DQK = q.shape
    DV = v.shape[-1]
    return (q.new_empty((B, NH, DV)), q.new_empty((B, NH, DQK), dtype=torch.float32),
            q.new_empty((B, NH, 1), dtype=torch.float32))


# -------------------------------------------------------- chunkwise / sequence
def _seq_shapes(q, k, v, i, f, c0, n0, m0, what):
    _check(q.dim() == 4, what, f"q must be (B, NH, S, DHQK), got {tuple(q.shape)}")
    B, NH, S, DQK = q.shape
    _check(k.shape == q.shape, what, "q and k must have the same shape")
    _check(v.dim() == 4 and v.shape[:3] == (B, NH, S), what, f"v must be (B, NH, S, DHV), got {tuple(v.shape)}")
    DV = v.shape[-1]
    _check(q.dtype == k.dtype == v.dtype, what, "q, k, v must share a dtype")
    _check(i.shape == (B, NH, S) and f.shape == (B, NH, S), what, "i and f must be (B, NH, S)")
    _check(i.dtype == f.dtype, what, "i and f must share a dtype")
    given = [t is not None for t in (c0, n0, m0)]
    _check(all(given) or not any(given), what, "Initial states must be provided together.")
    if c0 is not None:
        _check(c0.shape == (B, NH, DQK, DV), what, f"c_initial has wrong shape, got {tuple(c0.shape)}")
        _check(n0.shape == (B, NH, DQK), what, f"n_initial has wrong shape, got {tuple(n0.shape)}")
        _check(m0.numel() == B * NH, what, f"m_initial has wrong shape, got {tuple(m0.shape)}")
    return B, NH, S, DQK, DV


_ALGO_NAMES = {1: "two_pass", 2: "fused", 3: "pipelined"}
_fallback_warned: set = set()


def chunkwise_algorithm(B, NH, S, DQK, DV, L, dtype, algo="auto") -> str:
    """The algorithm ("fused", "pipelined" or "two_pass") xl_mlstm_chunkwise_fwd takes for these arguments."""
    lib = _lib.load()
    rc = int(lib.xl_mlstm_chunkwise_algo(B, NH, S, DQK, DV, L, _lib.XL_DTYPE[dtype], _lib.ALGO[algo]))
    if rc < 0:
        _lib.check(rc, "mlstm_chunkwise")
    return _ALGO_NAMES[rc]


def _warn_slow_fallback(B, NH, S, DQK, DV, L, dtype) -> None:
    """One warning per reason when algo="auto" leaves 16-bit inputs on the two-pass kernels (several
    times slower than the single-pass kernels, and holding every chunk's state in a workspace)."""
    lib = _lib.load()
    if int(lib.xl_mlstm_chunkwise_algo(B, NH, S, DQK, DV, L, _lib.XL_DTYPE[dtype], 0)) != 1:
        return
    why = lib.xl_last_error().decode(errors="replace")
    if why not in _fallback_warned:
        _fallback_warned.add(why)
        warnings.warn(f"xlstm_hip.mlstm_chunkwise: {dtype} inputs run the two-pass kernels ({why}); "
                      "bf16 or f16 q/k/v with DQK 32, 64, 96, 128, 192 or 256 and DV a multiple of 64 take "
                      "the single-pass kernels",
                      RuntimeWarning, stacklevel=3)


def chunkwise_workspace_bytes(B, NH, S, DQK, DV, L, dtype, algo="auto") -> int:
    return int(_lib.load().xl_mlstm_chunkwise_workspace_size(B, NH, S, DQK, DV, L, _lib.XL_DTYPE[dtype],
                                                             _lib.ALGO[algo]))


def _state_outs(ret, B, NH, DQK, DV, dev):
    if not ret:  # three distinct empties: custom-op outputs may not alias each other
        return tuple(torch.empty(_EMPTY_SHAPE, dtype=torch.float32, device=dev) for _ in range(3))
    return (torch.empty((B, NH, DQK, DV), dtype=torch.float32, device=dev),
            torch.empty((B, NH, DQK), dtype=torch.float32, device=dev),
            torch.empty((B, NH, 1), dtype=torch.float32, device=dev))


@torch.library.custom_op("xlstm_hip::mlstm_chunkwise", mutates_args=())
def mlstm_chunkwise_op(q: Tensor, k: Tensor, v: Tensor, i: Tensor, f: Tensor, c0: Optional[Tensor],
                       n0: Optional[Tensor], m0: Optional[Tensor], qk_scale: float, chunk_size: int, eps: float,
                       return_last_states: bool, algo: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    what = "mlstm_chunkwise"
    _lib.require_gpu(q, k, v, i, f, c0, n0, m0, what=what)
    B, NH, S, DQK, DV = _seq_shapes(q, k, v, i, f, c0, n0, m0, what)
    if S % chunk_size != 0 and algo not in (_lib.ALGO["fused"], _lib.ALGO["pipelined"]):  # single pass: ragged last chunk OK
        raise AssertionError(f"Sequence length {S} is not divisible by chunk size {chunk_size}.")
    q, k, v, i, f = (_prep(t) for t in (q, k, v, i, f))
    c0, n0, m0 = _f32(c0), _f32(n0), _f32(m0)
    h = torch.empty((B, NH, S, DV), dtype=q.dtype, device=q.device)
    cl, nl, ml = _state_outs(return_last_states, B, NH, DQK, DV, q.device)
    lib = _lib.load()
    dq = _lib.dtype_code(q, what)
    if algo == _lib.ALGO["auto"] and q.dtype != torch.float32:
        _warn_slow_fallback(B, NH, S, DQK, DV, chunk_size, q.dtype)
    ws_bytes = int(lib.xl_mlstm_chunkwise_workspace_size(B, NH, S, DQK, DV, chunk_size, dq, int(algo)))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=q.device) if ws_bytes else None
    rc = lib.xl_mlstm_chunkwise_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(),
        _lib.ptr(c0), _lib.ptr(n0), _lib.ptr(m0), h.data_ptr(),
        cl.data_ptr() if return_last_states else None, nl.data_ptr() if return_last_states else None,
        ml.data_ptr() if return_last_states else None,
        B, NH, S, DQK, DV, int(chunk_size), float(qk_scale), float(eps), dq, _lib.dtype_code(i, what), int(algo),
        _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    _lib.check(rc, what)
    return h, cl, nl, ml


@mlstm_chunkwise_op.register_fake
def _(q, k, v, i, f, c0, n0, m0, qk_scale, chunk_size, eps, return_last_states, algo):
    B, NH, S, DQK = q.shape
    DV = v.shape[-1]
    h = q.new_empty((B, NH, S, DV))
    if not return_last_states:
        return (h,) + tuple(q.new_empty(_EMPTY_SHAPE, dtype=torch.float32) for _ in range(3))
    return (h, q.new_empty((B, NH, DQK, DV), dtype=torch.float32), q.new_empty((B, NH, DQK), dtype=torch.float32),
            q.new_empty((B, NH, 1), dtype=torch.float32))


# ----------------------------------------------------------- chunkwise backward
@torch.library.custom_op("xlstm_hip::mlstm_chunkwise_bwd", mutates_args=())
def mlstm_chunkwise_bwd_op(q: Tensor, k: Tensor, v: Tensor, i: Tensor, f: Tensor, c0: Optional[Tensor],
                           n0: Optional[Tensor], m0: Optional[Tensor], dh: Tensor, dc_last: Optional[Tensor],
                           qk_scale: float, chunk_size: int, eps: float
                           ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The reference's custom backward (mlstm_chunkwise_bw, bw.py:198-352): dq, dk, dv (q's dtype),
    di, df (the gates' dtype) and dc0 (float32; an empty placeholder without initial states)."""
    what = "mlstm_chunkwise_bwd"
    _lib.require_gpu(q, k, v, i, f, c0, n0, m0, dh, dc_last, what=what)
    B, NH, S, DQK, DV = _seq_shapes(q, k, v, i, f, c0, n0, m0, what)
    _check(tuple(dh.shape) == (B, NH, S, DV), what, f"dh must be (B, NH, S, DHV), got {tuple(dh.shape)}")
    _check(dc_last is None or tuple(dc_last.shape) == (B, NH, DQK, DV), what, "dC_last must be (B, NH, DHQK, DHV)")
    if S % chunk_size != 0:
        raise AssertionError(f"Sequence length {S} is not divisible by chunk size {chunk_size}.")
    q, k, v, i, f = (_prep(t) for t in (q, k, v, i, f))
    dh = _prep(dh.to(q.dtype))
    c0, n0, m0, dcl = _f32(c0), _f32(n0), _f32(m0), _f32(dc_last)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    di, df = torch.empty_like(i), torch.empty_like(f)
    dc0 = (torch.empty((B, NH, DQK, DV), dtype=torch.float32, device=q.device) if c0 is not None
           else torch.empty(_EMPTY_SHAPE, dtype=torch.float32, device=q.device))
    lib = _lib.load()
    ws_bytes = int(lib.xl_mlstm_chunkwise_bwd_workspace_size(B, NH, S, DQK, DV, int(chunk_size)))
    _check(ws_bytes > 0, what, f"unsupported shape or chunk_size {chunk_size} (16, 32 or 64)")
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=q.device)
    rc = lib.xl_mlstm_chunkwise_bwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(),
        _lib.ptr(c0), _lib.ptr(n0), _lib.ptr(m0), dh.data_ptr(), _lib.ptr(dcl),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), di.data_ptr(), df.data_ptr(),
        dc0.data_ptr() if c0 is not None else None,
        B, NH, S, DQK, DV, int(chunk_size), float(qk_scale), float(eps), _lib.dtype_code(q, what),
        _lib.dtype_code(i, what), ws.data_ptr(), ws_bytes, _lib.stream_of(q))
    _lib.check(rc, what)
    return dq, dk, dv, di, df, dc0


@mlstm_chunkwise_bwd_op.register_fake
def _(q, k, v, i, f, c0, n0, m0, dh, dc_last, qk_scale, chunk_size, eps):
    dc0 = (q.new_empty(tuple(c0.shape), dtype=torch.float32) if c0 is not None
           else q.new_empty(_EMPTY_SHAPE, dtype=torch.float32))
    return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape), i.new_empty(i.shape), \
        f.new_empty(f.shape), dc0


def _chunkwise_setup_context(ctx, inputs, output):
    q, k, v, i, f, c0, n0, m0, qk_scale, chunk_size, eps, return_last_states, algo = inputs
    ctx.save_for_backward(q, k, v, i, f, c0, n0, m0)
    ctx.params = (qk_scale, chunk_size, eps, return_last_states)


# Tokens appended to a ragged sequence for its backward: an input gate this negative makes
# exp(i - m) = 0 and leaves every stabiliser alone, and logsigmoid(30) = -9.4e-14 makes the
# forget factor 1 to float32 precision, so (C, n, m) pass through them unchanged and so does the
# gradient of the last state; their h gradient is zero and their own gradients are dropped.
_PAD_I, _PAD_F = -3.0e4, 30.0


def _chunkwise_backward(ctx, dh, dC, dn, dm):
    """Gradients of (h, C_last) through the reference's custom backward; those of n_last and m_last
    are dropped and the initial n and m get zeros, as there (bw.py:340-342).

    The backward kernels take chunk sizes 16, 32 and 64.  The custom backward's gradients do not
    depend on the chunk size (tests/test_oracle_chunkwise_bw.py::test_chunk_size_invariant), so
    chunk_size 128 (S % 128 == 0, hence S % 64 == 0) runs at 64, and so does a sequence the
    single-pass forward took with a ragged last chunk (S % chunk_size != 0), padded to whole
    64-token chunks with state-preserving tokens (_PAD_I, _PAD_F) whose gradients are dropped."""
    q, k, v, i, f, c0, n0, m0 = ctx.saved_tensors
    qk_scale, chunk_size, eps, return_last_states = ctx.params
    S = q.shape[2]
    if dh is None:
        dh = torch.zeros(q.shape[:3] + (v.shape[-1],), dtype=q.dtype, device=q.device)
    dcl = dC if (return_last_states and dC is not None) else None
    L = int(chunk_size)
    if L not in (16, 32, 64) or S % L != 0:
        L = 64
    pad = (-S) % L
    if pad:
        q, k, v, dh = (torch.nn.functional.pad(t, (0, 0, 0, pad)) for t in (q, k, v, dh))
        i = torch.nn.functional.pad(i, (0, pad), value=_PAD_I)
        f = torch.nn.functional.pad(f, (0, pad), value=_PAD_F)
    dq, dk, dv, di, df, dc0 = mlstm_chunkwise_bwd_op(q, k, v, i, f, c0, n0, m0, dh, dcl, qk_scale, L, eps)
    if pad:
        dq, dk, dv = (t[:, :, :S].contiguous() for t in (dq, dk, dv))
        di, df = (t[:, :, :S].contiguous() for t in (di, df))
    g_c0 = dc0.to(c0.dtype) if c0 is not None else None
    g_n0 = torch.zeros_like(n0) if n0 is not None else None
    g_m0 = torch.zeros_like(m0) if m0 is not None else None
    return dq, dk, dv, di, df, g_c0, g_n0, g_m0, None, None, None, None, None


torch.library.register_autograd("xlstm_hip::mlstm_chunkwise", _chunkwise_backward,
                                setup_context=_chunkwise_setup_context)


@torch.library.custom_op("xlstm_hip::mlstm_sequence", mutates_args=())
def mlstm_sequence_op(q: Tensor, k: Tensor, v: Tensor, i: Tensor, f: Tensor, c0: Optional[Tensor],
                      n0: Optional[Tensor], m0: Optional[Tensor], qk_scale: float, eps: float,
                      return_last_states: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    what = "mlstm_sequence"
    _lib.require_gpu(q, k, v, i, f, c0, n0, m0, what=what)
    B, NH, S, DQK, DV = _seq_shapes(q, k, v, i, f, c0, n0, m0, what)
    q, k, v, i, f = (_prep(t) for t in (q, k, v, i, f))
    c0, n0, m0 = _f32(c0), _f32(n0), _f32(m0)
    h = torch.empty((B, NH, S, DV), dtype=q.dtype, device=q.device)
    cl, nl, ml = _state_outs(return_last_states, B, NH, DQK, DV, q.device)
    rc = _lib.load().xl_mlstm_sequence_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(),
        _lib.ptr(c0), _lib.ptr(n0), _lib.ptr(m0), h.data_ptr(),
        cl.data_ptr() if return_last_states else None, nl.data_ptr() if return_last_states else None,
        ml.data_ptr() if return_last_states else None,
        B, NH, S, DQK, DV, float(qk_scale), float(eps), _lib.dtype_code(q, what), _lib.dtype_code(i, what),
        _lib.stream_of(q))
    _lib.check(rc, what)
    return h, cl, nl, ml


@mlstm_sequence_op.register_fake
def _(q, k, v, i, f, c0, n0, m0, qk_scale, eps, return_last_states):
    B, NH, S, DQK = q.shape
    DV = v.shape[-1]
    h = q.new_empty((B, NH, S, DV))
    if not return_last_states:
        return (h,) + tuple(q.new_empty(_EMPTY_SHAPE, dtype=torch.float32) for _ in range(3))
    return (h, q.new_empty((B, NH, DQK, DV), dtype=torch.float32), q.new_empty((B, NH, DQK), dtype=torch.float32),
            q.new_empty((B, NH, 1), dtype=torch.float32))


# ------------------------------------------------------------------- sLSTM
def _slstm_out_dtype(z, i, c):
    return torch.promote_types(torch.promote_types(z.dtype, i.dtype), c.dtype)


@torch.library.custom_op("xlstm_hip::slstm_step", mutates_args=())
def slstm_step_op(z: Tensor, i: Tensor, f: Tensor, o: Tensor, c: Tensor, n: Tensor, m: Tensor,
                  eps: float) -> tuple[Tensor, Tensor]:
    """Returns h and the new states packed as one flat tensor [c | n | m] (``state_views``
    splits it): one allocation and, for 16-bit outputs, one conversion kernel."""
    what = "slstm_step"
    _lib.require_gpu(z, i, f, o, c, n, m, what=what)
    _check(z.dim() == 3, what, f"z must be (B, NH, H), got {tuple(z.shape)}")
    B, NH, H = z.shape
    for name, t in (("i_preact", i), ("f_preact", f), ("o_preact", o), ("m_state", m)):
        _check(t.shape == (B, NH), what, f"{name} must be (B, NH), got {tuple(t.shape)}")
    _check(c.shape == (B, NH, H) and n.shape == (B, NH, H), what, "c_state and n_state must be (B, NH, H)")
    _check(i.dtype == f.dtype == o.dtype, what, "gates must share a dtype")
    out_dt = _slstm_out_dtype(z, i, c)
    z, i, f, o = (_prep(t) for t in (z, i, f, o))
    c, n, m = _f32(c), _f32(n), _f32(m)
    h = torch.empty((B, NH, H), dtype=out_dt, device=z.device)
    st = torch.empty(2 * B * NH * H + B * NH, dtype=torch.float32, device=z.device)
    c_new, n_new, m_new = state_views(st, B, NH, H)
    rc = _lib.load().xl_slstm_step_fwd(
        z.data_ptr(), i.data_ptr(), f.data_ptr(), o.data_ptr(), c.data_ptr(), n.data_ptr(), m.data_ptr(),
        h.data_ptr(), c_new.data_ptr(), n_new.data_ptr(), m_new.data_ptr(), B, NH, H, float(eps),
        _lib.dtype_code(z, what), _lib.dtype_code(i, what), _lib.dtype_code(h, what), _lib.stream_of(z))
    _lib.check(rc, what)
    return h, (st.to(out_dt) if out_dt != torch.float32 else st)


@slstm_step_op.register_fake
def _(z, i, f, o, c, n, m, eps):
    out_dt = _slstm_out_dtype(z, i, c)
    B, NH, H = z.shape
    return z.new_empty((B, NH, H), dtype=out_dt), z.new_empty((2 * B * NH * H + B * NH,), dtype=out_dt)


def state_views(st: Tensor, B: int, NH: int, H: int) -> tuple[Tensor, Tensor, Tensor]:
    """c [B,NH,H], n [B,NH,H], m [B,NH]: the consecutive pieces of a flat sLSTM state tensor."""
    k = B * NH * H
    return st[:k].view(B, NH, H), st[k:2 * k].view(B, NH, H), st[2 * k:].view(B, NH)


@torch.library.custom_op("xlstm_hip::slstm_sequence", mutates_args=())
def slstm_sequence_op(z: Tensor, i: Tensor, f: Tensor, o: Tensor, c0: Optional[Tensor], n0: Optional[Tensor],
                      m0: Optional[Tensor], eps: float) -> tuple[Tensor, Tensor]:
    """Returns h and the last states packed as one flat tensor [c | n | m] (``state_views``)."""
    what = "slstm_sequence"
    _lib.require_gpu(z, i, f, o, c0, n0, m0, what=what)
    _check(z.dim() == 4, what, f"z must be (B, S, NH, H), got {tuple(z.shape)}")
    B, S, NH, H = z.shape
    for name, t in (("i_preact", i), ("f_preact", f), ("o_preact", o)):
        _check(t.shape == (B, S, NH), what, f"{name} must be (B, S, NH), got {tuple(t.shape)}")
    _check(i.dtype == f.dtype == o.dtype, what, "gates must share a dtype")
    given = [t is not None for t in (c0, n0, m0)]
    _check(all(given) or not any(given), what, "initial states must be provided together")
    if c0 is not None:
        _check(c0.shape == (B, NH, H) and n0.shape == (B, NH, H) and m0.shape == (B, NH), what,
               "state must be c, n (B, NH, H) and m (B, NH)")
    out_dt = torch.promote_types(z.dtype, i.dtype) if c0 is None else _slstm_out_dtype(z, i, c0)
    z, i, f, o = (_prep(t) for t in (z, i, f, o))
    c0, n0, m0 = _f32(c0), _f32(n0), _f32(m0)
    h = torch.empty((B, S, NH, H), dtype=out_dt, device=z.device)
    st = torch.empty(2 * B * NH * H + B * NH, dtype=torch.float32, device=z.device)
    cl, nl, ml = state_views(st, B, NH, H)
    rc = _lib.load().xl_slstm_seq_fwd(
        z.data_ptr(), i.data_ptr(), f.data_ptr(), o.data_ptr(), _lib.ptr(c0), _lib.ptr(n0), _lib.ptr(m0),
        h.data_ptr(), cl.data_ptr(), nl.data_ptr(), ml.data_ptr(), B, S, NH, H, float(eps),
        _lib.dtype_code(z, what), _lib.dtype_code(i, what), _lib.dtype_code(h, what), _lib.stream_of(z))
    _lib.check(rc, what)
    return h, (st.to(out_dt) if out_dt != torch.float32 else st)


@slstm_sequence_op.register_fake
def _(z, i, f, o, c0, n0, m0, eps):
    B, S, NH, H = z.shape
    out_dt = torch.promote_types(z.dtype, i.dtype) if c0 is None else _slstm_out_dtype(z, i, c0)
    return z.new_empty((B, S, NH, H), dtype=out_dt), z.new_empty((2 * B * NH * H + B * NH,), dtype=out_dt)


# ------------------------------------------- sLSTM layer: causal conv1d + SiLU, GroupNorm
CONV_ACTS = {None: 0, "silu": 1}


@torch.library.custom_op("xlstm_hip::causal_conv1d", mutates_args=())
def causal_conv1d_op(x: Tensor, weight: Tensor, bias: Optional[Tensor], act: int) -> Tensor:
    what = "causal_conv1d"
    _lib.require_gpu(x, weight, bias, what=what)
    _check(x.dim() == 3, what, f"x must be (B, S, D) channels last, got {tuple(x.shape)}")
    B, S, D = x.shape
    _check(weight.dim() in (2, 3) and weight.shape[0] == D and (weight.dim() == 2 or weight.shape[1] == 1), what,
           f"weight must be (D, K) or (D, 1, K) with D = {D}, got {tuple(weight.shape)}")
    _check(bias is None or tuple(bias.shape) == (D,), what, f"bias must be ({D},)")
    _check(weight.dtype == x.dtype and (bias is None or bias.dtype == x.dtype), what,
           "x, weight and bias must share a dtype (as nn.Conv1d requires)")
    _check(act in (0, 1), what, f"act must be 0 (none) or 1 (SiLU), got {act}")
    K = weight.shape[-1]
    x, w = _prep(x), _prep(weight)
    b = None if bias is None else _prep(bias)
    y = torch.empty_like(x)
    rc = _lib.load().xl_causal_conv1d_fwd(x.data_ptr(), w.data_ptr(), _lib.ptr(b), y.data_ptr(), B, S, D, K,
                                          int(act), _lib.dtype_code(x, what), _lib.stream_of(x))
    _lib.check(rc, what)
    return y


@causal_conv1d_op.register_fake
def _(x, weight, bias, act):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("xlstm_hip::group_norm", mutates_args=())
def group_norm_op(x: Tensor, num_groups: int, weight: Optional[Tensor], bias: Optional[Tensor],
                  eps: float) -> Tensor:
    what = "group_norm"
    _lib.require_gpu(x, weight, bias, what=what)
    _check(x.dim() == 2, what, f"x must be (N, C), got {tuple(x.shape)}")
    N, C = x.shape
    _check(num_groups >= 1 and C % num_groups == 0, what, f"C = {C} is not a multiple of num_groups = {num_groups}")
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None:
            _check(tuple(t.shape) == (C,), what, f"{name} must be ({C},)")
            _check(t.dtype == x.dtype, what, f"{name} must have x's dtype {x.dtype}")
    x = _prep(x)
    w = None if weight is None else _prep(weight)
    b = None if bias is None else _prep(bias)
    y = torch.empty_like(x)
    rc = _lib.load().xl_group_norm_fwd(x.data_ptr(), _lib.ptr(w), _lib.ptr(b), y.data_ptr(), N, int(num_groups),
                                       C // num_groups, float(eps), _lib.dtype_code(x, what), _lib.stream_of(x))
    _lib.check(rc, what)
    return y


@group_norm_op.register_fake
def _(x, num_groups, weight, bias, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


# ------------------------------------------- mLSTM output cell: multi-head RMSNorm x sigmoid(o)
@torch.library.custom_op("xlstm_hip::mh_rmsnorm_gate", mutates_args=())
def mh_rmsnorm_gate_op(h: Tensor, weight: Optional[Tensor], o_preact: Optional[Tensor], heads_first: bool,
                       eps: float) -> Tensor:
    what = "mh_rmsnorm_gate"
    _lib.require_gpu(h, weight, o_preact, what=what)
    _check(h.dim() == 4, what, f"h must be 4-D, got {tuple(h.shape)}")
    if heads_first:
        B, NH, S, DH = h.shape
    else:
        B, S, NH, DH = h.shape
    _check(weight is None or tuple(weight.shape) == (NH * DH,), what, f"weight must be ({NH * DH},)")
    _check(o_preact is None or tuple(o_preact.shape) in ((B, S, NH * DH), (B, S, NH, DH)), what,
           f"o_preact must be (B, S, NH*DH) = {(B, S, NH * DH)}")
    for name, t in (("weight", weight), ("o_preact", o_preact)):
        _check(t is None or t.dtype == h.dtype, what, f"{name} must have h's dtype {h.dtype}")
    h = _prep(h)
    w = None if weight is None else _prep(weight)
    o = None if o_preact is None else _prep(o_preact)
    y = torch.empty((B, S, NH * DH), dtype=h.dtype, device=h.device)
    rc = _lib.load().xl_mh_rmsnorm_gate_fwd(h.data_ptr(), _lib.ptr(w), _lib.ptr(o), y.data_ptr(), B, NH, S, DH,
                                            1 if heads_first else 0, float(eps), _lib.dtype_code(h, what),
                                            _lib.stream_of(h))
    _lib.check(rc, what)
    return y


@mh_rmsnorm_gate_op.register_fake
def _(h, weight, o_preact, heads_first, eps):
    if heads_first:
        B, NH, S, DH = h.shape
    else:
        B, S, NH, DH = h.shape
    return h.new_empty((B, S, NH * DH))


# ------------------------------------------- projection cells: gate projection + soft-cap epilogue
@torch.library.custom_op("xlstm_hip::gate_proj_softcap", mutates_args=())
def gate_proj_softcap_op(x: Tensor, weight: Tensor, bias: Optional[Tensor], cap: float,
                         cap_rounding: int = 0) -> Tensor:
    what = "gate_proj_softcap"
    _lib.require_gpu(x, weight, bias, what=what)
    _check(x.dim() >= 1 and weight.dim() == 2 and weight.shape[1] == x.shape[-1], what,
           f"weight must be (G, D) with D = x.shape[-1], got {tuple(weight.shape)} for x {tuple(x.shape)}")
    G, D = weight.shape
    _check(bias is None or tuple(bias.shape) == (G,), what, f"bias must be ({G},)")
    _check(weight.dtype == x.dtype and (bias is None or bias.dtype == x.dtype), what,
           "x, weight and bias must share a dtype")
    lead = tuple(x.shape[:-1])
    M = 1
    for d in lead:
        M *= d
    x2, w = _prep(x.reshape(M, D)), _prep(weight)
    b = None if bias is None else _prep(bias)
    y = torch.empty(lead + (G,), dtype=x.dtype, device=x.device)
    rc = _lib.load().xl_gate_proj_softcap_fwd(x2.data_ptr(), w.data_ptr(), _lib.ptr(b), y.data_ptr(), M, D, G,
                                              float(cap), int(cap_rounding), _lib.dtype_code(x, what),
                                              _lib.stream_of(x))
    _lib.check(rc, what)
    return y


@gate_proj_softcap_op.register_fake
def _(x, weight, bias, cap, cap_rounding=0):
    return x.new_empty(tuple(x.shape[:-1]) + (weight.shape[0],))


# ------------------------------------------- logit projection + soft-cap epilogue
LM_HEAD_MAX_ROWS = 16
LM_HEAD_MAX_LDS = 160 * 1024  # the kernel stages rows * (D + 8) 16-bit values in LDS


@torch.library.custom_op("xlstm_hip::lm_head_softcap", mutates_args=())
def lm_head_softcap_op(x: Tensor, weight: Tensor, cap: float) -> Tensor:
    what = "lm_head_softcap"
    _lib.require_gpu(x, weight, what=what)
    _check(x.dim() >= 1 and weight.dim() == 2 and weight.shape[1] == x.shape[-1], what,
           f"weight must be (V, D) with D = x.shape[-1], got {tuple(weight.shape)} for x {tuple(x.shape)}")
    _check(weight.dtype == x.dtype, what, "x and weight must share a dtype")
    V, D = weight.shape
    lead = tuple(x.shape[:-1])
    M = 1
    for d in lead:
        M *= d
    _check(M <= LM_HEAD_MAX_ROWS, what, f"{M} rows (at most {LM_HEAD_MAX_ROWS}; logits of every position are a "
                                        "GEMM: use the Linear and soft_cap)")
    _check(M * (D + 8) * 2 <= LM_HEAD_MAX_LDS, what, f"{M} rows of D={D} exceed the kernel's LDS staging")
    x2, w = _prep(x.reshape(M, D)), _prep(weight)
    y = torch.empty(lead + (V,), dtype=x.dtype, device=x.device)
    rc = _lib.load().xl_lm_head_softcap_fwd(x2.data_ptr(), w.data_ptr(), y.data_ptr(), M, D, V, float(cap),
                                            _lib.dtype_code(x, what), _lib.stream_of(x))
    _lib.check(rc, what)
    return y


@lm_head_softcap_op.register_fake
def _(x, weight, cap):
    return x.new_empty(tuple(x.shape[:-1]) + (weight.shape[0],))
