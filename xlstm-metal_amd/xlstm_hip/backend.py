"""Kernel registry, arbitrary-length wrappers and the backend module, on HIP.

Mirrors kernel_development/xlstm/mlstm_block/mslstm_parallel/torch/:
``mLSTMBackendConfig`` / ``mLSTMBackend`` (backend_module.py:42-219),
``wrap_chunkwise__arbitrary_sequence_length`` / ``wrap_chunkwise__pad_zeros``
(kernel_wrappers.py:12-284), and the lookup functions ``get_mlstm_kernel``,
``get_mlstm_step_kernel``, ``get_mlstm_sequence_kernel`` that backend_module.py
imports (:11-15) but that are missing from the reference package.  Names of
kernels this build does not provide (the Triton and quadratic-parallel ones)
raise ``NotImplementedError``.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import partial
from typing import Callable, Literal

import torch
from torch import nn

from .chunkwise import mlstm_chunkwise__native_autograd, mlstm_chunkwise__native_custbw
from .ops import chunkwise_workspace_bytes
from .recurrent import mlstm_recurrent_sequence__native_fw, mlstm_recurrent_step__native

__all__ = [
    "get_mlstm_kernel", "get_mlstm_step_kernel", "get_mlstm_sequence_kernel", "available_kernels",
    "wrap_chunkwise__arbitrary_sequence_length", "wrap_chunkwise__pad_zeros",
    "mLSTMBackendConfig", "mLSTMBackend",
]

ChunkwiseKernelType = Literal[
    "chunkwise--native_autograd", "chunkwise--native_custbw", "chunkwise--triton_limit_chunk",
    "chunkwise--triton_xl_chunk", "parallel--native_autograd", "parallel--native_custbw",
    "parallel--native_stablef_autograd", "parallel--native_stablef_custbw", "parallel--triton_limit_headdim",
]
SequenceKernelType = Literal["native_sequence__native", "native_sequence__triton"]
StepKernelType = Literal["native", "triton"]
DtypeType = Literal["float32", "bfloat16", "float16"]
BackendModeType = Literal["train", "train_with_padding", "inference"]

_CHUNKWISE = {
    # both torch-native names run the same HIP forward and, under autograd, the reference's custom
    # backward (bw.py:198-352; equal to autograd's gradient behind the layer's multi-head norm)
    "chunkwise--native_autograd": mlstm_chunkwise__native_autograd,
    "chunkwise--native_custbw": mlstm_chunkwise__native_custbw,
}
_SEQUENCE = {"native_sequence__native": mlstm_recurrent_sequence__native_fw}
_STEP = {"native": mlstm_recurrent_step__native}


def _get(table: dict, name: str, kind: str) -> Callable:
    try:
        return table[name]
    except KeyError:
        raise NotImplementedError(
            f"xlstm_hip: {kind} kernel '{name}' is not provided (available: {sorted(table)})") from None


def get_mlstm_kernel(name: str) -> Callable:
    return _get(_CHUNKWISE, name, "chunkwise")


def get_mlstm_step_kernel(name: str) -> Callable:
    return _get(_STEP, name, "step")


def get_mlstm_sequence_kernel(name: str) -> Callable:
    return _get(_SEQUENCE, name, "sequence")


def available_kernels() -> dict:
    return {"chunkwise": sorted(_CHUNKWISE), "sequence": sorted(_SEQUENCE), "step": sorted(_STEP)}


def _fused_takes_any_length(q, k, v) -> bool:
    """True when this library's pipelined single-pass chunkwise kernel runs the whole sequence in
    one call (bf16 or f16 q/k/v and a head shape it supports; it runs 64-token chunks with a
    ragged last chunk)."""
    if not (q.dtype == k.dtype == v.dtype and q.dtype in (torch.bfloat16, torch.float16)):
        return False
    B, NH, S, DQK = q.shape
    return chunkwise_workspace_bytes(B, NH, S, DQK, v.shape[-1], 64, q.dtype, algo="pipelined") > 0


def wrap_chunkwise__arbitrary_sequence_length(mlstm_chunkwise_kernel, mlstm_sequence_kernel, mlstm_step_kernel, q,
                                              k, v, f, i, c_initial=None, n_initial=None, m_initial=None,
                                              return_last_states=True, eps=1e-6,
                                              autocast_kernel_dtype=torch.bfloat16, chunk_size=64,
                                              enable_logging=False):
    """Any-S inference (kernel_wrappers.py:12-202): chunk sizes chunk_size, /2, ... >= 16
    on the largest whole number of chunks each, carrying (C, n, m); the sequence kernel
    for a tail < 16; the step kernel when S == 1.  Zero states are float32 (:84-98).
    With this library's chunkwise kernel and inputs its fused kernel takes, the whole
    sequence is one fused call instead: the forward is chunk-size invariant, so the split
    above changes rounding only, and the slicing copies and the concatenation go away."""
    B, NH, S, DHQK = k.shape
    DHHV = v.shape[-1]
    sizes = []
    cs = chunk_size
    while cs >= 16:
        sizes.append(cs)
        cs //= 2
    dev = k.device
    c_state = c_initial if c_initial is not None else torch.zeros(B, NH, DHQK, DHHV, device=dev, dtype=torch.float32)
    n_state = n_initial if n_initial is not None else torch.zeros(B, NH, DHQK, device=dev, dtype=torch.float32)
    m_state = m_initial if m_initial is not None else torch.zeros(B, NH, 1, device=dev, dtype=torch.float32)
    if S > 1 and mlstm_chunkwise_kernel in (mlstm_chunkwise__native_autograd, mlstm_chunkwise__native_custbw) \
            and _fused_takes_any_length(q, k, v):
        # the fused kernel runs 64-token chunks whatever chunk_size names (the forward is
        # chunk-size invariant), so it is called with the size its support was checked for
        h_out, (c_state, n_state, m_state) = mlstm_chunkwise_kernel(
            q=q, k=k, v=v, f=f, i=i, c_initial=c_state, n_initial=n_state, m_initial=m_state, chunk_size=64,
            return_last_states=True, eps=eps, algo="pipelined")
    elif S > 1:
        h_outs = []
        start = 0
        for cs in sizes:
            rem = S - start
            if rem < cs:
                continue
            end = start + cs * (rem // cs)
            h_out, (c_state, n_state, m_state) = mlstm_chunkwise_kernel(
                q=q[..., start:end, :].contiguous(), k=k[..., start:end, :].contiguous(),
                v=v[..., start:end, :].contiguous(), f=f[..., start:end].contiguous(),
                i=i[..., start:end].contiguous(), c_initial=c_state, n_initial=n_state, m_initial=m_state,
                chunk_size=cs, return_last_states=True, autocast_kernel_dtype=autocast_kernel_dtype, eps=eps)
            start = end
            h_outs.append(h_out)
            if rem % cs == 0:
                break
        if S - start > 0:
            h_out, (c_state, n_state, m_state) = mlstm_sequence_kernel(
                q=q[..., start:S, :].contiguous(), k=k[..., start:S, :].contiguous(),
                v=v[..., start:S, :].contiguous(), i=i[..., start:S].contiguous(), f=f[..., start:S].contiguous(),
                c_initial=c_state, n_initial=n_state, m_initial=m_state, return_last_states=True, eps=eps)
            h_outs.append(h_out)
        h_out = torch.cat(h_outs, dim=2)
    else:
        assert S == 1, f"Received empty sequence (S={S}), require at least single element in the sequence."
        h_out, (c_state, n_state, m_state) = mlstm_step_kernel(
            q=q.squeeze(2), k=k.squeeze(2), v=v.squeeze(2), i=i, f=f, c=c_state, n=n_state, m=m_state, eps=eps)
        h_out = h_out[:, :, None, :]
    if return_last_states:
        return h_out, (c_state, n_state, m_state)
    return h_out


def wrap_chunkwise__pad_zeros(mlstm_chunkwise_kernel, q, k, v, f, i, c_initial=None, n_initial=None,
                              m_initial=None, return_last_states=False, eps=1e-6,
                              autocast_kernel_dtype=torch.bfloat16, chunk_size=64, **kwargs):
    """Zero-pads S up to a multiple of chunk_size and crops h (kernel_wrappers.py:205-284)."""
    assert not return_last_states, (
        "We are padding zeros, so we cannot return last states,", "as they would be not the true last states.")
    B, NH, S, DHQK = q.shape
    if S % chunk_size != 0:
        Sp = ((S + chunk_size - 1) // chunk_size) * chunk_size
        pad = Sp - S
        q = torch.nn.functional.pad(q, (0, 0, 0, pad))
        k = torch.nn.functional.pad(k, (0, 0, 0, pad))
        v = torch.nn.functional.pad(v, (0, 0, 0, pad))
        i = torch.nn.functional.pad(i, (0, pad))
        f = torch.nn.functional.pad(f, (0, pad))
    h = mlstm_chunkwise_kernel(q=q, k=k, v=v, i=i, f=f, c_initial=c_initial, n_initial=n_initial,
                               m_initial=m_initial, return_last_states=return_last_states, eps=eps,
                               autocast_kernel_dtype=autocast_kernel_dtype, chunk_size=chunk_size, **kwargs)
    return h[:, :, :S, :]


@dataclass
class mLSTMBackendConfig:
    """backend_module.py:42-85."""

    chunkwise_kernel: ChunkwiseKernelType = "chunkwise--native_autograd"
    sequence_kernel: SequenceKernelType = "native_sequence__native"
    step_kernel: StepKernelType = "native"
    mode: BackendModeType = "train"
    chunk_size: int = 64
    return_last_states: bool = True
    autocast_kernel_dtype: DtypeType = "bfloat16"
    eps: float = 1e-6
    inference_state_dtype: DtypeType = "float32"

    def __post_init__(self):
        if self.return_last_states and "parallel" in self.chunkwise_kernel:
            raise ValueError("return_last_states=True is not supported with parallel kernels.")
        if self.return_last_states and self.mode == "train_with_padding":
            raise ValueError("return_last_states=True is not supported with train_with_padding mode.")


class mLSTMBackend(nn.Module):
    """backend_module.py:88-219: dispatches train / inference calls to the HIP kernels."""

    config_class = mLSTMBackendConfig

    def __init__(self, config: mLSTMBackendConfig):
        super().__init__()
        self.config = config
        self.chunkwise_kernel_fn = get_mlstm_kernel(config.chunkwise_kernel)
        self.sequence_kernel_fn = get_mlstm_sequence_kernel(config.sequence_kernel)
        self.step_kernel_fn = get_mlstm_step_kernel(config.step_kernel)
        state_dt = getattr(torch, config.inference_state_dtype)
        self._inference_fn = partial(
            wrap_chunkwise__arbitrary_sequence_length,
            mlstm_chunkwise_kernel=self.chunkwise_kernel_fn,
            mlstm_sequence_kernel=partial(self.sequence_kernel_fn, dtype_state=state_dt),
            mlstm_step_kernel=partial(self.step_kernel_fn, dtype_state=state_dt),
            chunk_size=config.chunk_size, eps=config.eps,
            autocast_kernel_dtype=getattr(torch, config.autocast_kernel_dtype), return_last_states=True)
        train_fn = partial(self.chunkwise_kernel_fn, autocast_kernel_dtype=getattr(torch, config.autocast_kernel_dtype),
                           eps=config.eps, chunk_size=config.chunk_size)
        if "with_padding" in config.mode:
            train_fn = partial(wrap_chunkwise__pad_zeros, mlstm_chunkwise_kernel=train_fn)
        self._train_fn = train_fn

    def forward(self, q, k, v, i, f, c_initial=None, n_initial=None, m_initial=None, return_last_states=None,
                mode=None):
        if mode is None:
            mode = self.config.mode
        if "train" in mode:
            if return_last_states is None:
                return_last_states = self.config.return_last_states
            if self.config.mode == "train_with_padding":
                assert not return_last_states, "return_last_states=True is not supported with train_with_padding mode."
            return self._train_fn(q=q, k=k, v=v, i=i, f=f, c_initial=c_initial, n_initial=n_initial,
                                  m_initial=m_initial, return_last_states=return_last_states)
        if "inference" in mode:
            return self._inference_fn(q=q, k=k, v=v, i=i, f=f, c_initial=c_initial, n_initial=n_initial,
                                      m_initial=m_initial)
        raise ValueError(f"Unknown mode: {self.config.mode}")

    def extra_repr(self) -> str:
        return f"{self.config}"
