"""Random-init xLSTM stacks of BASELINE configs 3 and 4: the harness that runs the path's ops inside
a whole model, for the end-to-end tests and the tokens/s figures.

The block order is the reference's (paths relative to its root, ``TN`` = ``xlstm_metal/
torch_native``):

* mLSTM block (``TN/blocks/mlstm/mlstm_block.py:163-206``): x + mLSTM(RMSNorm(x)), then
  x + FFN(RMSNorm(x)) with the SwiGLU FFN ``down(silu(up_gate(x)) * up(x))``;
* sLSTM block (``TN/blocks/slstm/slstm_block.py:122-160``): the same with the sLSTM layer;
* the model: embedding, the blocks, a final RMSNorm, the lm_head and the logit soft-cap
  ``30 tanh(x / 30)`` (``TN/generate.py:131``); greedy decoding takes the argmax.

The mLSTM layer is mLSTMProjectionCell (q, k, v Linear layers; i, f by ``gate_proj_kernel`` with
the gate soft-cap) -> the chunkwise kernel over the prompt (the any-length wrapper) and the
recurrent step kernel per decoded token -> mLSTMOutputCell (``mh_rmsnorm_gate_kernel`` with
sigma(o), then out_proj).  The sLSTM layer is sLSTMProjectionCell (conv1d + SiLU kernel, gate
kernels, z Linear) -> the sLSTM sequence kernel over the prompt and the step kernel per token
-> sLSTMOutputCell (``group_norm_kernel``, out_proj).  The lm_head and the logit soft-cap are
one kernel of this library (``lm_head_softcap``; ``fused_lm_head = False`` runs torch's Linear and
then the soft_cap kernel instead).  Projections, FFN, norms and embedding are torch (hipBLASLt
GEMMs); every mLSTM/sLSTM kernel is this library's.

Weights are N(0, init_std) in the model dtype (there is no checkpoint); the mLSTM forget-gate
bias starts at +3 and the input-gate bias at 0, so the gates sit where a trained model keeps
them (f ~ sigma(3), decay close to 1).

Decoding keeps every state on the GPU and updates the mLSTM C state in place; one decode step
(all blocks, the lm_head, the soft-cap and the argmax) can be captured in a HIP graph
(``DecodeGraph``) so a token costs one graph launch instead of a few hundred kernel launches.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .backend import (get_mlstm_kernel, get_mlstm_sequence_kernel, get_mlstm_step_kernel,
                      wrap_chunkwise__arbitrary_sequence_length)
from .mlstm_layers import mLSTMOutputCell, mLSTMProjectionCell
from .recurrent import mlstm_recurrent_step_
from .slstm import slstm_sequence, slstm_step
from .slstm_layers import sLSTMOutputCell, sLSTMProjectionCell
from .soft_cap import lm_head_softcap, soft_cap

__all__ = ["StackConfig", "CFG3_STACK", "CFG4_STACK", "xLSTMStack", "DecodeGraph"]


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


@dataclass(frozen=True)
class StackConfig:
    name: str
    d_model: int
    num_blocks: int
    mlstm_heads: int
    qk_dim_factor: float = 0.5
    v_dim_factor: float = 1.0
    ffn_proj_factor: float = 2.667
    ffn_round: int = 64
    vocab: int = 50304
    gate_soft_cap: float = 15.0
    logit_soft_cap: float = 30.0
    slstm_every: int = 0          # every slstm_every-th block (1-based) is an sLSTM block; 0: none
    slstm_heads: int = 4
    conv_kernel: int = 4
    norm_eps: float = 1e-6
    eps: float = 1e-6
    init_std: float = 0.02
    dtype: torch.dtype = torch.bfloat16

    @property
    def qk_head_dim(self) -> int:
        return int(self.d_model * self.qk_dim_factor) // self.mlstm_heads

    @property
    def v_head_dim(self) -> int:
        return int(self.d_model * self.v_dim_factor) // self.mlstm_heads

    @property
    def ffn_dim(self) -> int:
        return _round_up(int(self.d_model * self.ffn_proj_factor), self.ffn_round)

    def is_slstm(self, block: int) -> bool:
        return self.slstm_every > 0 and (block + 1) % self.slstm_every == 0


# xLSTM-7B shapes, 32 mLSTM blocks, d 4096, 8 heads (DQK 256, DV 512), FFN 10944
CFG3_STACK = StackConfig("cfg3_xlstm7b", d_model=4096, num_blocks=32, mlstm_heads=8)
# d 2048, 24 blocks, mLSTM:sLSTM 7:1 (blocks 8, 16, 24 are sLSTM), mLSTM 8 heads
# (DQK 128, DV 256), sLSTM 4 heads of 512 with a causal conv of kernel 4
CFG4_STACK = StackConfig("cfg4_mixed", d_model=2048, num_blocks=24, mlstm_heads=8, slstm_every=8)


class _RMSNorm(nn.Module):
    """RMSNorm with the reduction in float32 (the reference's norm_reduce_force_float32 default)."""

    def __init__(self, d: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return F.rms_norm(x.float(), (x.shape[-1],), self.weight.float(), self.eps).to(x.dtype)


class _FFN(nn.Module):
    def __init__(self, d: int, hidden: int) -> None:
        super().__init__()
        self.proj_up = nn.Linear(d, hidden, bias=False)
        self.proj_up_gate = nn.Linear(d, hidden, bias=False)
        self.proj_down = nn.Linear(hidden, d, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        return self.proj_down(F.silu(self.proj_up_gate(x)) * self.proj_up(x))


@dataclass
class _MState:
    C: Tensor
    n: Tensor
    m: Tensor


@dataclass
class _SState:
    c: Tensor
    n: Tensor
    m: Tensor
    conv: Tensor  # the last conv_kernel - 1 normalised inputs [B, K - 1, d]


class _mLSTMBlock(nn.Module):
    def __init__(self, cfg: StackConfig) -> None:
        super().__init__()
        d, NH = cfg.d_model, cfg.mlstm_heads
        self.cfg = cfg
        self.norm_mlstm = _RMSNorm(d, cfg.norm_eps)
        self.proj = mLSTMProjectionCell(d, NH, cfg.qk_head_dim, cfg.v_head_dim, gate_soft_cap=cfg.gate_soft_cap)
        self.out = mLSTMOutputCell(d, NH, cfg.v_head_dim, eps=cfg.eps)
        self.norm_ffn = _RMSNorm(d, cfg.norm_eps)
        self.ffn = _FFN(d, cfg.ffn_dim)
        self._chunkwise = get_mlstm_kernel("chunkwise--native_autograd")
        self._sequence = get_mlstm_sequence_kernel("native_sequence__native")
        self._step = get_mlstm_step_kernel("native")

    def prefill(self, x: Tensor):
        xn = self.norm_mlstm(x)
        q, k, v, i, f = self.proj(xn)
        h, (C, n, m) = wrap_chunkwise__arbitrary_sequence_length(
            self._chunkwise, self._sequence, self._step, q.contiguous(), k.contiguous(), v.contiguous(),
            f.contiguous(), i.contiguous(), return_last_states=True, eps=self.cfg.eps)
        x = x + self.out.out_proj(self.out.gated(h, xn))
        return x + self.ffn(self.norm_ffn(x)), _MState(C.contiguous(), n.contiguous(), m.contiguous())

    def decode(self, x: Tensor, st: _MState) -> Tensor:
        """x [B, 1, d]; updates st in place (C in place, n and m replaced)."""
        xn = self.norm_mlstm(x)
        q, k, v, i, f = self.proj(xn)
        h, (_, n, m) = mlstm_recurrent_step_(q[:, :, 0], k[:, :, 0], v[:, :, 0], i, f, st.C, st.n, st.m,
                                             eps=self.cfg.eps)
        st.n.copy_(n)
        st.m.copy_(m)
        x = x + self.out.out_proj(self.out.gated(h[:, :, None, :], xn))
        return x + self.ffn(self.norm_ffn(x))


class _sLSTMBlock(nn.Module):
    def __init__(self, cfg: StackConfig) -> None:
        super().__init__()
        d, NH = cfg.d_model, cfg.slstm_heads
        self.cfg = cfg
        self.H = d // NH
        self.norm_slstm = _RMSNorm(d, cfg.norm_eps)
        self.proj = sLSTMProjectionCell(d, NH, self.H, conv1d_kernel_size=cfg.conv_kernel,
                                        gate_soft_cap=cfg.gate_soft_cap)
        self.out = sLSTMOutputCell(d, NH, self.H, eps=cfg.eps)
        self.norm_ffn = _RMSNorm(d, cfg.norm_eps)
        self.ffn = _FFN(d, cfg.ffn_dim)

    def prefill(self, x: Tensor):
        B, S, d = x.shape
        K = self.cfg.conv_kernel
        xn = self.norm_slstm(x)
        z, i, f, o, _ = self.proj(xn)
        h, (c, n, m) = slstm_sequence(z.contiguous(), i.contiguous(), f.contiguous(), o.contiguous(),
                                      eps=self.cfg.eps)
        x = x + self.out(h)
        conv = xn.new_zeros(B, K - 1, d)
        tail = xn[:, max(0, S - (K - 1)):]
        conv[:, K - 1 - tail.shape[1]:] = tail
        return x + self.ffn(self.norm_ffn(x)), _SState(c.contiguous(), n.contiguous(), m.contiguous(), conv)

    def decode(self, x: Tensor, st: _SState) -> Tensor:
        B = x.shape[0]
        NH, H = self.cfg.slstm_heads, self.H
        xn = self.norm_slstm(x)
        window = torch.cat([st.conv, xn], dim=1)          # [B, K, d]: the conv's receptive field
        p = self.proj
        x_conv = p.conv1d.forward_channels_last(window, activation="silu")[:, -1:]
        from .mlstm_layers import gate_proj_softcap, stacked_linears
        gif = gate_proj_softcap(x_conv, *stacked_linears(p.igate_proj, p.fgate_proj), p.gate_soft_cap,
                                cap_in_dtype=True)
        o = gate_proj_softcap(xn, p.ogate_proj.weight, p.ogate_proj.bias, p.gate_soft_cap, cap_in_dtype=True)
        z = p.z_proj(xn).view(B, NH, H)
        h, c, n, m = slstm_step(z, gif[:, 0, :NH], gif[:, 0, NH:], o[:, 0], st.c, st.n, st.m, eps=self.cfg.eps)
        st.c.copy_(c)
        st.n.copy_(n)
        st.m.copy_(m)
        st.conv.copy_(window[:, 1:])
        x = x + self.out(h.view(B, 1, NH, H))
        return x + self.ffn(self.norm_ffn(x))


class xLSTMStack(nn.Module):
    """Embedding -> blocks -> RMSNorm -> lm_head -> logit soft-cap, random init (see module doc)."""

    def __init__(self, cfg: StackConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.embedding = nn.Embedding(cfg.vocab, cfg.d_model)
        self.blocks = nn.ModuleList(
            [_sLSTMBlock(cfg) if cfg.is_slstm(b) else _mLSTMBlock(cfg) for b in range(cfg.num_blocks)])
        self.out_norm = _RMSNorm(cfg.d_model, cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab, bias=False)
        # the lm_head with the soft-cap in its epilogue (False: torch's Linear, then soft_cap)
        self.fused_lm_head = True

    @classmethod
    def random(cls, cfg: StackConfig, device, seed: int = 0) -> "xLSTMStack":
        """Allocates the model on `device` in cfg.dtype and draws its weights there: norm weights 1,
        forget-gate biases 3, other biases 0, every other weight N(0, init_std)."""
        with torch.device("meta"):
            model = cls(cfg).to(cfg.dtype)
        model = model.to_empty(device=device)
        g = torch.Generator(device=device).manual_seed(seed)
        with torch.no_grad():
            for name, p in model.named_parameters():
                owner, kind = name.split(".")[-2:]
                if "norm" in owner:
                    p.fill_(1.0 if kind == "weight" else 0.0)
                elif kind == "bias":
                    p.fill_(3.0 if owner == "fgate_proj" else 0.0)
                else:
                    p.copy_(torch.randn(p.shape, generator=g, device=device) * cfg.init_std)
        return model.eval()

    def logits(self, x: Tensor) -> Tensor:
        xn = self.out_norm(x)
        if self.fused_lm_head:
            return lm_head_softcap(xn, self.lm_head.weight, self.cfg.logit_soft_cap)
        return soft_cap(self.lm_head(xn), self.cfg.logit_soft_cap)

    @torch.no_grad()
    def prefill(self, tokens: Tensor):
        """tokens [B, S] -> (soft-capped logits of the last position [B, vocab], states)."""
        x = self.embedding(tokens)
        states: List = []
        for blk in self.blocks:
            x, st = blk.prefill(x)
            states.append(st)
        return self.logits(x[:, -1:])[:, 0], states

    @torch.no_grad()
    def decode_step(self, token: Tensor, states: List) -> Tensor:
        """token [B] -> soft-capped logits [B, vocab]; states updated in place."""
        x = self.embedding(token[:, None])
        for blk, st in zip(self.blocks, states):
            x = blk.decode(x, st)
        return self.logits(x)[:, 0]

    @torch.no_grad()
    def generate(self, tokens: Tensor, steps: int, graph: bool = True) -> Tensor:
        """Greedy decoding after the prompt: returns the `steps` new tokens [B, steps]."""
        logits, states = self.prefill(tokens)
        nxt = logits.argmax(-1)
        if graph:
            dg = DecodeGraph(self, states, nxt)
            return dg.run(steps)
        out = []
        for _ in range(steps):
            out.append(nxt)
            nxt = self.decode_step(nxt, states).argmax(-1)
        return torch.stack(out, dim=1)


class DecodeGraph:
    """One greedy decode step of `model` captured in a HIP graph over static buffers: the current
    token, every state (updated in place) and the next token.  ``run(steps)`` replays it."""

    def __init__(self, model: xLSTMStack, states: List, token: Tensor) -> None:
        self.model, self.states, self.token = model, states, token.clone()
        dev = self.token.device
        # torch's capture protocol: one warm-up step on a side stream first; it advances the
        # states, so they are saved before and restored after it
        saved = [[t.clone() for t in vars(st).values()] for st in states]
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            model.decode_step(self.token, states)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        for st, sv in zip(states, saved):
            for t, s in zip(vars(st).values(), sv):
                t.copy_(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.next_token = model.decode_step(self.token, states).argmax(-1)

    def step(self) -> Tensor:
        """Decodes one token: returns the token fed in and advances to the next."""
        cur = self.token.clone()
        self.graph.replay()
        self.token.copy_(self.next_token)
        return cur

    def run(self, steps: int) -> Tensor:
        return torch.stack([self.step() for _ in range(steps)], dim=1)
