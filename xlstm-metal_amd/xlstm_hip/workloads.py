"""Synthetic workloads of the benchmark configurations (seeded, CPU-drawn).

Shapes and distributions are BASELINE's configs; draws use
``torch.Generator('cpu').manual_seed(seed)`` in the order q, k, v, i, f (then
C, n, m), in float32, then cast.  Seeds: cfg0 -> 0, cfg1 -> 1, cfg2 -> 2,
cfg4 (the sLSTM layer) -> 4.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

__all__ = ["ChunkwiseConfig", "StepConfig", "SLSTMConfig", "CFG0", "CFG1", "CFG2", "CFG4_SLSTM",
           "chunkwise_inputs", "step_inputs", "slstm_inputs", "soft_cap15"]


@dataclass(frozen=True)
class ChunkwiseConfig:
    name: str
    B: int
    NH: int
    S: int
    DQK: int
    DV: int
    L: int
    dtype: torch.dtype
    seed: int


@dataclass(frozen=True)
class StepConfig:
    name: str
    B: int
    NH: int
    DQK: int
    DV: int
    dtype: torch.dtype
    seed: int


@dataclass(frozen=True)
class SLSTMConfig:
    name: str
    B: int
    S: int
    NH: int
    H: int
    dtype: torch.dtype
    seed: int


CFG0 = ChunkwiseConfig("cfg0_chunkwise_fp32", 1, 8, 256, 256, 512, 64, torch.float32, 0)
CFG1 = StepConfig("cfg1_decode_step_bf16", 16, 8, 256, 512, torch.bfloat16, 1)
CFG2 = ChunkwiseConfig("cfg2_chunkwise_prefill_bf16", 4, 8, 8192, 256, 512, 64, torch.bfloat16, 2)
# config 4's sLSTM layer: NH = 4 heads of H = 512 (d = 2048), B = 8, S = 4096 prefill
CFG4_SLSTM = SLSTMConfig("cfg4_slstm_layer_bf16", 8, 4096, 4, 512, torch.bfloat16, 4)


def soft_cap15(x: torch.Tensor) -> torch.Tensor:
    return 15.0 * torch.tanh(x / 15.0)


def chunkwise_inputs(cfg: ChunkwiseConfig, device="cpu", S: int | None = None, NH: int | None = None,
                     B: int | None = None):
    """q = N(0,1)/sqrt(DQK), k, v = N(0,1), i = N(0,1), f = N(3,1); returns (q, k, v, i, f)."""
    B = B or cfg.B
    NH = NH or cfg.NH
    S = S or cfg.S
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    q = torch.randn(B, NH, S, cfg.DQK, generator=g) / (cfg.DQK ** 0.5)
    k = torch.randn(B, NH, S, cfg.DQK, generator=g)
    v = torch.randn(B, NH, S, cfg.DV, generator=g)
    i = torch.randn(B, NH, S, generator=g)
    f = torch.randn(B, NH, S, generator=g) + 3.0
    return tuple(t.to(cfg.dtype).to(device) for t in (q, k, v, i, f))


def step_inputs(cfg: StepConfig, device="cpu", gate_dtype=torch.float32):
    """q, k, v ~ N(0,1) in cfg.dtype; C = 0.1 N(0,1), n = |N(0,1)|, m = N(0,1) float32;
    i = 15 tanh(N(0,1)/15), f = 15 tanh(N(3,1)/15)."""
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    B, NH, DQK, DV = cfg.B, cfg.NH, cfg.DQK, cfg.DV
    q = torch.randn(B, NH, DQK, generator=g)
    k = torch.randn(B, NH, DQK, generator=g)
    v = torch.randn(B, NH, DV, generator=g)
    i = soft_cap15(torch.randn(B, NH, 1, generator=g))
    f = soft_cap15(torch.randn(B, NH, 1, generator=g) + 3.0)
    C = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n = torch.randn(B, NH, DQK, generator=g).abs()
    m = torch.randn(B, NH, 1, generator=g)
    qkv = tuple(t.to(cfg.dtype).to(device) for t in (q, k, v))
    gates = tuple(t.to(gate_dtype).to(device) for t in (i, f))
    return qkv + gates + (C.to(device), n.to(device), m.to(device))


def slstm_inputs(cfg: SLSTMConfig, device="cpu"):
    """z [B,S,NH,H] ~ N(0,1); i ~ N(0,1), f ~ N(3,1), o ~ N(0,1) [B,S,NH]; drawn in that order, cast to
    cfg.dtype (the sequence starts from the zero state)."""
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    z = torch.randn(cfg.B, cfg.S, cfg.NH, cfg.H, generator=g)
    i = torch.randn(cfg.B, cfg.S, cfg.NH, generator=g)
    f = torch.randn(cfg.B, cfg.S, cfg.NH, generator=g) + 3.0
    o = torch.randn(cfg.B, cfg.S, cfg.NH, generator=g)
    return tuple(t.to(cfg.dtype).to(device) for t in (z, i, f, o))
