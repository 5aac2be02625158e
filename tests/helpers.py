"""Shared helpers of the GPU parity tests."""

import torch

# Tolerances of the parity bar (stated once, used by every GPU test):
#  float32 inputs: relative error <= 1e-4, measured as max|a-b| / max|b| over
#                  the tensor (so tiny elements do not dominate);
#  bf16/f16 inputs: max-abs error <= 2e-2 on h and on the final C, n, m,
#                  against the float32 oracle run on the 16-bit inputs upcast.
FP32_REL = 1e-4
LOWP_ABS = 2e-2


def relerr(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def maxabs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def assert_parity(got, want, dtype, what=""):
    """fp32: relerr <= FP32_REL; 16-bit: maxabs <= LOWP_ABS."""
    if dtype == torch.float32:
        e = relerr(got, want)
        assert e <= FP32_REL, f"{what}: rel-err {e:.3e} > {FP32_REL}"
    else:
        e = maxabs(got, want)
        assert e <= LOWP_ABS, f"{what}: max-abs {e:.3e} > {LOWP_ABS}"
    return e


def gpu_available() -> bool:
    return torch.cuda.is_available()


def dev():
    return torch.device("cuda:0")
