"""Shared helpers of the GPU parity tests."""

import torch

# Tolerances of the parity bar (stated once, used by every GPU test):
#  float32 inputs: relative error <= 1e-4, measured as max|a-b| / max|b| over
#                  the tensor (so tiny elements do not dominate);
#  bf16/f16 inputs: max-abs error <= 2e-2 on h and on the final C, n, m,
#                  against the float32 oracle run on the 16-bit inputs upcast.
#                  h itself is returned in the 16-bit dtype, and rounding the
#                  exact h to bf16 already costs up to half an ulp of |h|
#                  (0.030 at cfg2, where |h| reaches 11.4), so for a 16-bit
#                  output the 2e-2 applies on top of that half ulp:
#                  |a - b| <= 2e-2 + ulp(b)/2 elementwise (lowp_excess <= 2e-2).
FP32_REL = 1e-4
LOWP_ABS = 2e-2


def relerr(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def maxabs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def half_ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    """Half a unit in the last place of |x| in the 16-bit `dtype` (0 for float32)."""
    if dtype == torch.float32:
        return torch.zeros_like(x, dtype=torch.float64)
    mant = 7 if dtype == torch.bfloat16 else 10
    ax = x.detach().double().cpu().abs().clamp_min(1e-30)
    return torch.exp2(torch.floor(torch.log2(ax)) - mant - 1)


def lowp_excess(got: torch.Tensor, want: torch.Tensor, roundings: int = 1) -> float:
    """max(|got - want| - roundings * ulp(want)/2) with ulp in got's dtype: the error beyond
    `roundings` 16-bit roundings of the output (1: the output's own)."""
    d = (got.detach().double().cpu() - want.detach().double().cpu()).abs()
    return float((d - roundings * half_ulp(want, got.dtype)).max())


def print_margins(got, want, what=""):
    """Prints the raw max-abs error and the excess beyond one, two and three 16-bit roundings of
    the reference's output (the margin the bar at each choice would leave), and returns them."""
    raw = float((got.detach().double().cpu() - want.detach().double().cpu()).abs().max())
    ex = [lowp_excess(got, want, r) for r in (1, 2, 3)]
    print(f"[margin] {what}: max-abs {raw:.3e}; beyond 1 / 2 / 3 roundings {ex[0]:.3e} / {ex[1]:.3e} / {ex[2]:.3e}")
    return raw, ex


def assert_parity(got, want, dtype, what="", roundings=1):
    """fp32: relerr <= FP32_REL; 16-bit inputs: max-abs <= LOWP_ABS beyond the output's own rounding
    (and, with roundings=2, one more 16-bit rounding the reference applies on the way to it)."""
    if dtype == torch.float32:
        e = relerr(got, want)
        assert e <= FP32_REL, f"{what}: rel-err {e:.3e} > {FP32_REL}"
    else:
        e = lowp_excess(got, want, roundings)
        assert e <= LOWP_ABS, f"{what}: max-abs {e:.3e} beyond output rounding > {LOWP_ABS}"
    return e


def gpu_available() -> bool:
    return torch.cuda.is_available()


def dev():
    return torch.device("cuda:0")
