"""Input generation and comparison helpers shared by the parity tests.

Inputs are drawn on the CPU from a seeded ``torch.Generator`` and rounded to
the kernel dtype there, so the HIP path and the float64 oracle see the same
bits.
"""
from __future__ import annotations

import numpy as np
import torch

# Max-abs error bars against the float64 oracle.  fp16: the north-star bar.
# bf16 carries 8 mantissa bits (fp16: 11), so the same computation lands about
# 8x further from the oracle: outputs and P are rounded to bf16.
ATOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
INT8_ATOL = 2e-2


def randn(shape, seed, dtype=torch.float16, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * scale).to(dtype)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def max_abs(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    both_inf = np.isinf(a) & np.isinf(b) & (np.sign(a) == np.sign(b))
    diff = np.where(both_inf, 0.0, np.abs(a - b))
    return float(np.max(diff)) if diff.size else 0.0


def round_to(expected, dtype):
    """The oracle's answer as the output dtype can hold it (round to nearest)."""
    if dtype is None:
        return np.asarray(expected, dtype=np.float64)
    t = torch.from_numpy(np.ascontiguousarray(expected, dtype=np.float64))
    return t.to(dtype).double().numpy()


def half_ulp(expected, dtype):
    """Half the spacing of ``dtype`` values at |expected| (0 without a dtype)."""
    if dtype is None:
        return 0.0
    mant, emin = {torch.float16: (10, -14), torch.bfloat16: (7, -126),
                  torch.float32: (23, -126)}[dtype]
    a = np.abs(np.asarray(expected, dtype=np.float64))
    e = np.floor(np.log2(np.where((a > 0) & np.isfinite(a), a, 1.0)))
    return 0.5 * np.exp2(np.maximum(e, emin) - mant)


def assert_close(actual, expected, atol, what="", dtype=None):
    """Elementwise |actual - expected| <= atol, against the float64 oracle.

    With ``dtype`` the bar is widened by half an ulp of the output dtype at
    the expected value: the kernel's output is its fp32 result rounded once
    to that dtype, so an fp16 output in [4, 8) may sit 1.95e-3 from the exact
    value even when the fp32 result is exact.  The reported error is the
    largest excess over the rounding, i.e. the part the bar ``atol`` covers."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    assert np.all(np.isfinite(actual) | np.isinf(expected)), f"{what}: non-finite output"
    both_inf = np.isinf(actual) & np.isinf(expected) & (np.sign(actual) == np.sign(expected))
    diff = np.where(both_inf, 0.0, np.abs(actual - expected))
    excess = diff - half_ulp(expected, dtype)
    err = float(np.max(excess)) if excess.size else 0.0
    assert err <= atol, f"{what}: max-abs error {err:.3e} beyond rounding > {atol:.1e}"
