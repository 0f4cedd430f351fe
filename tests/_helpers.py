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


def assert_close(actual, expected, atol, what="", dtype=None):
    """max |actual - expected| <= atol.  With ``dtype`` the float64 oracle is
    first rounded to that output dtype: an fp16 output in [4, 8) cannot be
    closer than half an ulp (1.95e-3) to the exact value, so the bar applies
    to the distance from the nearest representable answer."""
    expected = round_to(expected, dtype)
    err = max_abs(actual, expected)
    assert np.all(np.isfinite(actual) | np.isinf(expected)), f"{what}: non-finite output"
    assert err <= atol, f"{what}: max-abs error {err:.3e} > {atol:.1e}"
