"""Bit-exact float32 restatement of the INT8 per-token quantizer and INT8-QK attention.

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg, never by the product package.

Quantizer (reference ``flash_attn_triton/triton_kernel/attention_kernel_int8.py``):

* K rows (``_quantize_k_rows``, ``:58-79``): ``amax = max|k|`` over the head
  dim (exact: fp16 -> fp32 widening is exact); ``s = fp32(max(amax, 1)) / 127``
  (IEEE fp32 division); ``x = fp32(k) * (1 / s)`` with ``1 / s`` an IEEE fp32
  division; ``k8 = x >= 0 ? floor(x + 0.5) : ceil(x - 0.5)`` with the ``+-0.5``
  an fp32 add (``_round_i8``, ``:27-30``).
* Q rows (``_quantize_rows``, ``:33-39``, applied at ``:100,202``): the same,
  except ``x = fp32(q) / s`` is a division, not a multiply by the reciprocal.

numpy float32 scalar/array arithmetic is IEEE-754 binary32 with
round-to-nearest-even, and ``np.floor``/``np.ceil`` are exact, so every step
above is reproduced bit for bit.  The reference's Triton ``/`` may lower to an
approximate divide on NVIDIA; this build defines the quantizer with IEEE
division (the HIP kernels use HIP's correctly rounded fp32 division).

INT8-QK attention (``_attn_fwd_int8``/``_attn_fwd_int8_inner``, ``:82-217``):
``score = f32(q8 . k8) * (s_q * s_k) * sm_scale`` then softmax and ``P V``.
The integer dot product is exact (|q8.k8| <= 127^2 * D < 2^24 for D <= 256), so
the float64 oracle below evaluates the same real-valued scores; the kernel's
fp16 rounding of P and fp32 accumulation stay within the 2e-2 INT8 tolerance.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

__all__ = ["round_half_away", "quantize_k_rows", "quantize_q_rows", "attention_int8"]

_F32 = np.float32


def round_half_away(x: np.ndarray) -> np.ndarray:
    """``x >= 0 ? floor(x + 0.5) : ceil(x - 0.5)`` in float32 (``_round_i8``, int8:27-30)."""
    x = np.asarray(x, dtype=_F32)
    half = _F32(0.5)
    return np.where(x >= 0, np.floor(x + half), np.ceil(x - half)).astype(_F32)


def _row_scale(x: np.ndarray) -> np.ndarray:
    amax = np.max(np.abs(x.astype(_F32)), axis=-1)
    return (np.maximum(amax, _F32(1.0)) / _F32(127.0)).astype(_F32)


def quantize_k_rows(k) -> Tuple[np.ndarray, np.ndarray]:
    """Per-row K quantization, multiply-by-reciprocal form (int8:74-76).

    ``k [..., D]`` (fp16/fp32).  Returns ``(k8 int8 [..., D], s float32 [...])``.
    """
    kf = np.asarray(k).astype(_F32)
    s = _row_scale(kf)
    inv = (_F32(1.0) / s).astype(_F32)
    x = (kf * inv[..., None]).astype(_F32)
    return round_half_away(x).astype(np.int8), s


def quantize_q_rows(q) -> Tuple[np.ndarray, np.ndarray]:
    """Per-row Q quantization, division form (int8:36-38 via :100)."""
    qf = np.asarray(q).astype(_F32)
    s = _row_scale(qf)
    x = (qf / s[..., None]).astype(_F32)
    return round_half_away(x).astype(np.int8), s


def attention_int8(q, k, v, causal: bool = False, sm_scale: Optional[float] = None,
                   seq_len_k: Optional[int] = None, seq_len_q: Optional[int] = None,
                   q_positions=None) -> Tuple[np.ndarray, np.ndarray]:
    """INT8-QK attention on ``[B,H,S,D]`` inputs.

    Keys ``>= seq_len_k`` are masked and query row ``i`` sits at position
    ``i + seq_len_k - seq_len_q`` for the causal test (int8:108-119).
    ``q_positions`` (optional, one per query row) evaluates a subset of query
    rows of a longer sequence: ``q`` then holds only those rows.  Returns
    ``(out [B,H,Sq,D] float64, lse [B,H,Sq] natural log float64)``; a row with
    no visible key gets out 0 and LSE -inf.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v, dtype=np.float64)
    n_ctx, head_dim = k.shape[2], q.shape[3]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    seq_len_k = n_ctx if seq_len_k is None else int(seq_len_k)
    seq_len_q = n_ctx if seq_len_q is None else int(seq_len_q)
    q8, s_q = quantize_q_rows(q)
    k8, s_k = quantize_k_rows(k)
    qk = np.einsum("bhid,bhjd->bhij", q8.astype(np.int64), k8.astype(np.int64))
    scores = qk.astype(np.float64) * (s_q.astype(np.float64)[..., :, None]
                                      * s_k.astype(np.float64)[..., None, :]) * float(sm_scale)
    if q_positions is None:
        q_pos = np.arange(q.shape[2])[:, None] + seq_len_k - seq_len_q
    else:
        q_pos = np.asarray(q_positions, dtype=np.int64)[:, None]
    k_pos = np.arange(n_ctx)[None, :]
    keep = k_pos < seq_len_k
    if causal:
        keep = keep & (q_pos >= k_pos)
    scores = np.where(keep[None, None], scores, -np.inf)
    row_max = np.max(scores, axis=-1, keepdims=True)
    finite = np.where(np.isfinite(row_max), row_max, 0.0)
    ex = np.exp(scores - finite)
    denom = ex.sum(-1, keepdims=True)
    probs = np.where(denom > 0, ex / np.where(denom > 0, denom, 1.0), 0.0)
    with np.errstate(divide="ignore"):
        lse = np.where(denom[..., 0] > 0, np.log(np.where(denom[..., 0] > 0, denom[..., 0], 1.0))
                       + finite[..., 0], -np.inf)
    return np.einsum("bhij,bhjd->bhid", probs, v), lse
