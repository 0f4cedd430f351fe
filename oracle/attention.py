"""Float64 CPU restatement of the reference's forward attention semantics.

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg, never by the product package.

All arrays are numpy.  Inputs may be any float dtype; they are widened to
float64 before any arithmetic, so the oracle carries no fp16/bf16 rounding of
its own (the reference's tests compare against SDPA at 2e-2, the build's
tolerance against this oracle is 2e-3 for fp16/bf16 and 2e-2 for INT8-QK).

Semantics (reference citations are into /root/reference):

* score pipeline order: scale -> ALiBi ``-slope*|qpos-kpos|`` -> attn_bias ->
  softcap ``C*tanh(s/C)`` -> mask to -inf -> softmax
  (``flash_attn_triton/flash_attn_interface.py:26,36-43``; the kernels do the
  same in ``attention_kernel.py:306-338`` and ``:80-86``).
* positions: ``qpos = i + causal_offset``, ``kpos = j``; causal keeps
  ``qpos >= kpos``; a window keeps ``kpos >= qpos-left`` (left >= 0) and
  ``kpos <= qpos+right`` (right >= 0)  (``flash_attn_interface.py:27-35``).
  Dense, cross and varlen use upper-left alignment (offset 0); the KV-cache
  path passes ``offset = L - Sq`` when causal (``flash_attn_interface.py:523``).
* GQA: query head ``h`` reads KV head ``h // (Hq // Hk)``, the mapping of
  ``repeat_interleave`` (``flash_attn_interface.py:21-24,189``).
* empty rows (every key masked): probabilities 0, output 0, LSE = -inf
  (``flash_attn_interface.py:44-45``; ``attention_kernel.py:522-532``).
* the returned LSE is the natural-log logsumexp, shape ``[B, H, Sq]``
  (``flash_attn_interface.py:45``).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np

__all__ = [
    "attention",
    "attention_backward",
    "attention_varlen",
    "attention_varlen_backward",
    "attention_kvcache",
    "gather_paged_kv",
    "compact_varlen",
    "apply_rotary",
    "philox4x32_10",
    "dropout_factors",
]


# ------------------------------------------------------------------ dropout
_PHILOX_M0, _PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
_PHILOX_W0, _PHILOX_W1 = 0x9E3779B9, 0xBB67AE85


def philox4x32_10(counter, key) -> np.ndarray:
    """Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
    easy as 1, 2, 3", SC 2011; the Random123 parameters) on ``counter [..., 4]``
    uint32 words under ``key = (k0, k1)``; returns ``[..., 4]`` uint32.

    The reference draws its dropout bits with Triton's ``tl.rand`` (Philox,
    attention_kernel.py:354, :92), which lives in the Triton dependency; this
    build defines its own mask (below) on the same generator family.
    """
    c = np.asarray(counter, dtype=np.uint64) & 0xFFFFFFFF
    c0, c1, c2, c3 = (c[..., i].copy() for i in range(4))
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    mask = np.uint64(0xFFFFFFFF)
    for r in range(10):
        if r:
            k0 = (k0 + _PHILOX_W0) & 0xFFFFFFFF
            k1 = (k1 + _PHILOX_W1) & 0xFFFFFFFF
        p0 = np.uint64(_PHILOX_M0) * c0
        p1 = np.uint64(_PHILOX_M1) * c2
        c0, c1, c2, c3 = (((p1 >> np.uint64(32)) ^ c1 ^ np.uint64(k0)) & mask, p1 & mask,
                          ((p0 >> np.uint64(32)) ^ c3 ^ np.uint64(k1)) & mask, p0 & mask)
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def dropout_factors(seed: int, p: float, batch_ids, heads: int, q_len: int,
                    k_len: int) -> np.ndarray:
    """Dropout multipliers ``[len(batch_ids), heads, q_len, k_len]``: 0 for a
    dropped element, ``65536 / (65536 - t16)`` for a kept one, where
    ``t16 = round(p * 65536)``: the reciprocal of the keep probability the
    16-bit draws actually give, so the mask is unbiased (equal to the
    reference's ``1 / (1 - p)`` when ``p * 65536`` is an integer).  A ``p`` that
    would round to ``t16 = 65536`` (no element kept) takes ``t16 = 65535``, as
    the C ABI does, so every ``p`` in [0, 1) is accepted (flash_attn_interface.py:99).

    Element (b, h, i, j) keeps iff its 16-bit draw >= round(p * 65536).  Its
    draw is half ``e = j % 4 + 4 ((j % 16) // 8)`` (word e // 2, high half
    when e is odd) of the Philox call with counter
    ``(2 (j // 16) + (j // 4) % 2, i, h, b)`` and key
    ``(seed mod 2^32, seed // 2^32)``.  Same role as the reference's
    ``tl.rand(seed, offsets) > p`` (attention_kernel.py:344-358, :91-93),
    with every head drawing its own mask.
    """
    p32 = float(np.float32(p))          # the C ABI takes p as an fp32 value
    t16 = min(65535, max(0, int(round(p32 * 65536.0))))
    scale = 65536.0 / (65536.0 - t16)
    b = np.asarray(batch_ids, dtype=np.int64)[:, None, None, None]
    h = np.arange(heads, dtype=np.int64)[None, :, None, None]
    i = np.arange(q_len, dtype=np.int64)[None, None, :, None]
    j = np.arange(k_len, dtype=np.int64)[None, None, None, :]
    shape = (b.shape[0], heads, q_len, k_len)
    ctr = np.stack(np.broadcast_arrays(2 * (j // 16) + (j // 4) % 2, i, h, b), axis=-1)
    words = philox4x32_10(ctr.reshape(-1, 4), (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))
    e = np.broadcast_to(j % 4 + 4 * ((j % 16) // 8), shape).reshape(-1)
    w = words[np.arange(e.size), e // 2].astype(np.int64)
    draw = np.where(e % 2 == 1, w >> 16, w & 0xFFFF).reshape(shape)
    return np.where(draw >= t16, scale, 0.0)


def _keep_mask(q_len: int, k_len: int, causal: bool, window_size: Sequence[int],
               causal_offset: int) -> np.ndarray:
    """Boolean keep-mask ``[q_len, k_len]`` (flash_attn_interface.py:27-35)."""
    q_pos = np.arange(q_len, dtype=np.int64)[:, None] + int(causal_offset)
    k_pos = np.arange(k_len, dtype=np.int64)[None, :]
    keep = np.ones((q_len, k_len), dtype=bool)
    if causal:
        keep &= q_pos >= k_pos
    left, right = int(window_size[0]), int(window_size[1])
    if left >= 0:
        keep &= k_pos >= q_pos - left
    if right >= 0:
        keep &= k_pos <= q_pos + right
    return keep


def attention(q, k, v, softmax_scale: Optional[float] = None, causal: bool = False,
              window_size: Sequence[int] = (-1, -1), softcap: float = 0.0,
              alibi_slopes=None, attn_bias=None, causal_offset: int = 0,
              dropout_p: float = 0.0, dropout_seed: int = 0, batch_ids=None
              ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Dense attention with materialized probabilities.

    Restates ``_attention_with_probs`` (flash_attn_interface.py:15-49) in
    float64.  ``q [B,Sq,Hq,D]``, ``k,v [B,Sk,Hk,D]``; ``alibi_slopes`` is
    ``(Hq,)`` or ``(B,Hq)``; ``attn_bias`` broadcasts to ``[B,Hq,Sq,Sk]``.
    Returns ``(out [B,Sq,Hq,D], lse [B,Hq,Sq], probs [B,Hq,Sq,Sk])``, all float64.
    With ``dropout_p > 0`` the probabilities are multiplied by
    :func:`dropout_factors` (``batch_ids`` name the batch index of each entry,
    default ``0..B-1``) before the product with V and in the returned
    ``probs``; the LSE is that of the undropped scores (:43-48).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    batch, q_len, q_heads, head_dim = q.shape
    k_len, kv_heads = k.shape[1], k.shape[2]
    if q_heads != kv_heads:
        rep = q_heads // kv_heads
        k = np.repeat(k, rep, axis=2)
        v = np.repeat(v, rep, axis=2)
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    # [B,H,Sq,D] @ [B,H,D,Sk]: a batched BLAS product (same sum as the
    # einsum "bqhd,bkhd->bhqk").
    scores = np.matmul(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 3, 1)) * scale
    q_pos = np.arange(q_len, dtype=np.int64) + int(causal_offset)
    k_pos = np.arange(k_len, dtype=np.int64)
    keep = _keep_mask(q_len, k_len, causal, window_size, causal_offset)
    if alibi_slopes is not None:
        slopes = np.asarray(alibi_slopes, dtype=np.float64)
        if slopes.ndim == 1:
            slopes = slopes[None, :]
        dist = np.abs(q_pos[:, None] - k_pos[None, :]).astype(np.float64)
        scores = scores - slopes[:, :, None, None] * dist[None, None]
    if attn_bias is not None:
        scores = scores + np.asarray(attn_bias, dtype=np.float64)
    if softcap > 0:
        scores = softcap * np.tanh(scores / softcap)
    scores = np.where(keep[None, None], scores, -np.inf)
    row_max = np.max(scores, axis=-1, keepdims=True)
    finite_max = np.where(np.isfinite(row_max), row_max, 0.0)
    ex = np.exp(scores - finite_max)
    denom = np.sum(ex, axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        probs = np.where(denom > 0, ex / np.where(denom > 0, denom, 1.0), 0.0)
        lse = np.where(denom[..., 0] > 0, np.log(np.where(denom[..., 0] > 0, denom[..., 0], 1.0))
                       + finite_max[..., 0], -np.inf)
    if dropout_p > 0:
        ids = np.arange(batch) if batch_ids is None else batch_ids
        probs = probs * dropout_factors(dropout_seed, dropout_p, ids, q_heads, q_len, k_len)
    out = np.matmul(probs, v.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3)
    return out, lse, probs


def attention_backward(q, k, v, dout, softmax_scale: Optional[float] = None,
                       causal: bool = False, window_size: Sequence[int] = (-1, -1),
                       softcap: float = 0.0, alibi_slopes=None, causal_offset: int = 0,
                       dropout_p: float = 0.0, dropout_seed: int = 0, batch_ids=None,
                       attn_bias=None, return_dbias: bool = False):
    """Exact gradients ``(dq, dk, dv)`` of :func:`attention`'s output against
    ``dout [B,Sq,Hq,D]``, in float64.

    The chain rule through the score pipeline, as the reference's backward
    kernels compute it (attention_kernel.py:569-668 dK/dV, :671-776 dQ,
    :536-566 delta; the reference's math path :15-49 is differentiated by
    torch autograd the same way): ``dV = P^T dO``, ``dP = dO V^T``,
    ``delta = rowsum(dO * O)``, ``dS = P (dP - delta) (1 - tanh^2)`` (the last
    factor only with softcap), ``dQ = scale dS K``, ``dK = scale dS^T Q``;
    grouped KV heads sum the gradients of their query heads.  With dropout
    (multipliers F): ``dV = (F P)^T dO`` and ``dS = P (F dP - delta)`` -- the
    reference's kernels use ``F P (dP - delta)`` (attention_kernel.py:661,
    :763), which drops the ``- P delta`` term of dropped elements; this is
    the derivative of the forward above.

    ``attn_bias`` (anything that broadcasts to ``[B,Hq,Sq,Sk]``) is added to
    the scaled scores before softcap, as in :func:`attention`; with
    ``return_dbias`` the result gains a fourth entry, ``dS`` summed to the
    bias's own shape (what torch autograd gives the reference's math path,
    flash_attn_interface.py:40-41).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    batch, q_len, q_heads, head_dim = q.shape
    k_len, kv_heads = k.shape[1], k.shape[2]
    rep = q_heads // kv_heads
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    out, _, probs = attention(q, k, v, scale, causal, window_size, softcap, alibi_slopes,
                              attn_bias, causal_offset)
    fac = None
    if dropout_p > 0:
        ids = np.arange(batch) if batch_ids is None else batch_ids
        fac = dropout_factors(dropout_seed, dropout_p, ids, q_heads, q_len, k_len)
        out = np.matmul(probs * fac, np.repeat(v, rep, axis=2).transpose(0, 2, 1, 3)
                        ).transpose(0, 2, 1, 3)
    kr = np.repeat(k, rep, axis=2).transpose(0, 2, 1, 3)     # [B,H,Sk,D]
    vr = np.repeat(v, rep, axis=2).transpose(0, 2, 1, 3)
    qh = q.transpose(0, 2, 1, 3)                              # [B,H,Sq,D]
    doh = dout.transpose(0, 2, 1, 3)
    pd = probs if fac is None else probs * fac
    dv_h = np.matmul(pd.transpose(0, 1, 3, 2), doh)           # [B,H,Sk,D]
    dp = np.matmul(doh, vr.transpose(0, 1, 3, 2))             # [B,H,Sq,Sk]
    if fac is not None:
        dp = dp * fac
    delta = np.sum(doh * out.transpose(0, 2, 1, 3), axis=-1, keepdims=True)
    ds = probs * (dp - delta)
    if softcap > 0:
        raw = np.matmul(qh, kr.transpose(0, 1, 3, 2)) * scale
        if alibi_slopes is not None:
            slopes = np.asarray(alibi_slopes, dtype=np.float64)
            if slopes.ndim == 1:
                slopes = slopes[None, :]
            q_pos = np.arange(q_len) + int(causal_offset)
            dist = np.abs(q_pos[:, None] - np.arange(k_len)[None, :]).astype(np.float64)
            raw = raw - slopes[:, :, None, None] * dist[None, None]
        if attn_bias is not None:
            raw = raw + np.asarray(attn_bias, dtype=np.float64)
        ds = ds * (1.0 - np.tanh(raw / softcap) ** 2)
    dq = (np.matmul(ds, kr) * scale).transpose(0, 2, 1, 3)
    dk_h = np.matmul(ds.transpose(0, 1, 3, 2), qh) * scale
    dk = dk_h.reshape(batch, kv_heads, rep, k_len, head_dim).sum(axis=2).transpose(0, 2, 1, 3)
    dv = dv_h.reshape(batch, kv_heads, rep, k_len, head_dim).sum(axis=2).transpose(0, 2, 1, 3)
    if return_dbias:
        shape = np.shape(attn_bias)
        full = (1,) * (4 - len(shape)) + tuple(shape)
        axes = tuple(i for i in range(4) if full[i] == 1 and ds.shape[i] != 1)
        dbias = np.sum(ds, axis=axes, keepdims=True).reshape(shape)
        return dq, dk, dv, dbias
    return dq, dk, dv


def attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale=None, causal=False,
                     window_size=(-1, -1), softcap=0.0, alibi_slopes=None, dropout_p=0.0,
                     dropout_seed=0) -> Tuple[np.ndarray, np.ndarray]:
    """Packed variable-length attention.

    ``q [Tq,Hq,D]``, ``k,v [Tk,Hk,D]``, ``cu_seqlens_*`` int prefix sums.
    Each sequence uses upper-left alignment with local positions
    (``attention_kernel.py:45-48``).  ``alibi_slopes`` is ``(Hq,)`` or
    ``(batch,Hq)``.  Returns ``(out [Tq,Hq,D], lse [Tq,Hq])`` float64; rows
    whose sequence has no visible key get out 0 and LSE -inf
    (``attention_kernel.py:99-104``).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    cu_k = np.asarray(cu_seqlens_k, dtype=np.int64)
    batch = cu_q.shape[0] - 1
    out = np.zeros(q.shape, dtype=np.float64)
    lse = np.full((q.shape[0], q.shape[1]), -np.inf, dtype=np.float64)
    slopes = None
    if alibi_slopes is not None:
        slopes = np.asarray(alibi_slopes, dtype=np.float64)
        if slopes.ndim == 1:
            slopes = np.broadcast_to(slopes[None, :], (batch, q.shape[1]))
    for b in range(batch):
        qs, qe = int(cu_q[b]), int(cu_q[b + 1])
        ks, ke = int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs:
            continue
        if ke == ks:
            continue
        o, l, _ = attention(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke],
                            softmax_scale, causal, window_size, softcap,
                            None if slopes is None else slopes[b:b + 1],
                            dropout_p=dropout_p, dropout_seed=dropout_seed, batch_ids=[b])
        out[qs:qe] = o[0]
        lse[qs:qe] = l[0].T
    return out, lse


def attention_varlen_backward(q, k, v, dout, cu_seqlens_q, cu_seqlens_k, softmax_scale=None,
                              causal=False, window_size=(-1, -1), softcap=0.0,
                              alibi_slopes=None, dropout_p=0.0, dropout_seed=0
                              ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Gradients of :func:`attention_varlen`: :func:`attention_backward` per
    sequence (attention_kernel.py:107-272); rows outside every sequence get
    zero gradients."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    cu_k = np.asarray(cu_seqlens_k, dtype=np.int64)
    batch = cu_q.shape[0] - 1
    dq, dk, dv = np.zeros(q.shape), np.zeros(k.shape), np.zeros(v.shape)
    slopes = None
    if alibi_slopes is not None:
        slopes = np.asarray(alibi_slopes, dtype=np.float64)
        if slopes.ndim == 1:
            slopes = np.broadcast_to(slopes[None, :], (batch, q.shape[1]))
    for b in range(batch):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs or ke == ks:
            continue
        g = attention_backward(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke],
                               dout[None, qs:qe], softmax_scale, causal, window_size, softcap,
                               None if slopes is None else slopes[b:b + 1],
                               dropout_p=dropout_p, dropout_seed=dropout_seed, batch_ids=[b])
        dq[qs:qe], dk[ks:ke], dv[ks:ke] = g[0][0], g[1][0], g[2][0]
    return dq, dk, dv


def gather_paged_kv(cache, block_table_row, length: int, start: int = 0) -> np.ndarray:
    """Contiguous ``[length, Hk, D]`` view of one sequence of a paged cache.

    ``cache [num_pages, page_size, Hk, D]``; logical token ``t`` lives in page
    ``block_table_row[t // page_size]`` at slot ``t % page_size``
    (``flash_attn_interface.py:509-512``).
    """
    cache = np.asarray(cache)
    page_size = cache.shape[1]
    n_pages = (start + length + page_size - 1) // page_size
    pages = np.asarray(block_table_row[:n_pages], dtype=np.int64)
    flat = cache[pages].reshape(-1, cache.shape[2], cache.shape[3])
    return flat[start:start + length]


def compact_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_q=None, seqused_k=None,
                   block_table=None):
    """The reference's input rewrite for paged / partially used varlen
    sequences (``flash_attn_interface.py:533-581``), in its order:

    1. ``block_table`` given: ``k, v [pages, page_size, Hk, D]`` become packed
       ``[sum(len_k), Hk, D]`` by gathering each sequence's first
       ``ceil(len_k / page_size)`` pages and keeping ``len_k`` rows
       (``:538-550``), ``len_k = cu_k[b+1] - cu_k[b]``;
    2. ``seqused_q``: sequence b keeps its first ``seqused_q[b]`` queries and
       ``cu_q`` is rebuilt from the used counts (``:551-563``);
    3. ``seqused_k``: the same for keys and values (``:564-581``).

    Returns ``(q, k, v, cu_q, cu_k)`` ready for :func:`attention_varlen`.
    """
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    cu_q = [int(x) for x in np.asarray(cu_seqlens_q)]
    cu_k = [int(x) for x in np.asarray(cu_seqlens_k)]
    batch = len(cu_q) - 1
    if block_table is not None:
        bt = np.asarray(block_table)
        kp = [gather_paged_kv(k, bt[b], cu_k[b + 1] - cu_k[b]) for b in range(batch)]
        vp = [gather_paged_kv(v, bt[b], cu_k[b + 1] - cu_k[b]) for b in range(batch)]
        k = np.concatenate(kp) if kp else k[:0, 0]
        v = np.concatenate(vp) if vp else v[:0, 0]
    if seqused_q is not None:
        used = [int(x) for x in np.asarray(seqused_q)]
        q = np.concatenate([q[cu_q[b]:cu_q[b] + used[b]] for b in range(batch)])
        cu_q = [0] + list(np.cumsum(used))
    if seqused_k is not None:
        used = [int(x) for x in np.asarray(seqused_k)]
        k = np.concatenate([k[cu_k[b]:cu_k[b] + used[b]] for b in range(batch)])
        v = np.concatenate([v[cu_k[b]:cu_k[b] + used[b]] for b in range(batch)])
        cu_k = [0] + list(np.cumsum(used))
    return q, k, v, np.asarray(cu_q, dtype=np.int64), np.asarray(cu_k, dtype=np.int64)


def apply_rotary(x, cos, sin, positions, interleaved: bool) -> np.ndarray:
    """Rotary embedding of ``x [S,H,D]`` at integer ``positions [S]``.

    ``cos, sin [max_pos, rotary_dim/2]``.  Interleaved (GPT-J) rotates pairs
    ``(x[2i], x[2i+1])``; otherwise (GPT-NeoX) rotates ``(x[i], x[i+r/2])``
    (``flash_attn_interface.py:52-66``).  Dimensions past ``rotary_dim`` pass
    through unchanged.
    """
    x = np.asarray(x, dtype=np.float64)
    cos = np.asarray(cos, dtype=np.float64)
    sin = np.asarray(sin, dtype=np.float64)
    rot = cos.shape[-1] * 2
    c = cos[np.asarray(positions, dtype=np.int64)][:, None, :]
    s = sin[np.asarray(positions, dtype=np.int64)][:, None, :]
    part = x[..., :rot]
    if interleaved:
        even, odd = part[..., 0::2], part[..., 1::2]
        rotated = np.stack((even * c - odd * s, even * s + odd * c), axis=-1).reshape(part.shape)
    else:
        first, second = part[..., :rot // 2], part[..., rot // 2:]
        rotated = np.concatenate((first * c - second * s, first * s + second * c), axis=-1)
    return np.concatenate((rotated, x[..., rot:]), axis=-1)


def attention_kvcache(q, k_cache, v_cache, cache_seqlens=None, block_table=None,
                      cache_batch_idx=None, cache_leftpad=None, softmax_scale=None,
                      causal=False, window_size=(-1, -1), alibi_slopes=None,
                      k_new=None, v_new=None, rotary_cos=None, rotary_sin=None,
                      rotary_interleaved=True):
    """Attention of ``q [B,Sq,Hq,D]`` against a (paged or batched) KV cache.

    Restates ``flash_attn_with_kvcache`` (flash_attn_interface.py:409-525)
    with the cache append actually performed (the reference's append writes
    into an advanced-indexing copy and is lost, flash_attn_interface.py:487-492;
    upstream FlashAttention-2 appends in place).  Returns
    ``(out [B,Sq,Hq,D], lse [B,Hq,Sq], k_cache, v_cache)`` with the caches
    after the append (copies; the inputs are not modified).

    Per batch ``b`` with ``L`` visible keys (after any append) the query
    position offset is ``L - Sq`` when causal and 0 otherwise
    (flash_attn_interface.py:519-524); keys are the cache rows
    ``[leftpad, leftpad + L)`` of cache row ``cache_batch_idx[b]``, or logical
    tokens ``[0, L)`` through ``block_table[b]`` for a paged cache.
    """
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.array(k_cache, dtype=np.float64, copy=True)
    v_cache = np.array(v_cache, dtype=np.float64, copy=True)
    batch, q_len = q.shape[0], q.shape[1]
    paged = block_table is not None
    if paged:
        bt = np.asarray(block_table, dtype=np.int64)
        page_size = k_cache.shape[1]
        capacity = bt.shape[1] * page_size
    else:
        capacity = k_cache.shape[1]
    rows = (np.arange(batch) if cache_batch_idx is None
            else np.asarray(cache_batch_idx, dtype=np.int64).reshape(-1))
    leftpad = (np.zeros(batch, dtype=np.int64) if cache_leftpad is None
               else np.asarray(cache_leftpad, dtype=np.int64).reshape(-1))
    if cache_seqlens is None:
        lengths = np.zeros(batch, dtype=np.int64) if k_new is not None else np.full(batch, capacity, dtype=np.int64)
    else:
        lengths = np.asarray(cache_seqlens, dtype=np.int64).reshape(-1).copy()
        if lengths.size == 1 and batch > 1:
            lengths = np.full(batch, int(lengths[0]), dtype=np.int64)
    if k_new is not None:
        k_new = np.asarray(k_new, dtype=np.float64)
        v_new = np.asarray(v_new, dtype=np.float64)
        n_new = k_new.shape[1]
        for b in range(batch):
            kb = k_new[b]
            if rotary_cos is not None:
                pos = np.arange(n_new) + lengths[b] + leftpad[b]
                kb = apply_rotary(kb, rotary_cos, rotary_sin, pos, rotary_interleaved)
            for t in range(n_new):
                logical = int(lengths[b] + leftpad[b] + t)
                if paged:
                    page = int(bt[b, logical // page_size])
                    k_cache[page, logical % page_size] = kb[t]
                    v_cache[page, logical % page_size] = v_new[b, t]
                else:
                    k_cache[rows[b], logical] = kb[t]
                    v_cache[rows[b], logical] = v_new[b, t]
        lengths = lengths + n_new
    out = np.zeros(q.shape, dtype=np.float64)
    lse = np.full((batch, q.shape[2], q_len), -np.inf, dtype=np.float64)
    slopes = None
    if alibi_slopes is not None:
        slopes = np.asarray(alibi_slopes, dtype=np.float64)
        if slopes.ndim == 1:
            slopes = np.broadcast_to(slopes[None, :], (batch, q.shape[2]))
    for b in range(batch):
        length = int(lengths[b])
        start = int(leftpad[b])
        if paged:
            kb = gather_paged_kv(k_cache, bt[b], length, start)
            vb = gather_paged_kv(v_cache, bt[b], length, start)
        else:
            kb = k_cache[rows[b], start:start + length]
            vb = v_cache[rows[b], start:start + length]
        qb = q[b]
        if rotary_cos is not None:
            pos = np.arange(q_len) + length - q_len + start
            qb = apply_rotary(qb, rotary_cos, rotary_sin, pos, rotary_interleaved)
        if length == 0:
            continue
        o, l, _ = attention(qb[None], kb[None], vb[None], softmax_scale, causal,
                            window_size, 0.0,
                            None if slopes is None else slopes[b:b + 1],
                            causal_offset=(length - q_len) if causal else 0)
        out[b] = o[0]
        lse[b] = l[0]
    return out, lse, k_cache, v_cache
