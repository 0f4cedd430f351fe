"""Public FlashAttention-2 style API of the gfx950 build.

Same names, signatures, defaults, validation order and messages as the
reference's ``flash_attn_triton/flash_attn_interface.py`` (cited per
function), so existing call sites keep working.  Every attention result is
computed by the HIP kernels in ``libfa_gfx950.so``; there is no Triton and no
host-side fallback.

Deliberate differences from the reference (each one removes a reference
defect or a host-side copy, never changes a correct result):

* inputs are not padded to multiples of 64, grouped KV heads are never
  repeated, strided inputs are read in place: the kernels handle ragged
  lengths, GQA and BSHD strides directly;
* bf16 inputs are accepted in addition to the reference's fp16 / fp32
  (fp32 runs in fp32 throughout, on the fp32 matrix core);
* ``flash_attn_with_kvcache`` runs one batched split-KV launch instead of a
  Python loop of gathers and O(L^2) padded launches, and its causal
  alignment is bottom-right for every cache length (the reference's dense
  stage split drops keys past the first tile when ``L > BLOCK_M``);
* gradients run on HIP backward kernels (deterministic: grouped KV heads
  are reduced in the kernel, not with atomics) for dense, cross and varlen
  calls in fp16 / bf16 / fp32, ``attn_bias``, seqused / paged varlen and
  the KV-cache path, which, when gradients are needed, gathers each
  sequence's keys as the reference does and runs the dense kernels;
* dropout draws its mask from a counter-based Philox4x32-10 generator keyed
  by a seed from torch's default CPU generator, one independent mask per
  (batch, head) (the reference's ``tl.rand`` offsets repeat the same mask for
  every head), and the backward uses the exact gradient of the dropped
  forward.
"""
from __future__ import annotations

import itertools
import math
from typing import Optional

import torch

from .triton_kernel.attention_kernel import (
    _kernel_ready,
    _needs_grad,
    _wrap_grad,
    attention,
    attention_varlen,
    dense_attention,
    dense_forward,
    new_dropout_seed,
    varlen_attention,
    varlen_forward,
)
from . import _native
from ._checks import Deferred

BLOCK_SIZE = 64

def _normalize_alibi(alibi_slopes, batch, heads, device):
    """(H,) or (B,H) fp32 slopes -> contiguous (B,H) (flash_attn_interface.py:128-136)."""
    if alibi_slopes is None:
        return None
    alibi_slopes = torch.as_tensor(alibi_slopes, device=device, dtype=torch.float32)
    if alibi_slopes.ndim == 1:
        if alibi_slopes.shape[0] != heads:
            raise ValueError("alibi_slopes must have one value per query head")
        alibi_slopes = alibi_slopes.unsqueeze(0).expand(batch, -1)
    elif alibi_slopes.shape != (batch, heads):
        raise ValueError("alibi_slopes must have shape (nheads,) or (batch, nheads)")
    return alibi_slopes.contiguous()


def _bias4(attn_bias, batch, heads, q_len, k_len, device):
    """``attn_bias`` as a 4-D fp32 tensor that broadcasts to the ``[B, H, Sq,
    Sk]`` scores (leading size-1 dims added); the kernels read it through the
    expanded view, whose broadcast dims have stride 0.  The conversion is a
    differentiable torch op, so a gradient of this tensor reaches attn_bias.

    The reference adds it to the score tensor with torch broadcasting
    (flash_attn_interface.py:40-41), so any shape that broadcasts to the
    scores is accepted.
    """
    bias = torch.as_tensor(attn_bias, device=device)
    if bias.device != device:
        bias = bias.to(device)
    bias = bias.to(torch.float32)
    shape = (batch, heads, q_len, k_len)
    try:
        fits = bias.ndim <= 4 and torch.broadcast_shapes(tuple(bias.shape), shape) == shape
    except RuntimeError:
        fits = False
    if not fits:
        raise ValueError(
            f"attn_bias of shape {tuple(bias.shape)} does not broadcast to the scores "
            f"({batch}, {heads}, {q_len}, {k_len})")
    return bias.reshape((1,) * (4 - bias.ndim) + tuple(bias.shape))


def _attention_with_probs(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap,
                          alibi_slopes, attn_bias=None, causal_offset=0):
    """Materialized-probabilities path (``return_attn_probs`` / ``attn_bias``).

    Same contract as the reference's dense torch path
    (flash_attn_interface.py:15-49): scores are scaled, ALiBi is subtracted at
    ``|i + causal_offset - j|``, ``attn_bias`` is added, softcap applied, the
    causal/window mask uses ``qpos = i + causal_offset``; returns ``(out [B,Sq,Hq,D],
    lse [B,Hq,Sq] fp32, probs [B,Hq,Sq,Sk] fp32)`` with -inf LSE and zero
    probabilities for rows that see no key.  ``out`` and ``lse`` come from the
    flash kernel (bias applied in its score epilogue), ``probs`` from
    ``fa_attn_probs``.  With dropout the returned probabilities are the
    dropped and rescaled ones the output was computed from (:46-48).
    """
    seed = new_dropout_seed() if dropout_p > 0.0 else 0
    batch, q_len, q_heads, head_dim = q.shape
    k_len = k.shape[1]
    if head_dim not in (16, 32, 64, 128, 256):
        raise ValueError("head dimension must be one of 16, 32, 64, 128, or 256")
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    bias = None
    if attn_bias is not None:
        bias = _bias4(attn_bias, batch, q_heads, q_len, k_len, q.device)
    alibi = None
    if alibi_slopes is not None:
        alibi = _normalize_alibi(alibi_slopes, batch, q_heads, q.device)
    out, lse = dense_attention(q, k, v, softmax_scale=scale, causal=causal,
                             q_pos_offset=causal_offset, window_left=window_size[0],
                             window_right=window_size[1], softcap=softcap, alibi=alibi,
                             return_lse=True, bias=bias, dropout_p=dropout_p,
                             dropout_seed=seed)
    probs = torch.empty((batch, q_heads, q_len, k_len), dtype=torch.float32, device=q.device)
    _native.attn_probs(_kernel_ready(q), _kernel_ready(k), lse, probs, None, None, None,
                       q_len, k_len, scale, causal, causal_offset, window_size[0],
                       window_size[1], softcap, alibi,
                       None if bias is None else bias.detach().expand(batch, q_heads, q_len, k_len),
                       dropout_p, seed)
    return out, lse, probs


def _varlen_attention_with_probs(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                 max_seqlen_k, dropout_p, softmax_scale, causal, window_size,
                                 softcap, alibi):
    """``flash_attn_varlen_func(return_attn_probs=True)`` (reference :642-659).

    Returns ``(out [Tq,Hq,D], lse [B,Hq,max_seqlen_q] fp32 (-inf padding),
    probs [B,Hq,max_seqlen_q,max_seqlen_k] fp32 (zero padding))``; each
    sequence is upper-left aligned with local positions.
    """
    seed = new_dropout_seed() if dropout_p > 0.0 else 0
    batch = cu_seqlens_q.numel() - 1
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else softmax_scale
    out, lse_tok = varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                  max_seqlen_k, softmax_scale=scale, causal=causal,
                                  window_left=window_size[0], window_right=window_size[1],
                                  softcap=softcap, alibi=alibi, return_lse=True,
                                  dropout_p=dropout_p, dropout_seed=seed)
    lses = torch.empty((batch, q.shape[1], max_seqlen_q), dtype=torch.float32, device=q.device)
    probs = torch.empty((batch, q.shape[1], max_seqlen_q, max_seqlen_k), dtype=torch.float32,
                        device=q.device)
    _native.attn_probs(_kernel_ready(q), _kernel_ready(k), lse_tok, probs, lses, cu_seqlens_q,
                       cu_seqlens_k, max_seqlen_q, max_seqlen_k, scale, causal, 0,
                       window_size[0], window_size[1], softcap, alibi, None, dropout_p, seed)
    return out, lses, probs


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                    window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                    deterministic=False, return_attn_probs=False, use_native_gqa=False,
                    attn_bias=None):
    """Flash attention forward (reference flash_attn_interface.py:68-246).

    Arguments:
        q: (batch_size, seqlen, nheads, headdim)
        k: (batch_size, seqlen, nheads_k, headdim)
        v: (batch_size, seqlen, nheads_k, headdim)
        dropout_p: float. Dropout probability on the attention probabilities.
        softmax_scale: float. Default 1 / sqrt(headdim).
        causal: bool. Upper-left aligned causal mask.
        window_size: (left, right). Sliding window, -1 = unbounded.
        softcap: float. softcap * tanh(score / softcap) when > 0.
        alibi_slopes: (nheads,) or (batch_size, nheads) fp32; subtracted as
            slope * |i - j| before softcap.
        deterministic, use_native_gqa: accepted for compatibility; the forward
            kernel is deterministic and always reads grouped KV heads natively.
    Return:
        out: (batch_size, seqlen, nheads, headdim).
    """
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("This implementation supports FP16, BF16 and FP32 tensors")
    if softcap < 0.0:
        raise ValueError("softcap must be non-negative")
    if dropout_p < 0.0 or dropout_p >= 1.0:
        raise ValueError("dropout_p must be in the range [0, 1)")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("All attention tensors must be CUDA tensors")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have shape (batch, seqlen, heads, headdim)")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, and v must have the same dtype")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, and v must be on the same CUDA device")

    batch_size, seq_len_q, n_heads_q, head_dim = q.shape
    key_batch_size, seq_len_k, n_heads_k, key_head_dim = k.shape
    value_batch_size, value_seq_len, value_heads, value_head_dim = v.shape
    if key_batch_size != batch_size or value_batch_size != batch_size:
        raise ValueError("q, k, and v must have the same batch size")
    if value_seq_len != seq_len_k:
        raise ValueError("k and v must have the same sequence length")
    if key_head_dim != head_dim or value_head_dim != head_dim:
        raise ValueError("q, k, and v must have the same head dimension")
    if value_heads != n_heads_k:
        raise ValueError("k and v must have the same number of heads")
    if n_heads_k == 0 or n_heads_q % n_heads_k != 0:
        raise ValueError(
            f"Number of heads in Q ({n_heads_q}) must be divisible by number of heads in K/V ({n_heads_k})"
        )
    alibi_slopes = _normalize_alibi(alibi_slopes, batch_size, n_heads_q, q.device)
    use_alibi = alibi_slopes is not None and bool(torch.any(alibi_slopes != 0))

    if return_attn_probs:
        return _attention_with_probs(q, k, v, dropout_p, softmax_scale, causal, window_size,
                                     softcap, alibi_slopes, attn_bias)
    if attn_bias is not None:
        return _attention_with_probs(q, k, v, dropout_p, softmax_scale, causal, window_size,
                                     softcap, alibi_slopes, attn_bias)[0]

    if seq_len_q != seq_len_k:
        return flash_attn_func_cross(
            q, k, v, dropout_p=dropout_p, softmax_scale=softmax_scale,
            causal=causal, use_native_gqa=use_native_gqa, softcap=softcap,
            alibi_slopes=alibi_slopes, window_size=window_size,
            deterministic=deterministic,
        )
    # Equal-length path: unsupported head dims surface as AssertionError, as in
    # the reference's _launch_dense_forward (attention_kernel.py:1063-1064).
    assert head_dim in {16, 32, 64, 128, 256}
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(head_dim)
    return dense_attention(q, k, v, softmax_scale=softmax_scale, causal=causal,
                           window_left=window_size[0], window_right=window_size[1],
                           softcap=softcap, alibi=alibi_slopes if use_alibi else None,
                           dropout_p=dropout_p,
                           dropout_seed=new_dropout_seed() if dropout_p > 0.0 else 0)


def flash_attn_func_cross(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                          use_native_gqa=False, softcap=0.0, alibi_slopes=None,
                          window_size=(-1, -1), deterministic=False,
                          return_attn_probs=False, attn_bias=None, _causal_offset=0):
    """Cross attention for unequal query and KV lengths (reference :249-330).

    Query row ``i`` sits at position ``i + _causal_offset`` (0: upper-left,
    the SDPA convention for rectangular masks).
    """
    if (q.dtype not in (torch.float16, torch.bfloat16, torch.float32) or k.dtype != q.dtype
            or v.dtype != q.dtype):
        raise ValueError("flash_attn_func_cross supports matching FP16, BF16 or FP32 tensors")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("All attention tensors must be CUDA tensors")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have shape (batch, seqlen, heads, headdim)")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, and v must be on the same CUDA device")
    if k.shape[0] != q.shape[0] or v.shape[:2] != k.shape[:2]:
        raise ValueError("q, k, and v have incompatible batch or sequence dimensions")
    if q.shape[-1] != k.shape[-1] or k.shape[-1] != v.shape[-1]:
        raise ValueError("q, k, and v must have the same head dimension")
    if q.shape[-1] not in (16, 32, 64, 128, 256):
        raise ValueError("head dimension must be one of 16, 32, 64, 128, or 256")
    if q.shape[2] % k.shape[2] != 0:
        raise ValueError("The number of query heads must be divisible by KV heads")
    if dropout_p < 0.0 or dropout_p >= 1.0:
        raise ValueError("dropout_p must be in the range [0, 1)")
    if softcap < 0.0:
        raise ValueError("softcap must be non-negative")
    if v.shape[2] != k.shape[2]:
        raise ValueError("k and v must have the same number of heads")

    q_heads = q.shape[2]
    alibi_slopes = _normalize_alibi(alibi_slopes, q.shape[0], q_heads, q.device)
    use_alibi = alibi_slopes is not None and bool(torch.any(alibi_slopes != 0))

    if return_attn_probs:
        return _attention_with_probs(q, k, v, dropout_p, softmax_scale, causal, window_size,
                                     softcap, alibi_slopes, attn_bias,
                                     causal_offset=_causal_offset)
    if attn_bias is not None:
        return _attention_with_probs(q, k, v, dropout_p, softmax_scale, causal, window_size,
                                     softcap, alibi_slopes, attn_bias,
                                     causal_offset=_causal_offset)[0]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    return dense_attention(q, k, v, softmax_scale=softmax_scale, causal=causal,
                           q_pos_offset=_causal_offset, window_left=window_size[0],
                           window_right=window_size[1], softcap=softcap,
                           alibi=alibi_slopes if use_alibi else None, dropout_p=dropout_p,
                           dropout_seed=new_dropout_seed() if dropout_p > 0.0 else 0)


def flash_attn_qkvpacked_func(qkv, dropout_p=0.0, softmax_scale=None, causal=False,
                              window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                              deterministic=False, return_attn_probs=False,
                              use_native_gqa=False, attn_bias=None):
    """Packed QKV (reference :337-371). qkv: (batch_size, seqlen, 3, nheads, headdim).

    The three strided slices are read in place (token stride 3*H*D); the
    reference copies each slice to a contiguous tensor first.
    """
    qkv = qkv.contiguous() if not qkv.is_contiguous() else qkv
    q, k, v = qkv.unbind(dim=2)
    return flash_attn_func(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap,
                           alibi_slopes, deterministic, return_attn_probs, use_native_gqa,
                           attn_bias)


def flash_attn_kvpacked_func(q, kv, dropout_p=0.0, softmax_scale=None, causal=False,
                             window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                             deterministic=False, return_attn_probs=False,
                             use_native_gqa=False, attn_bias=None):
    """Packed KV (reference :374-406). kv: (batch_size, seqlen_k, 2, nheads_k, headdim)."""
    kv = kv.contiguous() if not kv.is_contiguous() else kv
    k, v = kv.unbind(dim=2)
    return flash_attn_func(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap,
                           alibi_slopes, deterministic, return_attn_probs, use_native_gqa,
                           attn_bias)


def flash_attn_with_kvcache(
    q,
    k_cache,
    v_cache,
    k=None,
    v=None,
    rotary_cos=None,
    rotary_sin=None,
    cache_seqlens=None,
    cache_batch_idx=None,
    cache_leftpad=None,
    block_table=None,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    rotary_interleaved=True,
    alibi_slopes=None,
):
    """Attention against a (paged or batched) KV cache (reference :409-525).

    q: (batch, seqlen_q, nheads, headdim).  Paged: k_cache/v_cache
    (num_pages, page_size, nheads_k, headdim) with block_table
    (batch, max_num_pages) int32; batched: (batch_cache, seqlen_cache,
    nheads_k, headdim).  cache_seqlens: visible keys per batch item.  With
    ``causal`` query i sits at position ``i + L - seqlen_q`` (bottom-right).
    Returns (batch, seqlen_q, nheads, headdim).
    """
    paged = block_table is not None
    # Without an append, rotary or ALiBi slopes nothing the launch needs comes
    # from the device checks, and the kernels keep every read inside the
    # caches and the block table whatever cache_seqlens and block_table hold
    # (fa_fwd_kvcache clamps them): the checks then run on a second stream
    # and the attention launch goes out before the host waits for them; they
    # still raise before this call returns.
    launch_first = k is None and v is None and rotary_cos is None and alibi_slopes is None
    chk = Deferred(side=launch_first)
    if (rotary_cos is None) != (rotary_sin is None):
        raise ValueError("rotary_cos and rotary_sin must be supplied together")
    if q.ndim != 4 or k_cache.ndim != 4 or v_cache.ndim != 4:
        raise ValueError("q and KV caches must be rank-4 tensors")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")
    if paged:
        if block_table.ndim != 2 or block_table.shape[0] != q.shape[0]:
            raise ValueError("block_table must have shape (batch, max_num_pages)")
        if block_table.dtype not in (torch.int32, torch.int64):
            raise ValueError("block_table must contain integer page indices")
        chk.check_range(block_table, 0, k_cache.shape[0] - 1,
                        ValueError("block_table contains an invalid physical page index"))
        if cache_leftpad is not None:
            chk.fail(ValueError("cache_leftpad cannot be combined with paged KV caches"))
        page_size = k_cache.shape[1]
        cache_capacity = block_table.shape[1] * page_size
    else:
        cache_capacity = k_cache.shape[1]
    if q.shape[-1] != k_cache.shape[-1]:
        chk.fail(ValueError("q and KV cache dimensions are incompatible"))
    if q.device != k_cache.device or q.device != v_cache.device:
        chk.fail(ValueError("q and KV caches must be on the same device"))
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        chk.fail(ValueError("q and KV caches must have the same dtype"))
    if paged and cache_batch_idx is not None:
        chk.fail(ValueError("cache_batch_idx cannot be combined with paged KV caches"))
    if cache_batch_idx is None:
        cache_rows = None
    else:
        cache_rows = torch.as_tensor(cache_batch_idx, device=q.device, dtype=torch.long).flatten()
        bad_rows = ValueError("cache_batch_idx must contain valid cache-row indices")
        if cache_rows.numel() != q.shape[0]:
            chk.fail(bad_rows)
        chk.check_range(cache_rows, 0, k_cache.shape[0] - 1, bad_rows)
    if cache_leftpad is None:
        leftpads = None
    else:
        leftpads = torch.as_tensor(cache_leftpad, device=q.device, dtype=torch.long).flatten()
        bad_pads = ValueError("cache_leftpad must contain one non-negative value per query batch")
        if leftpads.numel() != q.shape[0]:
            chk.fail(bad_pads)
        chk.check_range(leftpads, 0, None, bad_pads)
    zero_pad = 0 if leftpads is None else leftpads
    cos_t = sin_t = None
    if rotary_cos is not None:
        # The reference casts the tables to the input dtype before rotating
        # (flash_attn_interface.py:56-57); the kernels then rotate in fp32.
        if rotary_cos.ndim != 2 or rotary_sin.shape != rotary_cos.shape:
            chk.fail(ValueError("rotary_cos and rotary_sin must be (seqlen_ro, rotary_dim / 2) "
                                "tables of the same shape"))
        if rotary_cos.shape[-1] * 2 > q.shape[-1]:
            chk.fail(ValueError("rotary tables exceed the head dimension"))
        cos_t = rotary_cos.to(device=q.device).to(q.dtype).float().contiguous()
        sin_t = rotary_sin.to(device=q.device).to(q.dtype).float().contiguous()
    bad_rotary = IndexError("rotary position out of range of the cos/sin tables")
    n_new = 0
    if k is not None or v is not None:
        # Append (reference :468-493), performed in place on the cache.
        if k is None or v is None or k.shape != v.shape:
            chk.fail(ValueError("k and v must be supplied together with matching shapes"))
        if k.shape[0] != q.shape[0] or k.shape[2:] != k_cache.shape[2:]:
            chk.fail(ValueError("new k/v tensors are incompatible with the cache"))
        n_new = k.shape[1]
        if cache_seqlens is None:
            lengths = torch.zeros(q.shape[0], dtype=torch.int64, device=q.device)
        else:
            lengths = torch.as_tensor(cache_seqlens, device=q.device, dtype=torch.int64).flatten()
        bad_fit = ValueError("new KV tensors do not fit in the cache")
        if lengths.numel() != q.shape[0]:
            chk.fail(bad_fit)
        chk.check_range(lengths, 0, None, bad_fit)
        chk.check_range(lengths + zero_pad + n_new, None, cache_capacity, bad_fit)
        if cos_t is not None and lengths.numel() and n_new:
            chk.check((lengths + zero_pad + n_new > cos_t.shape[0]).any(), bad_rotary)
    else:
        if cache_seqlens is None:
            lengths = torch.full((q.shape[0],), cache_capacity, dtype=torch.int32, device=q.device)
        elif (isinstance(cache_seqlens, torch.Tensor) and cache_seqlens.device == q.device
              and cache_seqlens.dtype in (torch.int32, torch.int64)):
            lengths = cache_seqlens.flatten()   # no conversion launch on the common path
        else:
            lengths = torch.as_tensor(cache_seqlens, device=q.device, dtype=torch.int64).flatten()
        bad_lengths = ValueError("cache_seqlens must contain valid lengths for every batch item")
        if lengths.numel() != q.shape[0]:
            chk.fail(bad_lengths)
        if leftpads is None:
            chk.check_range(lengths, 0, cache_capacity, bad_lengths)
        else:
            chk.check_range(lengths, 0, None, bad_lengths)
            chk.check_range(lengths, None, cache_capacity, bad_lengths, plus=leftpads)
    if cos_t is not None and lengths.numel() and q.shape[1]:
        # Query rows rotate at L + leftpad - Sq + i (L after the append);
        # negative positions index from the end of the tables, as torch
        # indexing does in the reference (:516-517).
        first = lengths + n_new + zero_pad - q.shape[1]
        chk.check((first + q.shape[1] > cos_t.shape[0]).any() | (first < -cos_t.shape[0]).any(),
                  bad_rotary)
    if q.shape[-1] not in (16, 32, 64, 128, 256):
        chk.fail(ValueError("head dimension must be one of 16, 32, 64, 128, or 256"))
    if q.shape[2] % k_cache.shape[2] != 0:
        chk.fail(ValueError("The number of query heads must be divisible by KV heads"))
    if q.shape[0] == 0:
        chk.flush()
        return q.new_empty(q.shape)
    try:
        alibi = _normalize_alibi(alibi_slopes, q.shape[0], q.shape[2], q.device)
    except ValueError as exc:
        chk.fail(exc)
    if not launch_first:
        alibi_bits = chk.value_range(alibi.view(torch.int32)) if alibi is not None else None
        values = chk.flush()   # the one host synchronization of this call
        if alibi is not None and values[alibi_bits] == (0, 0):   # every slope +0.0
            alibi = None
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    from .triton_kernel.attention_kernel import _kernel_ready
    lengths32 = lengths.to(torch.int32).contiguous()
    bt32 = block_table.to(device=q.device, dtype=torch.int32).contiguous() if paged else None
    rows32 = cache_rows.to(torch.int32).contiguous() if cache_rows is not None else None
    pads32 = leftpads.to(torch.int32).contiguous() if leftpads is not None else None
    if n_new:
        kn = k.to(device=q.device, dtype=k_cache.dtype)
        vn = v.to(device=q.device, dtype=v_cache.dtype)
        _native.kvcache_append(kn, vn, k_cache, v_cache, lengths32, bt32, rows32, pads32,
                               int(cache_capacity), cos_t, sin_t, rotary_interleaved)
        lengths32 = (lengths32 + n_new).to(torch.int32)
    if _needs_grad(q, k_cache, v_cache):
        if launch_first:
            chk.flush()
        return _kvcache_differentiable(q, k_cache, v_cache, lengths32, bt32, cache_rows, pads32,
                                       cos_t, sin_t, rotary_interleaved, softmax_scale, causal,
                                       window_size, alibi)
    qk = _kernel_ready(q)
    if cos_t is not None and q.shape[1]:
        q_rot = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        _native.rotary_q(q, q_rot, lengths32, pads32, cos_t, sin_t, rotary_interleaved)
        qk = q_rot
    kc, vc = _kernel_ready(k_cache), _kernel_ready(v_cache)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)

    def launch():
        _native.fwd_kvcache(
            qk, kc, vc, out, None, lengths32,
            bt32, rows32, pads32,
            int(cache_capacity), softmax_scale, causal, window_size[0], window_size[1], alibi)

    if launch_first:
        chk.flush(launch)   # the one host synchronization of this call
    else:
        launch()
    return _wrap_grad(out, q)


def _rotary_torch(x, cos_t, sin_t, positions, interleaved):
    """The query rotation of the KV-cache path (``_native.rotary_q``) as torch
    ops, differentiable in ``x`` [1, S, H, D]: tables already rounded to the
    input dtype and held in fp32, the rotation in fp32, one rounding back
    (reference ``_apply_rotary``, flash_attn_interface.py:52-66)."""
    half = cos_t.shape[-1]
    c = cos_t[positions][None, :, None, :]
    s = sin_t[positions][None, :, None, :]
    xf = x.float()
    xr, rest = xf[..., :2 * half], xf[..., 2 * half:]
    if interleaved:
        x1, x2 = xr[..., 0::2], xr[..., 1::2]
        rot = torch.stack((x1 * c - x2 * s, x1 * s + x2 * c), dim=-1).flatten(-2)
    else:
        x1, x2 = xr[..., :half], xr[..., half:]
        rot = torch.cat((x1 * c - x2 * s, x1 * s + x2 * c), dim=-1)
    return torch.cat((rot, rest), dim=-1).to(x.dtype)


def _kvcache_differentiable(q, k_cache, v_cache, lengths32, bt32, cache_rows, pads32, cos_t,
                            sin_t, interleaved, softmax_scale, causal, window_size, alibi):
    """The KV-cache attention when gradients are needed, as the reference
    computes it (flash_attn_interface.py:494-525): per sequence, its keys
    gathered from the cache by differentiable indexing and the dense
    attention with query row i at position i + L - Sq (causal) on the HIP
    forward / backward kernels.  Gradients reach q, k_cache and v_cache (the
    rows a sequence reads); the new k / v of an append are written into the
    cache beforehand and get none, as in the reference, whose append writes
    into a copy."""
    batch, sq = q.shape[0], q.shape[1]
    hk, d = k_cache.shape[2], k_cache.shape[3]
    lens = lengths32.tolist()
    pads = pads32.tolist() if pads32 is not None else [0] * batch
    rows = cache_rows.tolist() if cache_rows is not None else list(range(batch))
    outs = []
    for b in range(batch):
        L, st = int(lens[b]), int(pads[b])
        qb = q[b:b + 1]
        if cos_t is not None and sq:
            pos = torch.arange(sq, device=q.device) + (L - sq + st)
            qb = _rotary_torch(qb, cos_t, sin_t, pos, interleaved)
        if L == 0 or sq == 0:
            outs.append(torch.zeros(qb.shape, dtype=q.dtype, device=q.device))
            continue
        if bt32 is not None:
            page = k_cache.shape[1]
            pages = bt32[b, :(st + L + page - 1) // page].long()
            kb = k_cache[pages].reshape(-1, hk, d)[st:st + L]
            vb = v_cache[pages].reshape(-1, hk, d)[st:st + L]
        else:
            kb = k_cache[rows[b], st:st + L]
            vb = v_cache[rows[b], st:st + L]
        outs.append(dense_attention(
            qb, kb.unsqueeze(0), vb.unsqueeze(0), softmax_scale=softmax_scale, causal=causal,
            q_pos_offset=(L - sq) if causal else 0, window_left=window_size[0],
            window_right=window_size[1], alibi=None if alibi is None else alibi[b:b + 1]))
    return torch.cat(outs, dim=0)


def _packed_index(starts, lengths, device):
    """Row indices ``starts[b] + [0, lengths[b])`` concatenated over b (host lists)."""
    parts = [torch.arange(s, s + n, device=device) for s, n in zip(starts, lengths) if n > 0]
    return torch.cat(parts) if parts else torch.zeros((0,), dtype=torch.long, device=device)


def _compact_varlen(q, k, v, cu_q, cu_k, used_q, used_k, block_table):
    """Gathered ``(q, k, v, cu_q, cu_k)`` holding only the used rows of every
    sequence and the keys of a paged cache in order; the reference builds its
    inputs this way (flash_attn_interface.py:533-581).  Only the
    ``return_attn_probs`` path, which materialises probabilities anyway, uses
    it, and so do gradients through seqused_* and the block table: the forward
    kernels read seqused_* and the block table directly."""
    dev = q.device
    cq, ck = cu_q.tolist(), cu_k.tolist()
    lq = [b - a for a, b in zip(cq[:-1], cq[1:])]
    lk = [b - a for a, b in zip(ck[:-1], ck[1:])]
    uq = used_q.tolist() if used_q is not None else lq
    uk = used_k.tolist() if used_k is not None else lk
    if block_table is not None:
        page = k.shape[1]
        bt = block_table.to(device=dev, dtype=torch.long)
        parts = []
        for b, n in enumerate(uk):
            if n > 0:
                j = torch.arange(n, device=dev)
                parts.append(bt[b, j // page] * page + j % page)
        idx = torch.cat(parts) if parts else torch.zeros((0,), dtype=torch.long, device=dev)
        k = k.reshape(-1, k.shape[2], k.shape[3])[idx]
        v = v.reshape(-1, v.shape[2], v.shape[3])[idx]
    elif used_k is not None:
        idx = _packed_index(ck[:-1], uk, dev)
        k, v = k[idx], v[idx]
    if used_q is not None:
        q = q[_packed_index(cq[:-1], uq, dev)]

    def prefix(lengths):
        return torch.tensor([0] + list(itertools.accumulate(lengths)), dtype=torch.int32,
                            device=dev)
    return q, k, v, prefix(uq), prefix(uk)


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                           max_seqlen_k, dropout_p=0.0, softmax_scale=None, causal=False,
                           window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                           deterministic=False, return_attn_probs=False, block_table=None,
                           seqused_q=None, seqused_k=None, **kwargs):
    """Packed variable-length attention (reference :527-690).

    q: (total_q, nheads, headdim), k/v: (total_k, nheads_k, headdim),
    cu_seqlens_*: (batch + 1,) int32 prefix sums.  Returns (total_q, nheads, headdim).

    block_table (batch, max_pages) int32 makes k / v paged caches
    (num_pages, page_size, nheads_k, headdim): key j of sequence b sits in
    slot j % page_size of page block_table[b, j // page_size], and
    cu_seqlens_k only gives the key counts.  seqused_q / seqused_k (batch,)
    keep the first seqused_*[b] queries / keys of sequence b; the output
    then packs the used queries only (sum(seqused_q) rows), as the
    reference's compaction does (:551-581).  The kernels read the block
    table and the used counts directly: nothing is gathered or copied.
    """
    batch_size = cu_seqlens_q.numel() - 1
    chk = Deferred()
    paged = block_table is not None
    if paged:
        if k.ndim != 4 or v.ndim != 4 or k.shape != v.shape:
            raise ValueError("paged varlen k and v must have shape (pages, page_size, heads, dim)")
        if block_table.ndim != 2 or block_table.shape[0] != cu_seqlens_k.numel() - 1:
            raise ValueError("block_table must have shape (batch, max_num_pages)")
        page_size = k.shape[1]
        lengths_k = (cu_seqlens_k[1:] - cu_seqlens_k[:-1]).to(torch.long)
        page_counts = torch.div(lengths_k + page_size - 1, page_size, rounding_mode="floor")
        bt_long = block_table.to(device=cu_seqlens_k.device, dtype=torch.long)
        cols = torch.arange(block_table.shape[1], device=cu_seqlens_k.device)
        used_pages = cols[None, :] < page_counts[:, None]
        chk.check((((bt_long < 0) | (bt_long >= k.shape[0])) & used_pages).any(),
                  ValueError("block_table contains an invalid physical page index"))
        # Keys past the table's last page do not exist: the reference's gather
        # comes up short and its size check below fails.
        paged_short = (lengths_k > block_table.shape[1] * page_size).any()
    if seqused_q is not None:
        seqused_q = torch.as_tensor(seqused_q, device=q.device, dtype=torch.int64).flatten()
        if seqused_q.numel() != batch_size:
            chk.fail(ValueError("seqused_q must contain one value per sequence"))
        seqused_q = seqused_q.to(cu_seqlens_q.device)
        lengths_q = (cu_seqlens_q[1:] - cu_seqlens_q[:-1]).to(torch.long)
        chk.check(((seqused_q < 0) | (seqused_q > lengths_q)).any(),
                  ValueError("seqused_q exceeds the packed query sequence"))
    if seqused_k is not None:
        seqused_k = torch.as_tensor(seqused_k, device=k.device, dtype=torch.int64).flatten()
        if seqused_k.numel() != batch_size:
            chk.fail(ValueError("seqused_k must contain one value per sequence"))
        seqused_k = seqused_k.to(cu_seqlens_k.device)
        lengths_k = (cu_seqlens_k[1:] - cu_seqlens_k[:-1]).to(torch.long)
        chk.check(((seqused_k < 0) | (seqused_k > lengths_k)).any(),
                  ValueError("seqused_k exceeds the packed KV sequence"))
    if q.ndim != 3 or (not paged and (k.ndim != 3 or v.ndim != 3 or k.shape != v.shape)):
        chk.fail(ValueError("packed q, k, and v must be rank-3 tensors with matching KV shapes"))
    if cu_seqlens_q.ndim != 1 or cu_seqlens_k.ndim != 1:
        chk.fail(ValueError("cu_seqlens arrays must be one-dimensional"))
    if cu_seqlens_q.numel() != cu_seqlens_k.numel():
        chk.fail(ValueError("cu_seqlens_q and cu_seqlens_k must describe the same batch size"))
    bad_start = ValueError("cu_seqlens arrays must start at zero and contain a batch boundary")
    if cu_seqlens_q.numel() == 0:
        chk.fail(bad_start)
    # With seqused_* the reference re-derives that side's cu_seqlens from the
    # used counts (:563, :581), so its start/order/size checks always pass.
    # Range checks on cu_seqlens slices and on its adjacent differences (the
    # sequence lengths): all of them reduce in one fa_check_ranges launch.
    cu_q_first, cu_k_first = cu_seqlens_q[:1], cu_seqlens_k[:1]
    cu_q_last, cu_k_last = cu_seqlens_q[-1:], cu_seqlens_k[-1:]
    if seqused_q is None:
        chk.check_range(cu_q_first, 0, 0, bad_start)
    if seqused_k is None:
        chk.check_range(cu_k_first, 0, 0, bad_start)
    if cu_seqlens_q.numel() > 1:
        bad_order = ValueError("cu_seqlens arrays must be monotonically non-decreasing")
        if seqused_q is None:
            chk.check_range(cu_seqlens_q, 0, None, bad_order, diff=True)
        if seqused_k is None and cu_seqlens_k.numel() > 1:
            chk.check_range(cu_seqlens_k, 0, None, bad_order, diff=True)
    bad_size = ValueError("cu_seqlens values exceed the packed tensor sizes")
    if seqused_q is None:
        chk.check_range(cu_q_last, None, q.shape[0], bad_size)
    else:
        chk.check((cu_seqlens_q[:-1] + seqused_q > q.shape[0]).any(), bad_size)
    if paged:
        chk.check(paged_short, bad_size)
    elif seqused_k is None:
        chk.check_range(cu_k_last, None, k.shape[0], bad_size)
    else:
        chk.check((cu_seqlens_k[:-1] + seqused_k > k.shape[0]).any(), bad_size)
    kv_heads = k.shape[-2]
    if (q.dtype not in (torch.float16, torch.bfloat16, torch.float32) or k.dtype != q.dtype
            or v.dtype != q.dtype):
        chk.fail(ValueError(
            "flash_attn_varlen_func supports matching FP16, BF16 or FP32 tensors"))
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        chk.fail(ValueError("All attention tensors must be CUDA tensors"))
    if q.device != k.device or q.device != v.device:
        chk.fail(ValueError("q, k, and v must be on the same CUDA device"))
    if q.shape[-1] != k.shape[-1] or k.shape[-1] != v.shape[-1]:
        chk.fail(ValueError("q, k, and v must have the same head dimension"))
    if q.shape[-1] not in (16, 32, 64, 128, 256):
        chk.fail(ValueError("head dimension must be one of 16, 32, 64, 128, or 256"))
    if q.shape[1] % kv_heads != 0:
        chk.fail(ValueError("The number of query heads must be divisible by KV heads"))
    if dropout_p < 0.0 or dropout_p >= 1.0:
        chk.fail(ValueError("dropout_p must be in the range [0, 1)"))
    if softcap < 0.0:
        chk.fail(ValueError("softcap must be non-negative"))
    if cu_seqlens_q.device != q.device or cu_seqlens_k.device != q.device:
        chk.fail(ValueError(
            "cu_seqlens arrays must be on the same CUDA device as q, k, and v"))
    cu_seqlens_q = cu_seqlens_q.to(dtype=torch.int32).contiguous()
    cu_seqlens_k = cu_seqlens_k.to(dtype=torch.int32).contiguous()
    if max_seqlen_q < 0 or max_seqlen_k < 0:
        chk.fail(ValueError("max sequence lengths must be non-negative"))
    if not paged:
        # A paged k has exactly the keys cu_seqlens_k names once the size
        # check above passed; seqused_* sides are covered by construction.
        bad_cover = ValueError("cu_seqlens arrays must cover the packed q and KV tensors")
        if seqused_q is None:
            chk.check_range(cu_q_last, q.shape[0], q.shape[0], bad_cover)
        if seqused_k is None:
            chk.check_range(cu_k_last, k.shape[0], k.shape[0], bad_cover)
    elif seqused_q is None:
        chk.check_range(cu_q_last, q.shape[0], q.shape[0],
                        ValueError("cu_seqlens arrays must cover the packed q and KV tensors"))
    if cu_seqlens_q.numel() < 2:
        chk.fail(ValueError("cu_seqlens arrays must describe at least one sequence"))
    bad_max = ValueError("max sequence lengths must cover every packed sequence")
    if seqused_q is not None:
        chk.check_range(seqused_q, None, max_seqlen_q, bad_max)
    else:
        chk.check_range(cu_seqlens_q, None, max_seqlen_q, bad_max, diff=True)
    if seqused_k is not None:
        chk.check_range(seqused_k, None, max_seqlen_k, bad_max)
    else:
        chk.check_range(cu_seqlens_k, None, max_seqlen_k, bad_max, diff=True)
    out_rows = chk.value(seqused_q.sum()) if seqused_q is not None else None
    if max_seqlen_q == 0 or max_seqlen_k == 0:
        values = chk.flush()
        rows = values[out_rows] if out_rows is not None else q.shape[0]
        return q.new_zeros((rows, q.shape[1], q.shape[2]))
    try:
        alibi = _normalize_alibi(alibi_slopes, batch_size, q.shape[1], q.device)
    except ValueError as exc:
        chk.fail(exc)
    # Any nonzero slope?  The fp32 bit patterns' range (one array of the
    # range-check launch): all slopes +0.0 iff min and max are both 0.
    alibi_bits = chk.value_range(alibi.view(torch.int32)) if alibi is not None else None
    if return_attn_probs:
        chk.flush()
        if paged or seqused_q is not None or seqused_k is not None:
            q, k, v, cu_seqlens_q, cu_seqlens_k = _compact_varlen(
                q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, block_table)
        return _varlen_attention_with_probs(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                            max_seqlen_k, dropout_p, softmax_scale, causal,
                                            window_size, softcap, alibi)
    values = chk.flush()   # the one host synchronization of this call
    seed = new_dropout_seed() if dropout_p > 0.0 else 0
    use_alibi = alibi is not None and values[alibi_bits] != (0, 0)
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    cu_out = None
    if seqused_q is not None:
        cu_out = torch.zeros((batch_size + 1,), dtype=torch.int32, device=q.device)
        torch.cumsum(seqused_q, 0, out=cu_out[1:])
    if (paged or seqused_q is not None or seqused_k is not None) and _needs_grad(q, k, v):
        # Gradients: as the reference (:533-581), gather the used rows and the
        # paged keys into packed tensors (indexing that autograd scatters back
        # to q, k, v and the cache), then run the varlen forward and backward
        # on them.
        q, k, v, cu_seqlens_q, cu_seqlens_k = _compact_varlen(
            q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, block_table)
        return varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                softmax_scale=softmax_scale, causal=causal,
                                window_left=window_size[0], window_right=window_size[1],
                                softcap=softcap, alibi=alibi if use_alibi else None,
                                dropout_p=dropout_p, dropout_seed=seed)
    if paged or seqused_q is not None or seqused_k is not None:
        out = varlen_forward(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                             softmax_scale=softmax_scale, causal=causal,
                             window_left=window_size[0], window_right=window_size[1],
                             softcap=softcap, alibi=alibi if use_alibi else None,
                             seqused_q=seqused_q, seqused_k=seqused_k,
                             out_rows=values[out_rows] if out_rows is not None else None,
                             cu_out=cu_out, block_table=block_table, dropout_p=dropout_p,
                             dropout_seed=seed)
        return out
    return varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                            softmax_scale=softmax_scale, causal=causal,
                            window_left=window_size[0], window_right=window_size[1],
                            softcap=softcap, alibi=alibi if use_alibi else None,
                            dropout_p=dropout_p, dropout_seed=seed)


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                    max_seqlen_k, dropout_p=0.0, softmax_scale=None,
                                    causal=False, **kwargs):
    """Varlen with packed KV (reference :692-699). kv: (total_k, 2, nheads_k, headdim)."""
    k, v = kv.unbind(dim=1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                  max_seqlen_k, dropout_p=dropout_p,
                                  softmax_scale=softmax_scale, causal=causal, **kwargs)


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, dropout_p=0.0,
                                     softmax_scale=None, causal=False, **kwargs):
    """Varlen with packed QKV (reference :702-708). qkv: (total, 3, nheads, headdim)."""
    q, k, v = qkv.unbind(dim=1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen,
                                  dropout_p=dropout_p, softmax_scale=softmax_scale,
                                  causal=causal, **kwargs)


class _AttentionModule(torch.nn.Module):
    """Shared configuration of the nn.Module front ends below.

    They mirror the reference's modules (flash_attn_interface.py:711-804):
    the same constructor arguments and attribute names, dropout taken from a
    ``torch.nn.Dropout`` member only in training mode, and a per-call
    ``causal`` that overrides the constructor's.
    """

    def __init__(self, causal, softmax_scale, attention_dropout, window_size, alibi_slopes,
                 deterministic):
        super().__init__()
        self.causal = causal
        self.softmax_scale = softmax_scale
        self.drop = torch.nn.Dropout(attention_dropout)
        self.window_size = window_size
        self.alibi_slopes = alibi_slopes
        self.deterministic = deterministic

    def _options(self, causal):
        """Keyword options shared by every call these modules make."""
        return dict(dropout_p=self.drop.p if self.training else 0.0,
                    softmax_scale=self.softmax_scale,
                    causal=self.causal if causal is None else causal,
                    window_size=self.window_size, alibi_slopes=self.alibi_slopes,
                    deterministic=self.deterministic)


class FlashSelfAttention(_AttentionModule):
    """Self-attention on packed QKV: ``[B, S, 3, H, D]``, or ``[T, 3, H, D]``
    with ``cu_seqlens`` / ``max_seqlen`` (reference :711-736)."""

    def __init__(self, causal=False, softmax_scale=None, attention_dropout=0.0,
                 window_size=(-1, -1), alibi_slopes=None, deterministic=False):
        super().__init__(causal, softmax_scale, attention_dropout, window_size, alibi_slopes,
                         deterministic)

    def forward(self, qkv, causal=None, cu_seqlens=None, max_seqlen=None):
        opts = self._options(causal)
        if cu_seqlens is not None:
            return flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, **opts)
        return flash_attn_qkvpacked_func(qkv, softcap=0.0, **opts)


class FlashCrossAttention(_AttentionModule):
    """Attention of ``q`` against packed ``kv``, split into K and V along
    dim 2 in both forms as the reference does: ``[B, Sk, 2, Hk, D]`` dense,
    ``[Tk, Hk, 2, D]`` with cu_seqlens.  The dense form takes grouped KV heads
    natively outside training (reference :739-770)."""

    def __init__(self, causal=False, softmax_scale=None, attention_dropout=0.0,
                 window_size=(-1, -1), alibi_slopes=None, deterministic=False):
        super().__init__(causal, softmax_scale, attention_dropout, window_size, alibi_slopes,
                         deterministic)

    def forward(self, q, kv, causal=None, cu_seqlens=None, max_seqlen=None,
                cu_seqlens_k=None, max_seqlen_k=None):
        opts = self._options(causal)
        k, v = kv.unbind(dim=2)
        if cu_seqlens is not None:
            return flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens_k, max_seqlen,
                                          max_seqlen_k, **opts)
        return flash_attn_func_cross(q, k, v, use_native_gqa=not self.training, softcap=0.0,
                                     **opts)


class FlashAttention(torch.nn.Module):
    """``flash_attn_func`` as a module with a fixed dropout rate and scale,
    dropout only in training mode (reference :773-804)."""

    def __init__(self, attention_dropout=0.0, softmax_scale=None):
        super().__init__()
        self.dropout_p = attention_dropout
        self.softmax_scale = softmax_scale

    def forward(self, q, k, v, causal=False, attn_bias=None):
        rate = self.dropout_p if self.training else 0.0
        return flash_attn_func(q, k, v, dropout_p=rate, softmax_scale=self.softmax_scale,
                               causal=causal, attn_bias=attn_bias)


__all__ = [
    "BLOCK_SIZE",
    "attention",
    "attention_varlen",
    "flash_attn_func",
    "flash_attn_func_cross",
    "flash_attn_qkvpacked_func",
    "flash_attn_kvpacked_func",
    "flash_attn_with_kvcache",
    "flash_attn_varlen_func",
    "flash_attn_varlen_kvpacked_func",
    "flash_attn_varlen_qkvpacked_func",
    "FlashSelfAttention",
    "FlashCrossAttention",
    "FlashAttention",
]
