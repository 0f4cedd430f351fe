"""Low-level launch layer (no Triton inside: the module path is kept for drop-in imports).

Mirrors the public launch functions of the reference's
``flash_attn_triton/triton_kernel/attention_kernel.py``:

* ``attention``        (reference ``:1201-1259``) - head-major ``[B, H, S, D]`` views.
* ``attention_varlen`` (reference ``:1364-1380``) - packed ``[T, H, D]`` sequences.

Both call the gfx950 HIP kernels of ``libfa_gfx950.so`` through ``_native``.
The kernels handle ragged lengths, strided inputs and grouped KV heads
directly, so nothing is padded, repeated or copied on the host.

Autograd: when q, k or v (or the dense path's ``attn_bias``) requires grad
the forward also keeps the LSE and the backward runs ``fa_bwd_dense`` /
``fa_bwd_varlen`` (the reference's ``_attention.backward`` :1185-1198 and
``_attention_varlen.backward`` :1322-1361): fp16, bf16 and fp32 at every head
dim; the bias gradient
is dS summed over the bias's broadcast dimensions, as torch autograd gives it
for the reference's math path (flash_attn_interface.py:15-49).  Dropout (``dropout_p > 0``) drops probabilities with the
counter-based Philox mask of the kernels; the seed is drawn from torch's
default CPU generator unless given, and the backward replays the same mask.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .. import _native

__all__ = ["attention", "attention_varlen", "dense_forward", "varlen_forward", "dense_attention",
           "varlen_attention", "dense_backward", "varlen_backward", "new_dropout_seed",
           "FORWARD_ONLY_MSG"]

FORWARD_ONLY_MSG = (
    "flash_attn_triton (gfx950 HIP build): this call has no backward (the KV-cache path is "
    "forward only)")


def new_dropout_seed() -> int:
    """A 62-bit dropout seed from torch's default CPU generator (so
    ``torch.manual_seed`` makes dropout reproducible; no device sync)."""
    return int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64).item())


class _ForwardOnly(torch.autograd.Function):
    """Attach a grad_fn that fails loudly for calls without a backward."""

    @staticmethod
    def forward(ctx, out, *inputs):
        return out.view_as(out)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(FORWARD_ONLY_MSG)


def _wrap_grad(out: torch.Tensor, *inputs: torch.Tensor) -> torch.Tensor:
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs if t is not None):
        return _ForwardOnly.apply(out, *inputs)
    return out


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """The kernels read rows with 16-byte loads: unit innermost stride, strides
    that are multiples of 16 bytes and a 16-byte aligned base.  Other layouts
    get one contiguous copy (the reference copies every non-contiguous input,
    flash_attn_interface.py:202-204)."""
    es = t.element_size()
    if (t.stride(-1) == 1 and all((s * es) % 16 == 0 for s in t.stride()[:-1])
            and t.data_ptr() % 16 == 0):
        return t
    return t.contiguous()


def dense_forward(q, k, v, *, softmax_scale: float, causal: bool, q_pos_offset: int = 0,
                  window_left: int = -1, window_right: int = -1, softcap: float = 0.0,
                  alibi: Optional[torch.Tensor] = None, return_lse: bool = False,
                  bias: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                  dropout_seed: int = 0):
    """Run the dense HIP kernel on ``[B, S, H, D]`` tensors (any BSHD strides).

    ``bias`` (optional) is an fp32 ``[B, Hq, Sq, Sk]`` view (broadcast strides
    allowed) added to the scaled scores.  Returns ``out [B, Sq, Hq, D]``
    (contiguous, dtype of q) and, if requested, the natural-log LSE
    ``[B, Hq, Sq]`` fp32.
    """
    qk, kk, vk = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    B, Sq, Hq, D = q.shape
    out = torch.empty((B, Sq, Hq, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device) if return_lse else None
    if alibi is not None:
        alibi = alibi.to(device=q.device, dtype=torch.float32).contiguous()
    _native.fwd_dense(qk, kk, vk, out, lse, softmax_scale, causal, q_pos_offset, window_left,
                      window_right, softcap, alibi, bias, dropout_p, dropout_seed)
    return (out, lse) if return_lse else out


def varlen_forward(q, k, v, cu_q, cu_k, max_seqlen_q: int, max_seqlen_k: int, *,
                   softmax_scale: float, causal: bool, window_left: int = -1,
                   window_right: int = -1, softcap: float = 0.0,
                   alibi: Optional[torch.Tensor] = None, return_lse: bool = False,
                   seqused_q: Optional[torch.Tensor] = None,
                   seqused_k: Optional[torch.Tensor] = None,
                   out_rows: Optional[int] = None, cu_out: Optional[torch.Tensor] = None,
                   block_table: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                   dropout_seed: int = 0):
    """Run the packed varlen HIP kernel on ``[T, H, D]`` tensors.

    ``seqused_q``/``seqused_k`` limit each sequence to its first queries /
    keys; with ``cu_out`` the outputs of the used queries are packed into
    ``out_rows`` rows (sequence b at ``cu_out[b]``).  With ``block_table``
    k / v are paged caches ``[pages, page_size, Hk, D]``."""
    dev = q.device
    qk, kk, vk = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    rows = q.shape[0] if out_rows is None else int(out_rows)
    out = torch.empty((rows, q.shape[1], q.shape[2]), dtype=q.dtype, device=dev)
    lse = (torch.empty((rows, q.shape[1]), dtype=torch.float32, device=dev)
           if return_lse else None)
    if alibi is not None:
        alibi = alibi.to(device=dev, dtype=torch.float32).contiguous()

    def i32(t):
        return None if t is None else t.to(device=dev, dtype=torch.int32).contiguous()

    _native.fwd_varlen(qk, kk, vk, out, lse, i32(cu_q), i32(cu_k), max_seqlen_q, max_seqlen_k,
                       softmax_scale, causal, window_left, window_right, softcap, alibi,
                       i32(seqused_q), i32(seqused_k), i32(cu_out), i32(block_table),
                       dropout_p, dropout_seed)
    return (out, lse) if return_lse else out


def _needs_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def _pad_head_dim(t: torch.Tensor, d: int) -> torch.Tensor:
    return torch.nn.functional.pad(t, (0, d - t.shape[-1]))


def _f32_alibi(alibi, device):
    return None if alibi is None else alibi.to(device=device, dtype=torch.float32).contiguous()


def dense_backward(q, k, v, out, dout, lse, *, softmax_scale: float, causal: bool,
                   q_pos_offset: int = 0, window_left: int = -1, window_right: int = -1,
                   softcap: float = 0.0, alibi: Optional[torch.Tensor] = None,
                   dropout_p: float = 0.0, dropout_seed: int = 0,
                   bias: Optional[torch.Tensor] = None, dbias: Optional[torch.Tensor] = None):
    """Gradients ``(dq, dk, dv)`` of ``dense_forward`` from ``dout``, given its
    output and LSE (``fa_bwd_dense``).  Head dim 16 runs at 32 with zero padding
    (the extra dims contribute nothing to the scores and get zero gradients).
    ``bias``: the forward's fp32 ``[B, Hq, Sq, Sk]`` view; ``dbias`` (optional):
    a zero-filled fp32 view of the same shape whose broadcast dims have stride
    0, which receives the bias gradient."""
    if q.shape[-1] == 16:
        grads = dense_backward(*(_pad_head_dim(t, 32) for t in (q, k, v, out, dout)), lse,
                               softmax_scale=softmax_scale, causal=causal,
                               q_pos_offset=q_pos_offset, window_left=window_left,
                               window_right=window_right, softcap=softcap, alibi=alibi,
                               dropout_p=dropout_p, dropout_seed=dropout_seed, bias=bias,
                               dbias=dbias)
        return tuple(g[..., :16] for g in grads)
    qk, kk, vk, ok, dok = (_kernel_ready(t) for t in (q, k, v, out, dout))
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    delta = torch.empty_like(lse)
    _native.bwd_dense(qk, kk, vk, ok, dok, lse, dq, dk, dv, delta, softmax_scale, causal,
                      q_pos_offset, window_left, window_right, softcap,
                      _f32_alibi(alibi, q.device), dropout_p, dropout_seed, bias=bias,
                      dbias=dbias)
    return dq, dk, dv


def varlen_backward(q, k, v, out, dout, lse, cu_q, cu_k, max_seqlen_q: int, max_seqlen_k: int,
                    *, softmax_scale: float, causal: bool, window_left: int = -1,
                    window_right: int = -1, softcap: float = 0.0,
                    alibi: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                    dropout_seed: int = 0):
    """Gradients ``(dq, dk, dv)`` of ``varlen_forward`` (``fa_bwd_varlen``).
    Rows outside every sequence get zero gradients."""
    if q.shape[-1] == 16:
        grads = varlen_backward(*(_pad_head_dim(t, 32) for t in (q, k, v, out, dout)), lse,
                                cu_q, cu_k, max_seqlen_q, max_seqlen_k,
                                softmax_scale=softmax_scale, causal=causal,
                                window_left=window_left, window_right=window_right,
                                softcap=softcap, alibi=alibi, dropout_p=dropout_p,
                                dropout_seed=dropout_seed)
        return tuple(g[..., :16] for g in grads)
    qk, kk, vk, ok, dok = (_kernel_ready(t) for t in (q, k, v, out, dout))
    dq = torch.zeros(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.zeros(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.zeros(v.shape, dtype=v.dtype, device=v.device)
    delta = torch.empty_like(lse)
    i32 = lambda t: t.to(device=q.device, dtype=torch.int32).contiguous()
    _native.bwd_varlen(qk, kk, vk, ok, dok, lse, dq, dk, dv, delta, i32(cu_q), i32(cu_k),
                       max_seqlen_q, max_seqlen_k, softmax_scale, causal, window_left,
                       window_right, softcap, _f32_alibi(alibi, q.device), dropout_p,
                       dropout_seed)
    return dq, dk, dv


def _expand_bias(bias4: torch.Tensor, q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """A 4-D fp32 bias as the ``[B, Hq, Sq, Sk]`` score view (stride 0 on its
    size-1 dims)."""
    return bias4.expand(q.shape[0], q.shape[2], q.shape[1], k.shape[1])


class _DenseAttention(torch.autograd.Function):
    """dense_forward with the fa_bwd_dense backward; returns (out, lse).

    ``bias4`` (optional) is the attn_bias as a 4-D fp32 tensor that broadcasts
    to the scores; its gradient comes back in that shape, summed over the
    broadcast dimensions."""

    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, causal, q_pos_offset, window_left, window_right,
                softcap, alibi, dropout_p, dropout_seed, bias4):
        bias = None if bias4 is None else _expand_bias(bias4, q, k)
        out, lse = dense_forward(q, k, v, softmax_scale=softmax_scale, causal=causal,
                                 q_pos_offset=q_pos_offset, window_left=window_left,
                                 window_right=window_right, softcap=softcap, alibi=alibi,
                                 return_lse=True, bias=bias, dropout_p=dropout_p,
                                 dropout_seed=dropout_seed)
        ctx.save_for_backward(q, k, v, out, lse, alibi, bias4)
        ctx.opts = (softmax_scale, causal, q_pos_offset, window_left, window_right, softcap,
                    dropout_p, dropout_seed)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, out, lse, alibi, bias4 = ctx.saved_tensors
        scale, causal, off, wl, wr, cap, dp, seed = ctx.opts
        bias = dbias4 = dbias = None
        if bias4 is not None:
            bias = _expand_bias(bias4, q, k)
            if ctx.needs_input_grad[12]:
                dbias4 = torch.zeros(bias4.shape, dtype=torch.float32, device=q.device)
                dbias = _expand_bias(dbias4, q, k)
        dq, dk, dv = dense_backward(q, k, v, out, dout, lse, softmax_scale=scale, causal=causal,
                                    q_pos_offset=off, window_left=wl, window_right=wr,
                                    softcap=cap, alibi=alibi, dropout_p=dp, dropout_seed=seed,
                                    bias=bias, dbias=dbias)
        return (dq, dk, dv) + (None,) * 9 + (dbias4,)


class _VarlenAttention(torch.autograd.Function):
    """varlen_forward with the fa_bwd_varlen backward; returns (out, lse)."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal,
                window_left, window_right, softcap, alibi, dropout_p, dropout_seed):
        out, lse = varlen_forward(q, k, v, cu_q, cu_k, max_seqlen_q, max_seqlen_k,
                                  softmax_scale=softmax_scale, causal=causal,
                                  window_left=window_left, window_right=window_right,
                                  softcap=softcap, alibi=alibi, return_lse=True,
                                  dropout_p=dropout_p, dropout_seed=dropout_seed)
        ctx.save_for_backward(q, k, v, out, lse, cu_q, cu_k, alibi)
        ctx.opts = (max_seqlen_q, max_seqlen_k, softmax_scale, causal, window_left,
                    window_right, softcap, dropout_p, dropout_seed)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, out, lse, cu_q, cu_k, alibi = ctx.saved_tensors
        mq, mk, scale, causal, wl, wr, cap, dp, seed = ctx.opts
        dq, dk, dv = varlen_backward(q, k, v, out, dout, lse, cu_q, cu_k, mq, mk,
                                     softmax_scale=scale, causal=causal, window_left=wl,
                                     window_right=wr, softcap=cap, alibi=alibi, dropout_p=dp,
                                     dropout_seed=seed)
        return (dq, dk, dv) + (None,) * 12


def dense_attention(q, k, v, *, softmax_scale: float, causal: bool, q_pos_offset: int = 0,
                    window_left: int = -1, window_right: int = -1, softcap: float = 0.0,
                    alibi: Optional[torch.Tensor] = None, return_lse: bool = False,
                    bias: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                    dropout_seed: int = 0):
    """``dense_forward`` that is differentiable in q, k, v and ``bias`` (fp16 /
    bf16).  ``bias`` (optional) is a 4-D fp32 tensor that broadcasts to the
    ``[B, Hq, Sq, Sk]`` scores."""
    if not _needs_grad(q, k, v, bias):
        res = dense_forward(q, k, v, softmax_scale=softmax_scale, causal=causal,
                            q_pos_offset=q_pos_offset, window_left=window_left,
                            window_right=window_right, softcap=softcap, alibi=alibi,
                            return_lse=return_lse,
                            bias=None if bias is None else _expand_bias(bias, q, k),
                            dropout_p=dropout_p, dropout_seed=dropout_seed)
        return res
    out, lse = _DenseAttention.apply(q, k, v, softmax_scale, causal, q_pos_offset, window_left,
                                     window_right, softcap, alibi, dropout_p, dropout_seed, bias)
    return (out, lse) if return_lse else out


def varlen_attention(q, k, v, cu_q, cu_k, max_seqlen_q: int, max_seqlen_k: int, *,
                     softmax_scale: float, causal: bool, window_left: int = -1,
                     window_right: int = -1, softcap: float = 0.0,
                     alibi: Optional[torch.Tensor] = None, return_lse: bool = False,
                     dropout_p: float = 0.0, dropout_seed: int = 0):
    """``varlen_forward`` that is differentiable in q, k, v (fp16 / bf16)."""
    if not _needs_grad(q, k, v):
        return varlen_forward(q, k, v, cu_q, cu_k, max_seqlen_q, max_seqlen_k,
                              softmax_scale=softmax_scale, causal=causal,
                              window_left=window_left, window_right=window_right,
                              softcap=softcap, alibi=alibi, return_lse=return_lse,
                              dropout_p=dropout_p, dropout_seed=dropout_seed)
    out, lse = _VarlenAttention.apply(q, k, v, cu_q, cu_k, max_seqlen_q, max_seqlen_k,
                                      softmax_scale, causal, window_left, window_right, softcap,
                                      alibi, dropout_p, dropout_seed)
    return (out, lse) if return_lse else out


def attention(q, k, v, causal=False, sm_scale=None, dropout_p=0.0, dropout_seed=None,
              seq_len_k=None, seq_len_q=None, kv_heads=None, softcap=0.0, alibi_slopes=None,
              window_left=-1, window_right=-1, use_alibi=None):
    """Flash attention forward on head-major views.

    Mirrors ``attention`` (reference attention_kernel.py:1201-1259): q, k, v
    are ``[batch, heads, seqlen, head_dim]`` with equal, 64-aligned lengths;
    ``seq_len_k``/``seq_len_q`` give the unpadded lengths (keys at or past
    ``seq_len_k`` are masked, query row ``i`` sits at position
    ``i + seq_len_k - seq_len_q``); ``kv_heads`` groups query heads.  Returns
    ``[batch, heads, seqlen, head_dim]``.
    """
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    if q.shape[2] != k.shape[2] or k.shape[2] != v.shape[2]:
        raise ValueError("The low-level attention kernel requires equal sequence lengths")
    if q.shape[2] % 64 != 0:
        raise ValueError("The low-level attention kernel requires sequence lengths divisible by 64")
    if kv_heads is None:
        kv_heads = k.shape[1]
    if q.shape[1] % kv_heads != 0:
        raise ValueError("The number of query heads must be divisible by KV heads")
    head_dim_q, head_dim_k, head_dim_v = q.shape[-1], k.shape[-1], v.shape[-1]
    assert head_dim_q == head_dim_k == head_dim_v
    assert head_dim_k in {16, 32, 64, 128, 256}
    if dropout_seed is None:
        dropout_seed = new_dropout_seed() if dropout_p > 0.0 else 0
    if alibi_slopes is None:
        use_alibi = False
    elif use_alibi is None:
        use_alibi = bool(torch.any(alibi_slopes != 0))
    if seq_len_k is None:
        seq_len_k = q.shape[2]
    if seq_len_q is None:
        seq_len_q = q.shape[2]
    alibi = None
    if use_alibi:
        alibi = alibi_slopes.reshape(-1, q.shape[1]).expand(q.shape[0], -1)
    out = dense_attention(
        q.transpose(1, 2), k.transpose(1, 2)[:, :seq_len_k], v.transpose(1, 2)[:, :seq_len_k],
        softmax_scale=sm_scale, causal=causal, q_pos_offset=seq_len_k - seq_len_q,
        window_left=window_left, window_right=window_right, softcap=softcap, alibi=alibi,
        dropout_p=dropout_p, dropout_seed=dropout_seed)
    return out.transpose(1, 2)


def attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                     causal=False, sm_scale=None, dropout_p=0.0, dropout_seed=None, softcap=0.0,
                     alibi_slopes=None, window_left=-1, window_right=-1, use_alibi=None):
    """Packed variable-length forward (reference attention_kernel.py:1364-1380)."""
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    if dropout_seed is None:
        dropout_seed = new_dropout_seed() if dropout_p > 0.0 else 0
    if alibi_slopes is None:
        use_alibi = False
    elif use_alibi is None:
        use_alibi = bool(torch.any(alibi_slopes != 0))
    return varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                            softmax_scale=sm_scale, causal=causal, window_left=window_left,
                            window_right=window_right, softcap=softcap,
                            alibi=alibi_slopes if use_alibi else None, dropout_p=dropout_p,
                            dropout_seed=dropout_seed)
