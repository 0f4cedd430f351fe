"""INT8-QK^T attention forward (module path kept from the reference for drop-in imports).

Mirrors ``attention_int8`` of the reference's
``flash_attn_triton/triton_kernel/attention_kernel_int8.py:270-299``: a
per-token K quantization prepass (``fa_quant_k_int8``, bit-exact with
``_quantize_k_rows`` :58-79) followed by the attention kernel
(``fa_fwd_int8``, the role of ``_attn_fwd_int8`` :167-217) with Q quantized
per row inside the kernel, QK^T on int8 matrix cores with i32 accumulation
and PV in fp16.

The reference gates this path to Turing (compute capability 7.5,
:275-279); this build gates it to gfx950 (the only target it is compiled
for).

Backward: as the reference's ``_attention_int8.backward`` (:255-267), the
gradients come from the dense fp16 backward (``fa_bwd_dense``) on the
unquantized q, k, v with the INT8 forward's output and LSE; keys at or past
``seq_len_k`` get zero gradients.
"""
from __future__ import annotations

import math

import torch

from .. import _native
from .attention_kernel import _needs_grad, dense_backward

__all__ = ["attention_int8", "quantize_k_int8"]


def quantize_k_int8(k: torch.Tensor):
    """Quantize K ``[B, H, S, D]`` fp16 per token: returns ``(k8 [B*H,S,D] int8, s_k [B*H,S] fp32)``."""
    B, H, S, D = k.shape
    if k.stride(-1) != 1 or any(s % 8 for s in k.stride()[:3]) or k.data_ptr() % 16:
        k = k.contiguous()
    k8 = torch.empty((B * H, S, D), dtype=torch.int8, device=k.device)
    s_k = torch.empty((B * H, S), dtype=torch.float32, device=k.device)
    _native.quant_k_int8(k, k8, s_k)
    return k8, s_k


def attention_int8(q, k, v, causal=False, sm_scale=None, seq_len_k=None, seq_len_q=None):
    """INT8 flash attention forward. q, k, v: ``[B, H, S, D]`` fp16, contiguous."""
    head_dim = q.shape[-1]
    if not q.is_cuda:
        raise ValueError("The INT8 kernel requires CUDA tensors")
    arch = getattr(torch.cuda.get_device_properties(q.device), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise ValueError(
            "The INT8 kernel requires an AMD gfx950 GPU (MI355X); other GPUs have no "
            "matching INT8 matrix-core path here, use the fp16 entry point")
    if head_dim < 32 or head_dim & (head_dim - 1):
        raise ValueError("The INT8 kernel requires a power-of-two head dim of at least 32")
    if head_dim > 256:
        raise ValueError("The INT8 kernel supports head dims up to 256")
    if q.shape[2] % 64:
        raise ValueError("The INT8 kernel requires sequence lengths divisible by 64")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError(
            "The INT8 kernel requires contiguous inputs; its backward addresses "
            "K/V with Q's strides and a strided input silently gives wrong results")
    if q.shape[2] != k.shape[2] or k.shape[2] != v.shape[2]:
        raise ValueError("The INT8 kernel requires equal sequence lengths")
    if q.dtype != torch.float16 or k.dtype != torch.float16 or v.dtype != torch.float16:
        raise ValueError("The INT8 kernel takes fp16 q, k and v")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    if seq_len_k is None:
        seq_len_k = q.shape[2]
    if seq_len_q is None:
        seq_len_q = q.shape[2]
    if _needs_grad(q, k, v):
        return _Int8Attention.apply(q, k, v, causal, sm_scale, seq_len_k, seq_len_q)
    return _int8_forward(q, k, v, causal, sm_scale, seq_len_k, seq_len_q, None)


def _int8_forward(q, k, v, causal, sm_scale, seq_len_k, seq_len_q, lse):
    k8, s_k = quantize_k_int8(k)
    out = torch.empty_like(q)
    _native.fwd_int8(q, k8, s_k, v, out, lse, sm_scale, causal, seq_len_k, seq_len_q)
    return out


class _Int8Attention(torch.autograd.Function):
    """INT8 forward; fp16 dense backward (reference attention_kernel_int8.py:255-267)."""

    @staticmethod
    def forward(ctx, q, k, v, causal, sm_scale, seq_len_k, seq_len_q):
        B, H, S, _ = q.shape
        lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
        out = _int8_forward(q, k, v, causal, sm_scale, seq_len_k, seq_len_q, lse)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.opts = (causal, sm_scale, seq_len_k, seq_len_q)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        causal, sm_scale, seq_len_k, seq_len_q = ctx.opts
        lk = max(0, min(int(seq_len_k), k.shape[2]))
        if lk == 0:   # no visible key: the output is zero and so are the gradients
            return torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v), None, None, None, None
        # The INT8 kernel's query row i sits at position i + seq_len_k - seq_len_q
        # and sees keys [0, seq_len_k): the dense layout over k[:, :, :seq_len_k].
        dq, dk_used, dv_used = dense_backward(
            q.transpose(1, 2), k.transpose(1, 2)[:, :lk], v.transpose(1, 2)[:, :lk],
            out.transpose(1, 2), dout.transpose(1, 2), lse, softmax_scale=sm_scale,
            causal=bool(causal), q_pos_offset=int(seq_len_k) - int(seq_len_q))
        dk = torch.zeros_like(k)
        dv = torch.zeros_like(v)
        dk[:, :, :lk] = dk_used.transpose(1, 2)
        dv[:, :, :lk] = dv_used.transpose(1, 2)
        return dq.transpose(1, 2), dk, dv, None, None, None, None
