"""ctypes binding of ``libfa_gfx950.so`` (C ABI: ``include/fa_gfx950.h``).

The library is built in tree by ``build_native.py`` (``__graft_entry__.build()``
runs it) into ``flash_attn_triton/_lib/``.  There is no fallback: if the
library is missing or cannot be loaded every attention entry point raises.

Each wrapper takes torch tensors, passes raw device pointers, element strides
and ``torch.cuda.current_stream()``'s handle, and turns a nonzero status into
``RuntimeError`` carrying ``fa_last_error_string()``.  Launches are
asynchronous on the current stream, as the reference's Triton launches are.
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading
from pathlib import Path
from typing import Optional, Sequence

import torch

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libfa_gfx950.so"

FA_OK = 0
FA_ERR_INVALID = 1
FA_ERR_UNSUPPORTED = 2
FA_ERR_HIP = 3
FA_DTYPE_F16 = 0
FA_DTYPE_BF16 = 1
FA_DTYPE_F32 = 2

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_f32 = ctypes.c_float
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); mirrors include/fa_gfx950.h
_SIGNATURES = {
    "fa_version": (_int, []),
    "fa_last_error_string": (ctypes.c_char_p, []),
    "fa_fwd_dense": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64p, _i64p, _i64p, _i64p, _i64p, _int, _f32, _int, _i64, _i64,
                            _i64, _f32, _vp, _i64, _vp, _i64p, _f32, _u64, _vp]),
    "fa_fwd_varlen": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                             _i64, _i64p, _i64p, _i64p, _i64p, _i64p, _int, _f32, _int, _i64,
                             _i64, _f32, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                             _f32, _u64, _vp]),
    "fa_bwd_dense": (_int, [_vp] * 10 + [_i64] * 6 + [_i64p] * 9 +
                     [_int, _f32, _int, _i64, _i64, _i64, _f32, _vp, _i64, _vp, _i64p, _vp,
                      _i64p, _f32, _u64, _vp]),
    "fa_bwd_varlen": (_int, [_vp] * 12 + [_i64] * 6 + [_i64p] * 9 +
                      [_int, _f32, _int, _i64, _i64, _f32, _vp, _i64, _f32, _u64, _vp]),
    "fa_fwd_kvcache_plan": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32p, _i64p]),
    "fa_fwd_kvcache": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp,
                              _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _i64p,
                              _i64p, _int, _f32, _int, _i64, _i64, _vp, _i64, _i32, _vp, _i64,
                              _vp]),
    "fa_fwd_kvcache_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp,
                                      _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p,
                                      _i64p, _i64p, _i64p, _int, _f32, _int, _i64, _i64, _vp,
                                      _i64, _vp]),
    "fa_attn_probs": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                             _i64, _i64p, _i64p, _i64p, _int, _f32, _int, _i64, _i64, _i64,
                             _f32, _vp, _i64, _vp, _i64p, _f32, _u64, _vp]),
    "fa_kvcache_append": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp,
                                 _i64, _vp, _vp, _i64, _i64, _int, _i64, _i64, _i64, _i64,
                                 _i64p, _i64p, _i64p, _i64p, _int, _vp]),
    "fa_rotary_q": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _int, _i64, _i64, _i64,
                           _i64, _i64p, _i64p, _int, _vp]),
    "fa_check_ranges": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "fa_quant_k_int8": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64p, _vp]),
    "fa_fwd_int8": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64p, _i64p,
                           _i64p, _f32, _int, _i64, _i64, _vp]),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise ``RuntimeError`` if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"flash_attn_triton: HIP library not found at {_LIB_PATH}; build it with "
                "`python flash-attn-triton_amd/build_native.py` (or __graft_entry__.build())")
        lib = ctypes.CDLL(os.fspath(_LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def _check(status: int, what: str) -> None:
    if status != FA_OK:
        msg = load().fa_last_error_string()
        msg = msg.decode() if msg else ""
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def _strides(values: Sequence[int]):
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return FA_DTYPE_F16
    if dtype == torch.bfloat16:
        return FA_DTYPE_BF16
    if dtype == torch.float32:
        return FA_DTYPE_F32
    raise RuntimeError(f"flash_attn_triton: the HIP kernels take fp16, bf16 or fp32, not {dtype}")


def fwd_dense(q, k, v, out, lse, softmax_scale: float, causal: bool, q_pos_offset: int,
              window_left: int, window_right: int, softcap: float, alibi, bias=None,
              dropout_p: float = 0.0, dropout_seed: int = 0) -> None:
    """q [B,Sq,Hq,D], k/v [B,Sk,Hk,D] (BSHD strides), out like q; lse [B,Hq,Sq] or None;
    bias None or fp32 [B,Hq,Sq,Sk] (any strides, 0 broadcasts)."""
    lib = load()
    B, Sq, Hq, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    lse_stride = _strides(lse.stride()) if lse is not None else None
    bias_stride = _strides(bias.stride()) if bias is not None else None
    status = lib.fa_fwd_dense(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse), B, Sq, Sk, Hq, Hk, D,
        _strides(q.stride()[:3]), _strides(k.stride()[:3]), _strides(v.stride()[:3]),
        _strides(out.stride()[:3]), lse_stride, dtype_code(q.dtype), float(softmax_scale),
        int(bool(causal)), int(q_pos_offset), int(window_left), int(window_right), float(softcap),
        _ptr(alibi), 0 if alibi is None else int(alibi.stride(0)), _ptr(bias), bias_stride,
        float(dropout_p), int(dropout_seed), _stream(q.device))
    _check(status, "fa_fwd_dense")


def bwd_dense(q, k, v, out, dout, lse, dq, dk, dv, delta, softmax_scale: float, causal: bool,
              q_pos_offset: int, window_left: int, window_right: int, softcap: float,
              alibi, dropout_p: float = 0.0, dropout_seed: int = 0, bias=None,
              dbias=None) -> None:
    """Gradients of fwd_dense: all tensors BSHD ([B,S,H,D]); lse / delta fp32
    [B,Hq,Sq]; dq/dk/dv are written.  bias / dbias None or fp32 [B,Hq,Sq,Sk]
    views (stride 0 on broadcast dims); dbias must hold zeros and receives the
    bias gradient.  See fa_bwd_dense."""
    lib = load()
    B, Sq, Hq, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    st = [_strides(t.stride()[:3]) for t in (q, k, v, out, dout, dq, dk, dv)]
    status = lib.fa_bwd_dense(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(dq), _ptr(dk),
        _ptr(dv), _ptr(delta), B, Sq, Sk, Hq, Hk, D, *st, _strides(lse.stride()),
        dtype_code(q.dtype), float(softmax_scale), int(bool(causal)), int(q_pos_offset),
        int(window_left), int(window_right), float(softcap), _ptr(alibi),
        0 if alibi is None else int(alibi.stride(0)), _ptr(bias),
        None if bias is None else _strides(bias.stride()), _ptr(dbias),
        None if dbias is None else _strides(dbias.stride()), float(dropout_p),
        int(dropout_seed), _stream(q.device))
    _check(status, "fa_bwd_dense")


def bwd_varlen(q, k, v, out, dout, lse, dq, dk, dv, delta, cu_q, cu_k, max_seqlen_q: int,
               max_seqlen_k: int, softmax_scale: float, causal: bool, window_left: int,
               window_right: int, softcap: float, alibi, dropout_p: float = 0.0,
               dropout_seed: int = 0) -> None:
    """Gradients of fwd_varlen: packed [T,H,D] tensors, lse / delta fp32 [Tq,Hq],
    cu_* int32 [batch+1].  See fa_bwd_varlen."""
    lib = load()
    Hq, D = q.shape[1], q.shape[2]
    Hk = k.shape[1]
    st = [_strides(t.stride()[:2]) for t in (q, k, v, out, dout, dq, dk, dv)]
    status = lib.fa_bwd_varlen(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(dq), _ptr(dk),
        _ptr(dv), _ptr(delta), _ptr(cu_q), _ptr(cu_k), cu_q.numel() - 1, int(max_seqlen_q),
        int(max_seqlen_k), Hq, Hk, D, *st, _strides(lse.stride()), dtype_code(q.dtype),
        float(softmax_scale), int(bool(causal)), int(window_left), int(window_right),
        float(softcap), _ptr(alibi), 0 if alibi is None else int(alibi.stride(0)),
        float(dropout_p), int(dropout_seed), _stream(q.device))
    _check(status, "fa_bwd_varlen")


def attn_probs(q, k, lse, probs, lse_out, cu_q, cu_k, max_seqlen_q: int, max_seqlen_k: int,
               softmax_scale: float, causal: bool, q_pos_offset: int, window_left: int,
               window_right: int, softcap: float, alibi, bias=None, dropout_p: float = 0.0,
               dropout_seed: int = 0) -> None:
    """probs fp32 [B,Hq,max_q,max_k] contiguous from q/k and the forward LSE.

    Dense (cu_q None): q [B,Sq,Hq,D], k [B,Sk,Hk,D], lse [B,Hq,Sq].  Varlen: q
    [Tq,Hq,D], k [Tk,Hk,D], lse [Tq,Hq], cu_* int32 [B+1]; lse_out (or None)
    gets [B,Hq,max_q] with -inf padding.
    """
    lib = load()
    if cu_q is None:
        B, Hq, D = q.shape[0], q.shape[2], q.shape[3]
        Hk = k.shape[2]
        q_stride, k_stride = q.stride()[:3], k.stride()[:3]
        ls = lse.stride()
        lse_stride = (ls[0], ls[2], ls[1])
    else:
        B, Hq, D = cu_q.numel() - 1, q.shape[1], q.shape[2]
        Hk = k.shape[1]
        q_stride, k_stride = (0,) + tuple(q.stride()[:2]), (0,) + tuple(k.stride()[:2])
        lse_stride = (0,) + tuple(lse.stride())
    bias_stride = _strides(bias.stride()) if bias is not None else None
    status = lib.fa_attn_probs(
        _ptr(q), _ptr(k), _ptr(lse), _ptr(probs), _ptr(lse_out), _ptr(cu_q), _ptr(cu_k), B,
        int(max_seqlen_q), int(max_seqlen_k), Hq, Hk, D, _strides(q_stride), _strides(k_stride),
        _strides(lse_stride), dtype_code(q.dtype), float(softmax_scale), int(bool(causal)),
        int(q_pos_offset), int(window_left), int(window_right), float(softcap), _ptr(alibi),
        0 if alibi is None else int(alibi.stride(0)), _ptr(bias), bias_stride,
        float(dropout_p), int(dropout_seed), _stream(q.device))
    _check(status, "fa_attn_probs")


def fwd_varlen(q, k, v, out, lse, cu_q, cu_k, max_seqlen_q: int, max_seqlen_k: int,
               softmax_scale: float, causal: bool, window_left: int, window_right: int,
               softcap: float, alibi, seqused_q=None, seqused_k=None, cu_out=None,
               block_table=None, dropout_p: float = 0.0, dropout_seed: int = 0) -> None:
    """q [Tq,Hq,D], k/v [Tk,Hk,D] (or paged [pages,page,Hk,D] with block_table);
    cu_* int32 [batch+1]; lse [Tout,Hq] or None; see fa_fwd_varlen."""
    lib = load()
    Hq, D = q.shape[1], q.shape[2]
    paged = block_table is not None
    Hk = k.shape[2] if paged else k.shape[1]
    nkv = 3 if paged else 2
    batch = cu_q.numel() - 1
    lse_stride = _strides(lse.stride()) if lse is not None else None
    status = lib.fa_fwd_varlen(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse), _ptr(cu_q), _ptr(cu_k), batch,
        int(max_seqlen_q), int(max_seqlen_k), Hq, Hk, D, _strides(q.stride()[:2]),
        _strides(k.stride()[:nkv]), _strides(v.stride()[:nkv]), _strides(out.stride()[:2]),
        lse_stride, dtype_code(q.dtype), float(softmax_scale), int(bool(causal)),
        int(window_left), int(window_right), float(softcap), _ptr(alibi),
        0 if alibi is None else int(alibi.stride(0)), _ptr(seqused_q), _ptr(seqused_k),
        _ptr(cu_out), _ptr(block_table), int(block_table.stride(0)) if paged else 0,
        int(k.shape[1]) if paged else 0, int(k.shape[0]) if paged else 0,
        int(block_table.shape[1]) if paged else 0, float(dropout_p), int(dropout_seed),
        _stream(q.device))
    _check(status, "fa_fwd_varlen")


@functools.lru_cache(maxsize=1024)
def kvcache_plan(batch: int, seqlen_q: int, heads_q: int, heads_k: int, head_dim: int,
                 max_keys: int, page_size: int = 0):
    lib = load()
    splits = ctypes.c_int32(0)
    ws = ctypes.c_int64(0)
    _check(lib.fa_fwd_kvcache_plan(batch, seqlen_q, heads_q, heads_k, head_dim, max_keys,
                                   page_size, ctypes.byref(splits), ctypes.byref(ws)),
           "fa_fwd_kvcache_plan")
    return int(splits.value), int(ws.value)


def fwd_kvcache(q, k_cache, v_cache, out, lse, cache_seqlens, block_table, cache_batch_idx,
                cache_leftpad, max_keys: int, softmax_scale: float, causal: bool,
                window_left: int, window_right: int, alibi, workspace=None) -> None:
    """Attention of q [B,Sq,Hq,D] against a paged or batched cache (see fa_fwd_kvcache)."""
    lib = load()
    B, Sq, Hq, D = q.shape
    Hk = k_cache.shape[2]
    page_size = k_cache.shape[1] if block_table is not None else 0
    splits, ws_bytes = kvcache_plan(B, Sq, Hq, Hk, D, max_keys, page_size)
    if ws_bytes > 0 and (workspace is None or workspace.numel() < ws_bytes):
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    bt_stride = block_table.stride(0) if block_table is not None else 0
    lse_stride = _strides(lse.stride()) if lse is not None else None
    status = lib.fa_fwd_kvcache(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(lse), _ptr(cache_seqlens),
        _ptr(block_table), int(bt_stride), int(page_size), int(k_cache.shape[0]),
        _ptr(cache_batch_idx),
        _ptr(cache_leftpad), B, Sq, int(max_keys), Hq, Hk, D, _strides(q.stride()[:3]),
        _strides(k_cache.stride()[:3]), _strides(v_cache.stride()[:3]),
        _strides(out.stride()[:3]), lse_stride, dtype_code(q.dtype), float(softmax_scale),
        int(bool(causal)), int(window_left), int(window_right), _ptr(alibi),
        0 if alibi is None else int(alibi.stride(0)), splits, _ptr(workspace),
        int(ws_bytes), _stream(q.device))
    _check(status, "fa_fwd_kvcache")


def fwd_kvcache_noalloc(q, k_cache, v_cache, out, lse, cache_seqlens, block_table,
                        cache_batch_idx, cache_leftpad, max_keys: int, softmax_scale: float,
                        causal: bool, window_left: int, window_right: int, alibi) -> None:
    """fwd_kvcache through fa_fwd_kvcache_noalloc: the split partials live in
    the library's per-GPU scratch array, so this call allocates nothing on the
    device (calls that overlap on one GPU race; see the header)."""
    lib = load()
    B, Sq, Hq, D = q.shape
    Hk = k_cache.shape[2]
    page_size = k_cache.shape[1] if block_table is not None else 0
    bt_stride = block_table.stride(0) if block_table is not None else 0
    lse_stride = _strides(lse.stride()) if lse is not None else None
    status = lib.fa_fwd_kvcache_noalloc(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(lse), _ptr(cache_seqlens),
        _ptr(block_table), int(bt_stride), int(page_size), int(k_cache.shape[0]),
        _ptr(cache_batch_idx), _ptr(cache_leftpad), B, Sq, int(max_keys), Hq, Hk, D,
        _strides(q.stride()[:3]), _strides(k_cache.stride()[:3]),
        _strides(v_cache.stride()[:3]), _strides(out.stride()[:3]), lse_stride,
        dtype_code(q.dtype), float(softmax_scale), int(bool(causal)), int(window_left),
        int(window_right), _ptr(alibi), 0 if alibi is None else int(alibi.stride(0)),
        _stream(q.device))
    _check(status, "fa_fwd_kvcache_noalloc")


def kvcache_append(k_new, v_new, k_cache, v_cache, cache_seqlens, block_table, cache_batch_idx,
                   cache_leftpad, capacity: int, rotary_cos, rotary_sin,
                   rotary_interleaved: bool) -> None:
    """Write k_new / v_new [B, n, Hk, D] into the cache in place (see fa_kvcache_append)."""
    lib = load()
    B, n, Hk, D = k_new.shape
    paged = block_table is not None
    rot = 2 * rotary_cos.shape[-1] if rotary_cos is not None else 0
    status = lib.fa_kvcache_append(
        _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(cache_seqlens),
        _ptr(block_table), int(block_table.stride(0)) if paged else 0,
        int(k_cache.shape[1]) if paged else 0, int(k_cache.shape[0]) if paged else 0,
        _ptr(cache_batch_idx), 0 if paged else int(k_cache.shape[0]), _ptr(cache_leftpad),
        int(capacity), _ptr(rotary_cos), _ptr(rotary_sin), rot,
        int(rotary_cos.shape[0]) if rotary_cos is not None else 0, int(bool(rotary_interleaved)),
        B, n, Hk, D, _strides(k_new.stride()[:3]), _strides(v_new.stride()[:3]),
        _strides(k_cache.stride()[:3]), _strides(v_cache.stride()[:3]), dtype_code(k_new.dtype),
        _stream(k_new.device))
    _check(status, "fa_kvcache_append")


def rotary_q(q, out, cache_seqlens, cache_leftpad, rotary_cos, rotary_sin,
             rotary_interleaved: bool) -> None:
    """out = q rotated at positions cache_seqlens[b] - Sq + leftpad[b] + i (see fa_rotary_q)."""
    lib = load()
    B, Sq, H, D = q.shape
    status = lib.fa_rotary_q(
        _ptr(q), _ptr(out), _ptr(cache_seqlens), _ptr(cache_leftpad), _ptr(rotary_cos),
        _ptr(rotary_sin), 2 * rotary_cos.shape[-1], int(rotary_cos.shape[0]),
        int(bool(rotary_interleaved)), B, Sq, H, D, _strides(q.stride()[:3]),
        _strides(out.stride()[:3]), dtype_code(q.dtype), _stream(q.device))
    _check(status, "fa_rotary_q")


MAX_RANGE_CHECKS = 8


def check_ranges(arrays, minmax, diff=None) -> None:
    """min / max of each ``a`` (+ ``b``) of ``arrays`` = [(a, b or None), ...]
    (contiguous int32 / int64 device tensors, at most MAX_RANGE_CHECKS) into
    ``minmax`` (int64, 2 per array: pinned host or device memory), in one
    launch on the current stream (fa_check_ranges).  ``diff[i]`` true: the
    adjacent differences of ``a`` instead (``b`` must be None)."""
    lib = load()
    n = len(arrays)
    diff = list(diff) if diff is not None else [False] * n
    for (a, b), d in zip(arrays, diff):
        assert a.is_contiguous() and a.dtype in (torch.int32, torch.int64)
        assert b is None or (b.is_contiguous() and b.dtype in (torch.int32, torch.int64)
                             and b.numel() == a.numel() and not d)
    assert minmax.dtype == torch.int64 and minmax.numel() >= 2 * n
    ptr_a = (ctypes.c_void_p * n)(*[a.data_ptr() for a, _ in arrays])
    bytes_a = (ctypes.c_int * n)(*[a.element_size() for a, _ in arrays])
    ptr_b = (ctypes.c_void_p * n)(*[None if b is None else b.data_ptr() for _, b in arrays])
    bytes_b = (ctypes.c_int * n)(*[4 if b is None else b.element_size() for _, b in arrays])
    numel = (ctypes.c_int64 * n)(*[a.numel() for a, _ in arrays])
    diffs = (ctypes.c_int * n)(*[1 if d else 0 for d in diff])
    device = arrays[0][0].device
    status = lib.fa_check_ranges(n, ptr_a, bytes_a, ptr_b, bytes_b, diffs, numel,
                                 ctypes.c_void_p(minmax.data_ptr()), _stream(device))
    _check(status, "fa_check_ranges")


def quant_k_int8(k, k8, s_k) -> None:
    """k [B,H,S,D] fp16 -> k8 [B*H,S,D] int8, s_k [B*H,S] fp32."""
    lib = load()
    B, H, S, D = k.shape
    st = k.stride()
    status = lib.fa_quant_k_int8(_ptr(k), _ptr(k8), _ptr(s_k), B, H, S, D,
                                 _strides((st[0], st[1], st[2])), _stream(k.device))
    _check(status, "fa_quant_k_int8")


def fwd_int8(q, k8, s_k, v, out, lse, sm_scale: float, causal: bool, seq_len_k: int,
             seq_len_q: int) -> None:
    """q/v/out [B,H,S,D] fp16 with {batch, head, seq} strides; lse [B,H,S] or None."""
    lib = load()
    B, H, S, D = q.shape
    status = lib.fa_fwd_int8(
        _ptr(q), _ptr(k8), _ptr(s_k), _ptr(v), _ptr(out), _ptr(lse), B, H, S, D,
        _strides(q.stride()[:3]), _strides(v.stride()[:3]), _strides(out.stride()[:3]),
        float(sm_scale), int(bool(causal)), int(seq_len_k), int(seq_len_q), _stream(q.device))
    _check(status, "fa_fwd_int8")
