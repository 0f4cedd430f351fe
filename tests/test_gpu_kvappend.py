"""flash_attn_with_kvcache with k/v append and rotary embedding, against the
float64 oracle (oracle/attention.py attention_kvcache, which performs the
append in place: the reference's append writes into a temporary copy and is
lost, flash_attn_interface.py:487-492).

Both the attention output and the cache contents after the call are checked:
the append must land in the caller's cache tensors, in the right slots, and
leave every other slot untouched.  Rotary tables are drawn in the input
dtype, so the reference's cast of the tables to that dtype (:56-57) is exact
and the oracle's float64 rotation is the exact answer; the kernel rotates in
fp32 and rounds once, so the cache bar is one rounding of the element type.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
CACHE_ATOL = {torch.float16: 4e-3, torch.bfloat16: 3.2e-2, torch.float32: 1e-5}
OUT_ATOL = {torch.float16: ATOL[torch.float16], torch.bfloat16: ATOL[torch.bfloat16],
            torch.float32: 5e-5}


def _tables(rows, rot, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    theta = torch.rand(rows, rot // 2, generator=gen, dtype=torch.float64) * 6.0
    return torch.cos(theta).to(dtype), torch.sin(theta).to(dtype)


def _paged(lengths, extra, page, hk, d, dtype, seed):
    pages = [(L + extra + page - 1) // page for L in lengths]
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(sum(pages) + 2, generator=gen)
    bt = torch.zeros((len(lengths), max(pages)), dtype=torch.int32)
    c = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[c:c + n]
        c += n
    kc = randn((sum(pages) + 2, page, hk, d), seed + 1, dtype)
    vc = randn((sum(pages) + 2, page, hk, d), seed + 2, dtype)
    return kc, vc, bt


def _run(q, kc, vc, dtype, causal=False, **kw):
    from flash_attn_triton import flash_attn_with_kvcache
    dev = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    out = flash_attn_with_kvcache(q.to(DEV), kcd, vcd, causal=causal, **dev)
    torch.cuda.synchronize()
    npkw = {k: (to_np(v) if isinstance(v, torch.Tensor) and v.is_floating_point()
                else (v.numpy() if isinstance(v, torch.Tensor) else v)) for k, v in kw.items()}
    ref, _, ref_kc, ref_vc = ora.attention_kvcache(
        to_np(q), to_np(kc), to_np(vc), causal=causal,
        cache_seqlens=npkw.get("cache_seqlens"), block_table=npkw.get("block_table"),
        cache_batch_idx=npkw.get("cache_batch_idx"), cache_leftpad=npkw.get("cache_leftpad"),
        k_new=npkw.get("k"), v_new=npkw.get("v"), rotary_cos=npkw.get("rotary_cos"),
        rotary_sin=npkw.get("rotary_sin"),
        rotary_interleaved=kw.get("rotary_interleaved", True))
    assert_close(to_np(out.cpu()), ref, OUT_ATOL[dtype], "out", dtype)
    assert_close(to_np(kcd.cpu()), ref_kc, CACHE_ATOL[dtype], "k_cache after append", dtype)
    assert_close(to_np(vcd.cpu()), ref_vc, 0.0, "v_cache after append", dtype)


@pytest.mark.parametrize("n_new", [1, 5])
@pytest.mark.parametrize("causal", [False, True])
def test_paged_append(n_new, causal):
    lengths = [0, 37, 255, 700]
    kc, vc, bt = _paged(lengths, n_new, 256, 2, 128, torch.float16, 40)
    q = randn((len(lengths), n_new, 8, 128), 43)
    kn = randn((len(lengths), n_new, 2, 128), 44)
    vn = randn((len(lengths), n_new, 2, 128), 45)
    _run(q, kc, vc, torch.float16, causal=causal, k=kn, v=vn,
         cache_seqlens=torch.tensor(lengths, dtype=torch.int32), block_table=bt)


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_batched_append_rotary(interleaved, dtype):
    B, cap, hq, hk, d, n = 3, 300, 4, 2, 64, 3
    kc = randn((5, cap, hk, d), 50, dtype)
    vc = randn((5, cap, hk, d), 51, dtype)
    q = randn((B, n, hq, d), 52, dtype)
    kn = randn((B, n, hk, d), 53, dtype)
    vn = randn((B, n, hk, d), 54, dtype)
    cos, sin = _tables(400, 32, dtype, 55)
    _run(q, kc, vc, dtype, causal=True, k=kn, v=vn,
         cache_seqlens=torch.tensor([0, 120, 290], dtype=torch.int32),
         cache_batch_idx=torch.tensor([4, 1, 2], dtype=torch.int32),
         cache_leftpad=torch.tensor([5, 0, 7], dtype=torch.int32),
         rotary_cos=cos, rotary_sin=sin, rotary_interleaved=interleaved)


@pytest.mark.parametrize("interleaved", [True, False])
def test_paged_append_rotary_full_dim(interleaved):
    lengths = [10, 513]
    kc, vc, bt = _paged(lengths, 4, 256, 2, 128, torch.float16, 60)
    q = randn((2, 4, 4, 128), 63)
    kn = randn((2, 4, 2, 128), 64)
    vn = randn((2, 4, 2, 128), 65)
    cos, sin = _tables(600, 128, torch.float16, 66)
    _run(q, kc, vc, torch.float16, causal=True, k=kn, v=vn,
         cache_seqlens=torch.tensor(lengths, dtype=torch.int32), block_table=bt,
         rotary_cos=cos, rotary_sin=sin, rotary_interleaved=interleaved)


def test_rotary_queries_without_append():
    # L < Sq for batch 0: its first query positions are negative and index
    # the tables from the end, as torch indexing does in the reference.
    B, cap, h, d = 2, 64, 2, 32
    kc = randn((B, cap, h, d), 70)
    vc = randn((B, cap, h, d), 71)
    q = randn((B, 6, h, d), 72)
    cos, sin = _tables(64, 16, torch.float16, 73)
    _run(q, kc, vc, torch.float16, causal=False,
         cache_seqlens=torch.tensor([3, 64], dtype=torch.int32), rotary_cos=cos, rotary_sin=sin)


def test_append_errors_follow_the_reference():
    from flash_attn_triton import flash_attn_with_kvcache
    kc = torch.zeros((2, 16, 1, 32), dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    q = torch.zeros((2, 1, 1, 32), dtype=torch.float16, device=DEV)
    kn = torch.zeros((2, 4, 1, 32), dtype=torch.float16, device=DEV)
    lens = torch.tensor([0, 13], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="supplied together"):
        flash_attn_with_kvcache(q, kc, vc, k=kn, v=None, cache_seqlens=lens)
    with pytest.raises(ValueError, match="incompatible with the cache"):
        flash_attn_with_kvcache(q, kc, vc, k=kn[:1], v=kn[:1], cache_seqlens=lens)
    with pytest.raises(ValueError, match="do not fit in the cache"):
        flash_attn_with_kvcache(q, kc, vc, k=kn, v=kn, cache_seqlens=lens)
    cos = torch.zeros((8, 8), dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="exceed the head dimension"):
        flash_attn_with_kvcache(q, kc, vc, k=kn[:, :1], v=kn[:, :1], cache_seqlens=lens,
                                rotary_cos=torch.zeros((8, 32), dtype=torch.float16, device=DEV),
                                rotary_sin=torch.zeros((8, 32), dtype=torch.float16, device=DEV))
    with pytest.raises(IndexError, match="rotary position"):
        flash_attn_with_kvcache(q, kc, vc, k=kn[:, :1], v=kn[:, :1], cache_seqlens=lens,
                                rotary_cos=cos, rotary_sin=cos)
    assert torch.all(kc == 0) and torch.all(vc == 0), "a rejected call must not touch the cache"
