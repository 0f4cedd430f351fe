"""The decode call's argument checks on the GPU (fa_check_ranges).

A plain decode call (no append, rotary or ALiBi) launches before it waits
for its checks: the range checks of the block table, cache_seqlens,
cache_batch_idx and cache_leftpad reduce in one fa_check_ranges launch on a
second stream into pinned host memory, and the reference's ValueError is
raised after the launch (flash_attn_interface.py:428-453).  The kernels
clamp cache lengths and left pads to the cache, so the failing cases here
feed only out-of-range lengths / pads (never page indices or cache rows
outside the cache).
"""
import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, randn, to_np
from oracle import attention as ora
from flash_attn_triton import _native

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.mark.parametrize("wide", [False, True])
def test_check_ranges_kernel_min_max(wide):
    # Direct C-ABI call: min / max of arrays with and without an addend, of
    # both element widths, sizes around the workgroup width, into pinned
    # host memory and into device memory.
    gen = torch.Generator().manual_seed(3)
    dt = torch.int64 if wide else torch.int32
    arrays = []
    for n in (1, 255, 256, 257, 5000):
        a = torch.randint(-(1 << 30), 1 << 30, (n,), generator=gen, dtype=torch.int64).to(dt)
        b = torch.randint(-1000, 1000, (n,), generator=gen, dtype=torch.int64)
        arrays.append((a, b if n % 2 else None))
    expect = []
    for a, b in arrays:
        s = a.long() + (b if b is not None else 0)
        expect += [int(s.min()), int(s.max())]
    dev = [(a.to(DEV), None if b is None else b.to(DEV)) for a, b in arrays]
    host = torch.empty(2 * len(dev), dtype=torch.int64, pin_memory=True)
    _native.check_ranges(dev, host)
    torch.cuda.synchronize()
    assert host.tolist() == expect
    on_dev = torch.empty(2 * len(dev), dtype=torch.int64, device=DEV)
    _native.check_ranges(dev, on_dev)
    assert on_dev.cpu().tolist() == expect


def test_check_ranges_adjacent_differences():
    # The monotonicity form: min / max of a[j+1] - a[j], for both widths.
    gen = torch.Generator().manual_seed(4)
    for dt in (torch.int32, torch.int64):
        for n in (2, 257, 3000):
            a = torch.randint(-1000, 1000, (n,), generator=gen, dtype=torch.int64).cumsum(0).to(dt)
            d = a[1:].long() - a[:-1].long()
            host = torch.empty(4, dtype=torch.int64, pin_memory=True)
            _native.check_ranges([(a.to(DEV), None), (a.to(DEV), None)], host, diff=[True, False])
            torch.cuda.synchronize()
            assert host.tolist() == [int(d.min()), int(d.max()), int(a.min()), int(a.max())]


def test_check_ranges_rejects_pageable_host_memory():
    a = torch.arange(10, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="pinned host memory"):
        _native.check_ranges([(a, None)], torch.empty(2, dtype=torch.int64))


def _paged(lengths, page, hk, d, seed):
    pages_per = [(L + page - 1) // page for L in lengths]
    n_pages = sum(pages_per)
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(n_pages, generator=gen)
    bt = torch.zeros((len(lengths), max(pages_per)), dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages_per):
        bt[b, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    return randn((n_pages, page, hk, d), seed + 1), randn((n_pages, page, hk, d), seed + 2), bt


@pytest.mark.parametrize("seqlens_dtype", [torch.int32, torch.int64])
def test_decode_checks_pass_at_the_edges(seqlens_dtype):
    # Lengths at the block table's capacity and page indices up to the last
    # page: the checks pass and the result matches the oracle.
    from flash_attn_triton import flash_attn_with_kvcache
    page, hq, hk, d = 64, 8, 2, 128
    lengths = [256, 64, 1, 200]
    kc, vc, bt = _paged(lengths, page, hk, d, 70)
    q = randn((4, 1, hq, d), 73)
    out = flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV),
                                  cache_seqlens=torch.tensor(lengths, dtype=seqlens_dtype).to(DEV),
                                  block_table=bt.to(DEV))
    ref, _, _, _ = ora.attention_kvcache(to_np(q), to_np(kc), to_np(vc),
                                         cache_seqlens=np.array(lengths),
                                         block_table=bt.numpy(), causal=False)
    assert_close(to_np(out.cpu()), ref, ATOL[torch.float16], "decode at capacity",
                 torch.float16)


@pytest.mark.parametrize("seqlens_dtype", [torch.int32, torch.int64])
def test_decode_rejects_lengths_beyond_the_cache(seqlens_dtype):
    from flash_attn_triton import flash_attn_with_kvcache
    page, hq, hk, d = 64, 8, 2, 128
    lengths = [256, 64, 1, 200]
    kc, vc, bt = _paged(lengths, page, hk, d, 80)
    q = randn((4, 1, hq, d), 83).to(DEV)
    for bad in ([256, 64, 257, 200], [256, -1, 1, 200]):
        with pytest.raises(ValueError, match="valid lengths"):
            flash_attn_with_kvcache(q, kc.to(DEV), vc.to(DEV),
                                    cache_seqlens=torch.tensor(bad, dtype=seqlens_dtype).to(DEV),
                                    block_table=bt.to(DEV))
    # A later good call on the same stream still works.
    out = flash_attn_with_kvcache(q, kc.to(DEV), vc.to(DEV),
                                  cache_seqlens=torch.tensor(lengths, dtype=seqlens_dtype).to(DEV),
                                  block_table=bt.to(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


def test_batched_decode_checks_length_plus_leftpad():
    # Batched cache with cache_leftpad: lengths + left pads must fit the
    # capacity (the check's addend form, no temporary sum tensor).
    from flash_attn_triton import flash_attn_with_kvcache
    B, cap, hq, hk, d = 3, 128, 4, 4, 64
    kc = randn((B, cap, hk, d), 91).to(DEV)
    vc = randn((B, cap, hk, d), 92).to(DEV)
    q = randn((B, 1, hq, d), 93)
    pads = torch.tensor([0, 28, 100], dtype=torch.int32)
    good = torch.tensor([128, 100, 28], dtype=torch.int32)
    out = flash_attn_with_kvcache(q.to(DEV), kc, vc, cache_seqlens=good.to(DEV),
                                  cache_leftpad=pads.to(DEV))
    ref, _, _, _ = ora.attention_kvcache(to_np(q), to_np(kc.cpu()), to_np(vc.cpu()),
                                         cache_seqlens=good.numpy(), cache_leftpad=pads.numpy(),
                                         causal=False)
    assert_close(to_np(out.cpu()), ref, ATOL[torch.float16], "batched leftpad", torch.float16)
    with pytest.raises(ValueError, match="valid lengths"):
        flash_attn_with_kvcache(q.to(DEV), kc, vc, cache_seqlens=(good + 1).to(DEV),
                                cache_leftpad=pads.to(DEV))


def test_varlen_checks_on_device_cu_seqlens():
    # The varlen call's range checks (start, order, sizes, cover, max lengths)
    # reduce in one launch; each failing case raises the reference's error
    # before anything is launched.
    from flash_attn_triton import flash_attn_varlen_func
    H, D = 4, 64
    lens = [5, 0, 70, 33]
    T = sum(lens)
    q, k, v = (randn((T, H, D), s).to(DEV) for s in (30, 31, 32))
    cu = torch.tensor([0, 5, 5, 75, 108], dtype=torch.int32, device=DEV)
    out = flash_attn_varlen_func(q, k, v, cu, cu, 70, 70, causal=True)
    ref, _ = ora.attention_varlen(to_np(q.cpu()), to_np(k.cpu()), to_np(v.cpu()), cu.cpu().numpy(),
                                  cu.cpu().numpy(), 1.0 / np.sqrt(D), True, (-1, -1), 0.0, None)
    assert_close(to_np(out.cpu()), ref, ATOL[torch.float16], "varlen", torch.float16)
    bad_order = torch.tensor([0, 5, 4, 75, 108], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="monotonically"):
        flash_attn_varlen_func(q, k, v, bad_order, cu, 70, 70)
    with pytest.raises(ValueError, match="start at zero"):
        flash_attn_varlen_func(q, k, v, cu + 1, cu, 70, 70)
    with pytest.raises(ValueError, match="exceed"):
        flash_attn_varlen_func(q, k, v, cu, torch.tensor([0, 5, 5, 75, 109], dtype=torch.int32,
                                                         device=DEV), 70, 70)
    with pytest.raises(ValueError, match="max sequence lengths must cover"):
        flash_attn_varlen_func(q, k, v, cu, cu, 69, 70)


def test_varlen_zero_alibi_slopes_take_the_plain_path():
    # All-+0.0 slopes (min and max of their bit patterns both 0) drop ALiBi;
    # -0.0 keeps the ALiBi path, whose zero slopes give the same attention.
    from flash_attn_triton import flash_attn_varlen_func
    H, D = 4, 64
    lens = [40, 90]
    T = sum(lens)
    q, k, v = (randn((T, H, D), s).to(DEV) for s in (40, 41, 42))
    cu = torch.tensor([0, 40, 130], dtype=torch.int32, device=DEV)
    plain = flash_attn_varlen_func(q, k, v, cu, cu, 90, 90, causal=True)
    zero = flash_attn_varlen_func(q, k, v, cu, cu, 90, 90, causal=True,
                                  alibi_slopes=torch.zeros(H, device=DEV))
    neg0 = flash_attn_varlen_func(q, k, v, cu, cu, 90, 90, causal=True,
                                  alibi_slopes=torch.full((H,), -0.0, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(zero.view(torch.int16), plain.view(torch.int16))
    assert (neg0.float() - plain.float()).abs().max().item() < 2e-3
