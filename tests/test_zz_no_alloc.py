"""fa_fwd_kvcache_noalloc (the entry point for callers that cannot allocate)
against fa_fwd_kvcache, through the C ABI.

Both run the same split and combine kernels; the no-alloc variant keeps the
split partials in the library's per-GPU scratch array instead of a caller
workspace, so its outputs must equal fa_fwd_kvcache's bit for bit.  Two calls
in a row, the second on a smaller input, check that the scratch array's
leftover contents from the first call do not leak into the second.  The
shapes take the split path (several key splits), once on the decode kernel
(paged cache) and once on the general KV-cache kernel (batched cache, 40 rows
per KV head).
"""
import math

import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _paged(lengths, page, hk, d, seed, cols):
    pages_per = [(L + page - 1) // page for L in lengths]
    n_pages = sum(pages_per) + 2
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(n_pages, generator=gen)
    bt = torch.zeros((len(lengths), cols), dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages_per):
        bt[b, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    kc = randn((n_pages, page, hk, d), seed + 1)
    vc = randn((n_pages, page, hk, d), seed + 2)
    return kc, vc, bt


def _both(q, kc, vc, lens, bt, max_keys, causal=False):
    from flash_attn_triton import _native
    qd, kcd, vcd, sld = (t.to(DEV) for t in (q, kc, vc, lens))
    btd = bt.to(DEV) if bt is not None else None
    B, Sq, Hq, D = q.shape
    scale = 1.0 / math.sqrt(D)
    splits, ws = _native.kvcache_plan(B, Sq, Hq, kc.shape[2], D, max_keys,
                                      kc.shape[1] if bt is not None else 0)
    assert splits > 1 and ws > 0, (splits, ws)   # the case must use the workspace
    ref = torch.full_like(qd, float("nan"))
    ref_lse = torch.full((B, Hq, Sq), float("nan"), device=DEV)
    _native.fwd_kvcache(qd, kcd, vcd, ref, ref_lse, sld, btd, None, None, max_keys, scale, causal,
                        -1, -1, None)
    got = torch.full_like(qd, float("nan"))
    got_lse = torch.full((B, Hq, Sq), float("nan"), device=DEV)
    _native.fwd_kvcache_noalloc(qd, kcd, vcd, got, got_lse, sld, btd, None, None, max_keys, scale,
                                causal, -1, -1, None)
    torch.cuda.synchronize()
    return ref.cpu(), ref_lse.cpu(), got.cpu(), got_lse.cpu()


def _check(q, kc, vc, lens, bt, max_keys, what, causal=False):
    ref, ref_lse, got, got_lse = _both(q, kc, vc, lens, bt, max_keys, causal)
    # Same kernels, same inputs: bit-exact against fa_fwd_kvcache.
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{what}: out differs"
    assert torch.equal(got_lse.view(torch.int32), ref_lse.view(torch.int32)), f"{what}: lse differs"
    # And both against the float64 oracle.
    exp, _, _, _ = ora.attention_kvcache(to_np(q), to_np(kc), to_np(vc),
                                         cache_seqlens=lens.tolist(),
                                         block_table=None if bt is None else bt.numpy(),
                                         causal=causal)
    assert_close(to_np(got), exp, ATOL[torch.float16], what, torch.float16)


def test_noalloc_paged_decode_two_calls():
    page, hq, hk, d, cols = 64, 8, 2, 128, 12
    big = [700, 1, 0, 768, 333, 64]
    kc, vc, bt = _paged(big, page, hk, d, seed=500, cols=cols)
    q = randn((len(big), 1, hq, d), 503)
    _check(q, kc, vc, torch.tensor(big, dtype=torch.int32), bt, cols * page, "paged call 1")
    # Second call: fewer sequences, shorter caches, fewer splits.
    small = [100, 250, 0]
    kc2, vc2, bt2 = _paged(small, page, hk, d, seed=600, cols=4)
    q2 = randn((len(small), 1, hq, d), 603)
    _check(q2, kc2, vc2, torch.tensor(small, dtype=torch.int32), bt2, 4 * page, "paged call 2")


def test_noalloc_batched_cache_two_calls():
    # 10 queries x GQA group 4 = 40 rows per KV head: the general KV-cache
    # kernel with split-KV partials.
    hq, hk, d, cap = 8, 2, 64, 2048
    lens = torch.tensor([2048, 1500, 40], dtype=torch.int32)
    kc = randn((3, cap, hk, d), 700)
    vc = randn((3, cap, hk, d), 701)
    q = randn((3, 10, hq, d), 702)
    _check(q, kc, vc, lens, None, cap, "batched call 1", causal=True)
    lens2 = torch.tensor([900, 10], dtype=torch.int32)
    kc2 = randn((2, 1024, hk, d), 710)
    vc2 = randn((2, 1024, hk, d), 711)
    q2 = randn((2, 10, hq, d), 712)
    _check(q2, kc2, vc2, lens2, None, 1024, "batched call 2", causal=True)


def test_noalloc_under_graph_capture_replays():
    # The entry point for code under HIP graph capture: captured once, replayed
    # with new cache lengths written into the captured length buffer (eager
    # work and a synchronization between replays); every replay equals an
    # eager fa_fwd_kvcache call on the same inputs bit for bit.
    from flash_attn_triton import _native
    page, hq, hk, d, cols = 64, 8, 2, 128, 12
    lens0 = [700, 1, 0, 768, 333, 64]
    kc, vc, bt = _paged([cols * page] * len(lens0), page, hk, d, seed=800, cols=cols)
    q = randn((len(lens0), 1, hq, d), 803).to(DEV)
    kcd, vcd, btd = kc.to(DEV), vc.to(DEV), bt.to(DEV)
    max_keys = cols * page
    scale = 1.0 / math.sqrt(d)
    lens = torch.tensor(lens0, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    lse = torch.empty((len(lens0), hq, 1), device=DEV)

    def call():
        _native.fwd_kvcache_noalloc(q, kcd, vcd, out, lse, lens, btd, None, None, max_keys,
                                    scale, False, -1, -1, None)

    call()                      # first call on the device: scratch address, kernel attributes
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    gen = torch.Generator().manual_seed(805)
    for rep in range(4):
        new = torch.randint(0, max_keys + 1, (len(lens0),), generator=gen, dtype=torch.int32)
        lens.copy_(new)
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        ref = torch.full_like(q, float("nan"))
        ref_lse = torch.empty_like(lse)
        _native.fwd_kvcache(q, kcd, vcd, ref, ref_lse, lens, btd, None, None, max_keys, scale,
                            False, -1, -1, None)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}: out"
        assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32)), f"replay {rep}: lse"


def test_noalloc_fp32_takes_no_scratch():
    # fp32 never splits a row's keys, so a shape whose 16-bit split workspace
    # would exceed the scratch array runs (and equals fa_fwd_kvcache).
    from flash_attn_triton import _native
    B, hq, hk, d, page, cols = 512, 32, 8, 128, 256, 32
    max_keys = page * cols
    _, ws = _native.kvcache_plan(B, 1, hq, hk, d, max_keys, page)
    assert ws > (16 << 20)
    gen = torch.Generator().manual_seed(900)
    lens = torch.randint(0, 2 * page + 1, (B,), generator=gen, dtype=torch.int32)
    bt = torch.randint(0, 4, (B, cols), generator=gen, dtype=torch.int32)   # 4 shared pages
    kc = randn((4, page, hk, d), 901, torch.float32).to(DEV)
    vc = randn((4, page, hk, d), 902, torch.float32).to(DEV)
    q = randn((B, 1, hq, d), 903, torch.float32).to(DEV)
    args = (lens.to(DEV), bt.to(DEV), None, None, max_keys, 1.0 / math.sqrt(d), False, -1, -1, None)
    got = torch.full_like(q, float("nan"))
    _native.fwd_kvcache_noalloc(q, kc, vc, got, None, *args)
    ref = torch.full_like(q, float("nan"))
    _native.fwd_kvcache(q, kc, vc, ref, None, *args)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
