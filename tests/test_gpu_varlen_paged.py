"""flash_attn_varlen_func with seqused_q / seqused_k and with a paged K/V
cache (block_table), against the float64 oracle applied to the reference's
own rewrite of those inputs (oracle/attention.py compact_varlen, following
flash_attn_interface.py:533-581): the kernels read the used counts and the
page table directly, the oracle gathers and compacts first, and the answers
must agree row for row, including the packed output layout.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float16: ATOL[torch.float16], torch.bfloat16: ATOL[torch.bfloat16],
       torch.float32: 5e-5}


def _cu(lengths):
    return torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)


def _pages(lengths, page, hk, d, seed, dtype):
    """A shuffled paged cache: sequence b owns ceil(len/page) pages, two spare
    pages hold noise, and the table's unused columns point nowhere valid."""
    gen = torch.Generator().manual_seed(seed)
    counts = [(L + page - 1) // page for L in lengths]
    n_pages = sum(counts) + 2
    perm = torch.randperm(n_pages, generator=gen)
    bt = torch.full((len(lengths), max(max(counts), 1) + 1), 1 << 20, dtype=torch.int32)
    c = 0
    for b, n in enumerate(counts):
        bt[b, :n] = perm[c:c + n]
        c += n
    kc = randn((n_pages, page, hk, d), seed + 1, dtype)
    vc = randn((n_pages, page, hk, d), seed + 2, dtype)
    return kc, vc, bt


def _case(lq, lk, *, hq=4, hk=2, d=64, dtype=torch.float16, seed=0, used_q=None,
          used_k=None, page=None, causal=False, probs=False, **kw):
    from flash_attn_triton import flash_attn_varlen_func
    cu_q, cu_k = _cu(lq), _cu(lk)
    q = randn((int(sum(lq)), hq, d), seed + 10, dtype)
    if page is None:
        k = randn((int(sum(lk)), hk, d), seed + 11, dtype)
        v = randn((int(sum(lk)), hk, d), seed + 12, dtype)
        bt = None
    else:
        k, v, bt = _pages(lk, page, hk, d, seed + 13, dtype)
    uq = None if used_q is None else torch.tensor(used_q, dtype=torch.int32)
    uk = None if used_k is None else torch.tensor(used_k, dtype=torch.int32)
    mq = max(used_q) if used_q is not None else max(lq)
    mk = max(used_k) if used_k is not None else max(lk)
    dev = lambda t: None if t is None else t.to(DEV)
    res = flash_attn_varlen_func(dev(q), dev(k), dev(v), dev(cu_q), dev(cu_k), mq, mk,
                                 causal=causal, block_table=dev(bt), seqused_q=dev(uq),
                                 seqused_k=dev(uk), return_attn_probs=probs, **kw)
    torch.cuda.synchronize()
    cq, ck_, ckv, cu_q2, cu_k2 = ora.compact_varlen(
        to_np(q), to_np(k), to_np(v), cu_q.numpy(), cu_k.numpy(),
        used_q, used_k, None if bt is None else bt.numpy())
    ref, ref_lse = ora.attention_varlen(cq, ck_, ckv, cu_q2, cu_k2, kw.get("softmax_scale"),
                                        causal, kw.get("window_size", (-1, -1)),
                                        kw.get("softcap", 0.0))
    out = res[0] if probs else res
    assert out.shape == (ref.shape[0], hq, d), (tuple(out.shape), ref.shape)
    assert_close(to_np(out.cpu()), ref, TOL[dtype], "out", dtype)
    if probs:
        lses = res[1].cpu().numpy()
        for b in range(len(lq)):
            n = int(cu_q2[b + 1] - cu_q2[b])
            assert_close(lses[b, :, :n], ref_lse[cu_q2[b]:cu_q2[b + 1]].T, 1e-3, "lse")
    return out


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_seqused_q_and_k(causal, d):
    lq, lk = [70, 300, 5, 257], [90, 300, 64, 260]
    _case(lq, lk, d=d, causal=causal, used_q=[33, 300, 0, 129], used_k=[90, 17, 64, 200],
          seed=1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_seqused_k_only(dtype):
    lq = lk = [130, 64, 400]
    _case(lq, lk, d=128, dtype=dtype, causal=True, used_k=[1, 64, 333], seed=2)


def test_seqused_q_only_output_is_packed():
    lq, lk = [10, 20, 30], [10, 20, 30]
    out = _case(lq, lk, d=32, used_q=[3, 0, 30], seed=3)
    assert out.shape[0] == 33


@pytest.mark.parametrize("page", [16, 64, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_paged_varlen(page, causal):
    lq, lk = [5, 200, 64, 1], [37, 513, 64, 300]
    _case(lq, lk, hq=8, hk=2, d=128, page=page, causal=causal, seed=4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_varlen_dtypes(dtype):
    _case([100, 3], [129, 700], hq=4, hk=4, d=64, page=32, dtype=dtype, causal=True, seed=5)


def test_paged_varlen_with_seqused_and_features():
    _case([40, 300, 2], [60, 500, 33], hq=8, hk=2, d=128, page=64, causal=True,
          used_q=[40, 256, 1], used_k=[60, 301, 0], window_size=(96, 0), softcap=20.0,
          softmax_scale=0.07, seed=6)


def test_paged_varlen_head_dims():
    for d in (16, 32, 256):
        _case([33, 70], [50, 90], hq=2, hk=1, d=d, page=16, causal=True, seed=7 + d)


def test_seqused_and_paged_with_probs():
    _case([12, 40], [20, 48], hq=2, hk=2, d=64, page=16, used_q=[5, 40], used_k=[20, 31],
          causal=True, probs=True, seed=8)


def test_errors_follow_the_reference():
    from flash_attn_triton import flash_attn_varlen_func
    q = torch.zeros((10, 2, 32), dtype=torch.float16, device=DEV)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="one value per sequence"):
        flash_attn_varlen_func(q, q, q, cu, cu, 6, 6, seqused_q=torch.tensor([1], device=DEV))
    with pytest.raises(ValueError, match="exceeds the packed query sequence"):
        flash_attn_varlen_func(q, q, q, cu, cu, 6, 6,
                               seqused_q=torch.tensor([5, 1], device=DEV))
    with pytest.raises(ValueError, match="exceeds the packed KV sequence"):
        flash_attn_varlen_func(q, q, q, cu, cu, 6, 6,
                               seqused_k=torch.tensor([1, -1], device=DEV))
    kc = torch.zeros((3, 4, 2, 32), dtype=torch.float16, device=DEV)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="invalid physical page index"):
        flash_attn_varlen_func(q, kc, kc, cu, cu, 6, 6, block_table=bt)
    bt_ok = torch.tensor([[0, 9], [1, 2]], dtype=torch.int32, device=DEV)   # col 1 of row 0 unused
    out = flash_attn_varlen_func(q, kc, kc, cu, cu, 6, 6, block_table=bt_ok)
    assert out.shape == q.shape
    with pytest.raises(ValueError, match="exceed the packed tensor sizes"):
        flash_attn_varlen_func(q, kc, kc, cu, torch.tensor([0, 4, 13], dtype=torch.int32,
                                                           device=DEV), 6, 9, block_table=bt_ok)
    with pytest.raises(ValueError, match=r"shape \(batch, max_num_pages\)"):
        flash_attn_varlen_func(q, kc, kc, cu, cu, 6, 6, block_table=bt_ok[:1])


def _grad_case(lq, lk, *, hq=4, hk=2, d=64, dtype=torch.float16, seed=0, used_q=None,
               used_k=None, page=None, causal=False, **kw):
    """Gradients through seqused_* and the block table: the reference gathers
    the used rows / pages with torch indexing and differentiates through it
    (flash_attn_interface.py:533-581), so the exact gradient is the packed
    sequences' gradient scattered back to the rows (and cache slots) it came
    from, every other row zero.  The row map comes from the oracle's own
    compaction applied to row indices."""
    from flash_attn_triton import flash_attn_varlen_func
    cu_q, cu_k = _cu(lq), _cu(lk)
    q = randn((int(sum(lq)), hq, d), seed + 10, dtype)
    if page is None:
        k = randn((int(sum(lk)), hk, d), seed + 11, dtype)
        v = randn((int(sum(lk)), hk, d), seed + 12, dtype)
        bt = None
    else:
        k, v, bt = _pages(lk, page, hk, d, seed + 13, dtype)
    uq = None if used_q is None else torch.tensor(used_q, dtype=torch.int32)
    uk = None if used_k is None else torch.tensor(used_k, dtype=torch.int32)
    mq = max(used_q) if used_q is not None else max(lq)
    mk = max(used_k) if used_k is not None else max(lk)
    rows_out = int(sum(used_q)) if used_q is not None else int(sum(lq))
    do = randn((rows_out, hq, d), seed + 14, dtype)
    dev = lambda t: None if t is None else t.to(DEV)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = flash_attn_varlen_func(qd, kd, vd, dev(cu_q), dev(cu_k), mq, mk, causal=causal,
                                 block_table=dev(bt), seqused_q=dev(uq), seqused_k=dev(uk), **kw)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    bt_np = None if bt is None else bt.numpy()
    cq, ck_, ckv, cu_q2, cu_k2 = ora.compact_varlen(to_np(q), to_np(k), to_np(v), cu_q.numpy(),
                                                    cu_k.numpy(), used_q, used_k, bt_np)
    qrow = np.arange(q.shape[0]).reshape(-1, 1, 1)
    krow = np.arange(int(np.prod(k.shape[:-2]))).reshape(*k.shape[:-2], 1, 1)
    qmap, kmap, _, _, _ = ora.compact_varlen(qrow, krow, krow, cu_q.numpy(), cu_k.numpy(),
                                             used_q, used_k, bt_np)
    grads = ora.attention_varlen_backward(cq, ck_, ckv, to_np(do), cu_q2, cu_k2,
                                          kw.get("softmax_scale"), causal,
                                          kw.get("window_size", (-1, -1)), kw.get("softcap", 0.0))
    for name, t, g, rmap in (("dq", qd, grads[0], qmap), ("dk", kd, grads[1], kmap),
                             ("dv", vd, grads[2], kmap)):
        exact = np.zeros((int(np.prod(t.shape[:-2])),) + tuple(t.shape[-2:]))
        exact[rmap[:, 0, 0]] = g
        got = to_np(t.grad.cpu()).reshape(exact.shape)
        err = np.abs(got - exact)
        atol, rtol = (5e-3, 1e-2) if dtype == torch.float16 else (4e-2, 4e-2)
        print(f"{name}: max-abs err {float(np.max(err)):.3e}")
        assert np.all(np.isfinite(got)) and np.all(err <= atol + rtol * np.abs(exact)), (
            f"{name}: max |err| {float(np.max(err)):.3e}")


@pytest.mark.parametrize("causal", [False, True])
def test_seqused_gradients(causal):
    _grad_case([70, 300, 5, 257], [90, 300, 64, 260], d=64, causal=causal,
               used_q=[33, 300, 0, 129], used_k=[90, 17, 64, 200], seed=21)


@pytest.mark.parametrize("causal", [False, True])
def test_paged_varlen_gradients(causal):
    # Gradients land in the cache pages the block table names; spare pages
    # and slots past each sequence stay zero.
    _grad_case([5, 200, 64, 1], [37, 513, 64, 300], hq=8, hk=2, d=128, page=64,
               causal=causal, seed=22)


def test_paged_varlen_gradients_with_seqused_and_features():
    _grad_case([40, 300, 2], [60, 500, 33], hq=8, hk=2, d=128, page=16, causal=True,
               used_q=[40, 256, 1], used_k=[60, 301, 0], window_size=(96, 0), softcap=20.0,
               softmax_scale=0.07, dtype=torch.bfloat16, seed=23)
