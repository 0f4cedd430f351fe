"""Dropout (the mask of fa_common.h: Philox4x32-10 draws, pinned against the
Random123 known answers in tests/test_oracle.py) against the float64 oracle
with the same seed: the kernels and oracle/attention.py dropout_factors draw
the same mask, so outputs, probabilities and gradients are compared element
by element at the usual bars; the keep rate and the reference's known-answer
test (tests/test_compare_implementations.py:161-168) are checked as well.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
OUT_ATOL = {torch.float16: ATOL[torch.float16], torch.bfloat16: ATOL[torch.bfloat16],
            torch.float32: 5e-5}
# The gradient bars of tests/test_gpu_backward.py.
GRAD_ATOL = {torch.float16: 5e-3, torch.bfloat16: 4e-2, torch.float32: 1e-4}
GRAD_RTOL = {torch.float16: 1e-2, torch.bfloat16: 4e-2, torch.float32: 1e-4}


def _grad_check(name, got, exact, dtype):
    got = to_np(got.cpu())
    bound = GRAD_ATOL[dtype] + GRAD_RTOL[dtype] * np.abs(exact)
    err = np.abs(got - exact)
    assert np.all(err <= bound), f"{name}: max |err| {float(err.max()):.3e}"


def _dense(B, Sq, Sk, Hq, Hk, D, p, seed, dtype=torch.float16, causal=False, window=(-1, -1),
           softcap=0.0, grads=True):
    from flash_attn_triton.triton_kernel.attention_kernel import dense_attention
    q = randn((B, Sq, Hq, D), seed + 1, dtype)
    k = randn((B, Sk, Hk, D), seed + 2, dtype)
    v = randn((B, Sk, Hk, D), seed + 3, dtype)
    do = randn((B, Sq, Hq, D), seed + 4, dtype)
    drop_seed = 0x1234_5678_9ABC + seed
    qd, kd, vd = (t.to(DEV).requires_grad_(grads) for t in (q, k, v))
    out = dense_attention(qd, kd, vd, softmax_scale=1 / math.sqrt(D), causal=causal,
                          window_left=window[0], window_right=window[1], softcap=softcap,
                          dropout_p=p, dropout_seed=drop_seed)
    kw = dict(causal=causal, window_size=window, softcap=softcap, dropout_p=p,
              dropout_seed=drop_seed)
    ref, _, _ = ora.attention(to_np(q), to_np(k), to_np(v), None, **kw)
    assert_close(to_np(out.detach().cpu()), ref, OUT_ATOL[dtype], "out", dtype)
    if grads:
        out.backward(do.to(DEV))
        refg = ora.attention_backward(to_np(q), to_np(k), to_np(v), to_np(do), None, **kw)
        for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), refg):
            _grad_check(name, t.grad, r, dtype)
    return out.detach()


@pytest.mark.parametrize("d", [16, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_dense_forward_and_backward(d, causal):
    _dense(2, 200, 200, 4, 2, d, 0.3, 10 + d, causal=causal)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dtypes_and_features(dtype):
    _dense(1, 300, 333, 8, 2, 128, 0.15, 20, dtype=dtype, causal=True, window=(100, 0),
           softcap=25.0)


def test_fp32_forward():
    _dense(1, 130, 130, 2, 2, 64, 0.4, 30, dtype=torch.float32, causal=True, grads=False)


def test_fp32_forward_and_backward():
    _dense(2, 130, 150, 4, 2, 64, 0.4, 31, dtype=torch.float32, causal=True)
    _dense(1, 200, 200, 2, 1, 128, 0.2, 32, dtype=torch.float32, causal=False, softcap=10.0)
    _dense(1, 96, 96, 2, 1, 256, 0.2, 33, dtype=torch.float32, causal=False)


def test_same_seed_same_output_and_seeds_differ():
    a = _dense(1, 128, 128, 2, 2, 64, 0.5, 40, grads=False)
    b = _dense(1, 128, 128, 2, 2, 64, 0.5, 40, grads=False)
    assert torch.equal(a, b)
    from flash_attn_triton.triton_kernel.attention_kernel import dense_forward
    q = randn((1, 128, 2, 64), 41).to(DEV)
    o1 = dense_forward(q, q, q, softmax_scale=0.125, causal=False, dropout_p=0.5, dropout_seed=1)
    o2 = dense_forward(q, q, q, softmax_scale=0.125, causal=False, dropout_p=0.5, dropout_seed=2)
    assert not torch.equal(o1, o2)


def test_public_api_seed_follows_torch_manual_seed():
    from flash_attn_triton import flash_attn_func
    from flash_attn_triton.triton_kernel.attention_kernel import new_dropout_seed
    q, k, v = (randn((1, 96, 2, 64), s) for s in (50, 51, 52))
    torch.manual_seed(123)
    seed = new_dropout_seed()
    torch.manual_seed(123)
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), dropout_p=0.25, causal=True)
    ref = ora.attention(to_np(q), to_np(k), to_np(v), None, True, dropout_p=0.25,
                        dropout_seed=seed)[0]
    assert_close(to_np(out.cpu()), ref, OUT_ATOL[torch.float16], "out", torch.float16)


def test_reference_known_answer():
    # tests/test_compare_implementations.py:161-168: q = k = 0, v = 1, one key:
    # every output element is 2 (kept, scaled by 1/(1-0.5)) or 0 (dropped).
    from flash_attn_triton import flash_attn_func
    q = torch.zeros(1, 1, 1, 16, device=DEV, dtype=torch.float16)
    seen = set()
    for s in range(32):
        torch.manual_seed(s)
        out = flash_attn_func(q, q, torch.ones_like(q), dropout_p=0.5)
        kept = torch.isclose(out, torch.full_like(out, 2.0), atol=1e-3, rtol=0)
        dropped = torch.isclose(out, torch.zeros_like(out), atol=1e-3, rtol=0)
        assert torch.all(kept | dropped)
        seen.add(bool(kept.all()))
    assert seen == {True, False}


def test_probs_are_the_dropped_probabilities_and_keep_rate():
    from flash_attn_triton import flash_attn_func
    q, k, v = (randn((2, 256, 4, 64), s).to(DEV) for s in (60, 61, 62))
    torch.manual_seed(7)
    out, lse, probs = flash_attn_func(q, k, v, dropout_p=0.25, return_attn_probs=True)
    torch.manual_seed(7)
    from flash_attn_triton.triton_kernel.attention_kernel import new_dropout_seed
    seed = new_dropout_seed()
    ref_out, ref_lse, ref_probs = ora.attention(to_np(q.cpu()), to_np(k.cpu()), to_np(v.cpu()),
                                                dropout_p=0.25, dropout_seed=seed)
    assert_close(to_np(out.cpu()), ref_out, OUT_ATOL[torch.float16], "out", torch.float16)
    assert_close(probs.cpu().numpy(), ref_probs, 1e-3, "probs")
    assert_close(lse.cpu().numpy(), ref_lse, 1e-3, "lse")
    kept = (probs > 0).float().mean().item()
    n = probs.numel()
    assert abs(kept - 0.75) < 6 * math.sqrt(0.25 * 0.75 / n)


def _varlen(lq, lk, p, seed, Hq=4, Hk=2, D=64, causal=True, paged=False):
    from flash_attn_triton.triton_kernel.attention_kernel import varlen_attention, varlen_forward
    cq = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32)
    ck = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32)
    q = randn((int(sum(lq)), Hq, D), seed + 1)
    k = randn((int(sum(lk)), Hk, D), seed + 2)
    v = randn((int(sum(lk)), Hk, D), seed + 3)
    do = randn((int(sum(lq)), Hq, D), seed + 4)
    dseed = 987654321 + seed
    kw = dict(softmax_scale=1 / math.sqrt(D), causal=causal, dropout_p=p, dropout_seed=dseed)
    ref = ora.attention_varlen(to_np(q), to_np(k), to_np(v), cq.numpy(), ck.numpy(), None, causal,
                               dropout_p=p, dropout_seed=dseed)[0]
    if paged:
        # The same keys laid out one 16-slot page at a time through a block table.
        page, pages, rows = 16, [], []
        for b in range(len(lk)):
            n = (lk[b] + page - 1) // page
            rows.append(list(range(len(pages), len(pages) + n)))
            pages += [b] * n
        kc = torch.zeros((len(pages), page, Hk, D), dtype=torch.float16)
        vc = torch.zeros_like(kc)
        for b in range(len(lk)):
            for t in range(lk[b]):
                kc[rows[b][t // page], t % page] = k[ck[b] + t]
                vc[rows[b][t // page], t % page] = v[ck[b] + t]
        bt = torch.zeros((len(lk), max(len(r) for r in rows)), dtype=torch.int32)
        for b, r in enumerate(rows):
            bt[b, :len(r)] = torch.tensor(r, dtype=torch.int32)
        out = varlen_forward(q.to(DEV), kc.to(DEV), vc.to(DEV), cq.to(DEV), ck.to(DEV), max(lq),
                             max(lk), block_table=bt.to(DEV), **kw)
        assert_close(to_np(out.cpu()), ref, OUT_ATOL[torch.float16], "paged out", torch.float16)
        return
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = varlen_attention(qd, kd, vd, cq.to(DEV), ck.to(DEV), max(lq), max(lk), **kw)
    assert_close(to_np(out.detach().cpu()), ref, OUT_ATOL[torch.float16], "out", torch.float16)
    out.backward(do.to(DEV))
    refg = ora.attention_varlen_backward(to_np(q), to_np(k), to_np(v), to_np(do), cq.numpy(),
                                         ck.numpy(), None, causal, dropout_p=p, dropout_seed=dseed)
    for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), refg):
        _grad_check(name, t.grad, r, torch.float16)


def test_varlen_forward_and_backward():
    _varlen([5, 130, 0, 77], [9, 130, 4, 200], 0.2, 70)


def test_paged_varlen_forward():
    _varlen([33, 100], [50, 140], 0.35, 80, paged=True)
