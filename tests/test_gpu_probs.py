"""Parity of the materialized-probabilities path and of ``attn_bias``.

``return_attn_probs=True`` and ``attn_bias`` follow the reference's dense
torch path (flash_attn_interface.py:15-49, varlen :642-659): out, the
natural-log LSE ``[B,H,Sq]`` and fp32 probabilities ``[B,H,Sq,Sk]``.  Here out
and LSE come from the flash kernel (bias in its score epilogue) and the
probabilities from ``fa_attn_probs``; all three are checked against the
float64 oracle.  The bias test mirrors the reference's
tests/test_compare_implementations.py:170-177 (cross 7x13, fp16 bias * 0.1,
head_dim 16), with the oracle in place of SDPA.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, max_abs, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
# fp32 probabilities exp(s - lse): the error is that of the score and LSE
# (fp32 dot products of exact fp16/bf16 inputs) times p <= 1.
PROBS_ATOL = 1e-3
LSE_ATOL = 1e-3


def _qkv(B, Sq, Sk, Hq, Hk, D, dtype, seed=0):
    return (randn((B, Sq, Hq, D), seed + 1, dtype), randn((B, Sk, Hk, D), seed + 2, dtype),
            randn((B, Sk, Hk, D), seed + 3, dtype))


def _check_triple(got, ref, dtype):
    out, lse, probs = got
    r_out, r_lse, r_probs = ref
    torch.cuda.synchronize()
    assert out.shape[:3] == r_out.shape[:3]
    assert tuple(lse.shape) == r_lse.shape and lse.dtype == torch.float32
    assert tuple(probs.shape) == r_probs.shape and probs.dtype == torch.float32
    assert_close(to_np(out), r_out, ATOL[dtype], "out", dtype)
    assert_close(lse.cpu().numpy(), r_lse, LSE_ATOL, "lse")
    assert_close(probs.cpu().numpy(), r_probs, PROBS_ATOL, "probs")


def test_cross_attention_bias_matches_oracle():
    from flash_attn_triton import flash_attn_func_cross
    q, k, v = _qkv(2, 7, 13, 2, 2, 16, torch.float16, seed=42)
    bias = (randn((2, 2, 7, 13), 11, torch.float16) * 0.1).to(torch.float16)
    out = flash_attn_func_cross(q.to(DEV), k.to(DEV), v.to(DEV), attn_bias=bias.to(DEV))
    torch.cuda.synchronize()
    ref, _, _ = ora.attention(to_np(q), to_np(k), to_np(v), attn_bias=to_np(bias))
    assert_close(to_np(out), ref, ATOL[torch.float16], "out", torch.float16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [16, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_return_attn_probs_dense(dtype, head_dim, causal):
    from flash_attn_triton import flash_attn_func
    q, k, v = _qkv(2, 97, 97, 4, 2, head_dim, dtype)
    got = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                          return_attn_probs=True)
    ref = ora.attention(to_np(q), to_np(k), to_np(v), causal=causal)
    _check_triple(got, ref, dtype)


@pytest.mark.parametrize("sq,sk", [(1, 1), (7, 13), (13, 7), (64, 200), (130, 33)])
@pytest.mark.parametrize("causal", [False, True])
def test_return_attn_probs_rectangular(sq, sk, causal):
    """flash_attn_func with Sq != Sk and return_attn_probs takes the materialized
    path before the cross routing (reference :139-143): upper-left causal."""
    from flash_attn_triton import flash_attn_func
    q, k, v = _qkv(1, sq, sk, 3, 3, 64, torch.float16, seed=sq * 7 + sk)
    got = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                          return_attn_probs=True)
    ref = ora.attention(to_np(q), to_np(k), to_np(v), causal=causal)
    _check_triple(got, ref, torch.float16)


@pytest.mark.parametrize("window", [(8, 0), (5, 9), (-1, 3)])
def test_return_attn_probs_window_alibi_softcap(window):
    from flash_attn_triton import flash_attn_func
    B, S, H, D = 2, 150, 4, 64
    q, k, v = _qkv(B, S, S, H, H, D, torch.float16, seed=5)
    slopes = torch.tensor([0.5, 0.25, 0.125, 0.0625], dtype=torch.float32)
    got = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), window_size=window, softcap=20.0,
                          alibi_slopes=slopes.to(DEV), return_attn_probs=True)
    ref = ora.attention(to_np(q), to_np(k), to_np(v), window_size=window, softcap=20.0,
                        alibi_slopes=slopes.numpy())
    _check_triple(got, ref, torch.float16)


@pytest.mark.parametrize("bias_shape", [(150,), (1, 4, 1, 150), (2, 1, 120, 150),
                                        (2, 4, 120, 150)])
@pytest.mark.parametrize("causal", [False, True])
def test_attn_bias_broadcast(bias_shape, causal):
    """Every shape that broadcasts to the scores, combined with ALiBi and softcap
    (bias after ALiBi, before softcap: reference :36-43)."""
    from flash_attn_triton import flash_attn_func_cross
    B, Sq, Sk, H, D = 2, 120, 150, 4, 128
    q, k, v = _qkv(B, Sq, Sk, H, 2, D, torch.bfloat16, seed=9)
    bias = randn(bias_shape, 21, torch.float32)
    slopes = torch.tensor([[0.3, 0.2, 0.1, 0.05], [0.05, 0.1, 0.2, 0.3]], dtype=torch.float32)
    got = flash_attn_func_cross(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, softcap=15.0,
                                alibi_slopes=slopes.to(DEV), attn_bias=bias.to(DEV),
                                return_attn_probs=True)
    ref = ora.attention(to_np(q), to_np(k), to_np(v), causal=causal, softcap=15.0,
                        alibi_slopes=slopes.numpy(), attn_bias=bias.numpy().astype(np.float64))
    _check_triple(got, ref, torch.bfloat16)
    out_only = flash_attn_func_cross(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                                     softcap=15.0, alibi_slopes=slopes.to(DEV),
                                     attn_bias=bias.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out_only.cpu(), got[0].cpu())


def test_attn_bias_rejects_bad_shape():
    from flash_attn_triton import flash_attn_func
    q, k, v = _qkv(1, 16, 16, 2, 2, 64, torch.float16)
    with pytest.raises(ValueError):
        flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), attn_bias=torch.zeros(3, 16, device=DEV))


def test_fully_masked_rows_give_zero_probs():
    """A negative causal offset leaves the first rows without keys: probabilities
    0 (nan_to_num of an empty softmax, reference :44), LSE -inf, out 0."""
    from flash_attn_triton import flash_attn_func_cross
    q, k, v = _qkv(1, 20, 20, 2, 2, 64, torch.float16, seed=3)
    out, lse, probs = flash_attn_func_cross(q.to(DEV), k.to(DEV), v.to(DEV), causal=True,
                                            return_attn_probs=True, _causal_offset=-3)
    torch.cuda.synchronize()
    r_out, r_lse, r_probs = ora.attention(to_np(q), to_np(k), to_np(v), causal=True,
                                          causal_offset=-3)
    assert np.all(np.isneginf(lse.cpu().numpy()[:, :, :3]))
    assert torch.count_nonzero(probs[:, :, :3]).item() == 0
    assert torch.count_nonzero(out[:, :3]).item() == 0
    _check_triple((out, lse, probs), (r_out, r_lse, r_probs), torch.float16)


def test_qkvpacked_return_attn_probs():
    from flash_attn_triton import flash_attn_qkvpacked_func
    qkv = randn((2, 80, 3, 4, 64), 17, torch.float16)
    got = flash_attn_qkvpacked_func(qkv.to(DEV), causal=True, return_attn_probs=True)
    ref = ora.attention(to_np(qkv[:, :, 0]), to_np(qkv[:, :, 1]), to_np(qkv[:, :, 2]),
                        causal=True)
    _check_triple(got, ref, torch.float16)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_varlen_return_attn_probs(causal, dtype):
    """Ragged batch with an empty query sequence and an empty key sequence;
    max_seqlen_* above the longest sequence.  lse [B,H,max_q] -inf padded,
    probs [B,H,max_q,max_k] zero padded (reference :642-659)."""
    from flash_attn_triton import flash_attn_varlen_func
    lens_q = [37, 0, 64, 5, 20]
    lens_k = [50, 12, 64, 0, 3]
    Hq, Hk, D = 4, 2, 64
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)
    q = randn((int(cu_q[-1]), Hq, D), 31, dtype)
    k = randn((int(cu_k[-1]), Hk, D), 32, dtype)
    v = randn((int(cu_k[-1]), Hk, D), 33, dtype)
    max_q, max_k = 70, 66
    slopes = torch.tensor([0.2, 0.1, 0.05, 0.0], dtype=torch.float32)
    out, lses, probs = flash_attn_varlen_func(
        q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(cu_q).to(DEV),
        torch.from_numpy(cu_k).to(DEV), max_q, max_k, causal=causal, alibi_slopes=slopes.to(DEV),
        return_attn_probs=True)
    torch.cuda.synchronize()
    assert tuple(lses.shape) == (5, Hq, max_q) and tuple(probs.shape) == (5, Hq, max_q, max_k)
    r_out, _ = ora.attention_varlen(to_np(q), to_np(k), to_np(v), cu_q, cu_k, causal=causal,
                                    alibi_slopes=slopes.numpy())
    assert_close(to_np(out), r_out, ATOL[dtype], "out", dtype)
    r_lses = np.full((5, Hq, max_q), -np.inf)
    r_probs = np.zeros((5, Hq, max_q, max_k))
    for b in range(5):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        if qe == qs or ke == ks:
            continue   # no query rows, or no keys: -inf LSE and zero probabilities
        _, l, pr = ora.attention(to_np(q[None, qs:qe]), to_np(k[None, ks:ke]),
                                 to_np(v[None, ks:ke]), causal=causal,
                                 alibi_slopes=slopes.numpy())
        r_lses[b, :, :qe - qs] = l[0]
        r_probs[b, :, :qe - qs, :ke - ks] = pr[0]
    assert_close(lses.cpu().numpy(), r_lses, LSE_ATOL, "lse")
    assert_close(probs.cpu().numpy(), r_probs, PROBS_ATOL, "probs")


def test_probs_rows_sum_to_one_at_size():
    """S=2048 causal D=128: every row of probabilities sums to 1 (a property
    that holds at any size) and sampled rows match the oracle."""
    from flash_attn_triton import flash_attn_func
    B, S, H, D = 1, 2048, 2, 128
    q, k, v = _qkv(B, S, S, H, H, D, torch.float16, seed=77)
    out, lse, probs = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True,
                                      return_attn_probs=True)
    torch.cuda.synchronize()
    # A row sums to exp(lse_exact - lse): within the LSE bar of 1 (fp16 rows
    # sum P after rounding it to fp16, as the P.V product uses it).
    sums = probs.sum(dim=-1, dtype=torch.float64).cpu().numpy()
    assert max_abs(sums, np.ones_like(sums)) < LSE_ATOL
    # One query row at a time: the oracle places it at position i through the
    # causal offset.
    for i in (0, 1, 511, 1024, 2047):
        o, l, pr = ora.attention(to_np(q[:, i:i + 1]), to_np(k), to_np(v), causal=True,
                                 causal_offset=int(i))
        assert_close(to_np(out[:, i:i + 1].cpu()), o, ATOL[torch.float16], f"out row {i}",
                     torch.float16)
        assert_close(lse[:, :, i:i + 1].cpu().numpy(), l, LSE_ATOL, f"lse row {i}")
        assert_close(probs[:, :, i:i + 1].cpu().numpy(), pr, PROBS_ATOL, f"probs row {i}")
