"""Parity of the fp32 HIP path (fp32 inputs computed in fp32) against the
float64 oracle.

The reference accepts fp32 q/k/v (flash_attn_interface.py:95-96) and keeps
the whole computation in fp32; BASELINE config 1 is an fp32 problem.  The
kernel multiplies and accumulates in fp32 on the fp32 matrix core, so the bar
is 5e-5 max-abs on outputs of O(1) (measured errors are ~1e-6), two orders of
magnitude below the fp16 bar: an accidental 16-bit rounding anywhere on the
path (inputs, P, output) would fail it.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import assert_close, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
F32 = torch.float32
ATOL32 = 5e-5


def _dense(q, k, v, **kw):
    from flash_attn_triton.triton_kernel.attention_kernel import dense_forward
    scale = kw.pop("softmax_scale", 1.0 / math.sqrt(q.shape[-1]))
    out, lse = dense_forward(q.to(DEV), k.to(DEV), v.to(DEV), softmax_scale=scale,
                             return_lse=True, **kw)
    torch.cuda.synchronize()
    assert out.dtype == F32
    return out.cpu(), lse.cpu(), scale


def _check(q, k, v, **kw):
    alibi = kw.get("alibi")
    out, lse, scale = _dense(q, k, v, **dict(kw))
    ref, ref_lse, _ = ora.attention(to_np(q), to_np(k), to_np(v), scale, kw.get("causal", False),
                                    (kw.get("window_left", -1), kw.get("window_right", -1)),
                                    kw.get("softcap", 0.0),
                                    None if alibi is None else to_np(alibi),
                                    causal_offset=kw.get("q_pos_offset", 0))
    assert_close(to_np(out), ref, ATOL32, "fp32 out")
    assert_close(lse.numpy(), ref_lse, ATOL32, "fp32 lse")


def test_baseline_config_c1():
    # dense non-causal, fp32, B=2, H=4, S=256, D=64, scale 1/sqrt(D).
    q, k, v = (randn((2, 256, 4, 64), s, F32) for s in (0, 1, 2))
    _check(q, k, v, causal=False)


@pytest.mark.parametrize("head_dim", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dims(head_dim, causal):
    q, k, v = (randn((2, 150, 3, head_dim), s, F32) for s in (3, 4, 5))
    _check(q, k, v, causal=causal)


@pytest.mark.parametrize("sq,sk", [(1, 1), (7, 300), (130, 64), (300, 129)])
def test_rectangular_gqa(sq, sk):
    q = randn((2, sq, 4, 64), 6, F32)
    k = randn((2, sk, 2, 64), 7, F32)
    v = randn((2, sk, 2, 64), 8, F32)
    _check(q, k, v, causal=True)
    _check(q, k, v, causal=False, q_pos_offset=sk - sq)


def test_window_alibi_softcap():
    H = 4
    q, k = (randn((2, 200, H, 128), s, F32, scale=2.0) for s in (9, 10))
    v = randn((2, 200, H, 128), 11, F32)
    slopes = (2.0 ** (-8.0 * (torch.arange(H) + 1) / H)).expand(2, H).contiguous().float()
    _check(q, k, v, causal=True, window_left=50, window_right=0, softcap=20.0, alibi=slopes)


def test_public_api_and_probs():
    from flash_attn_triton import flash_attn_func, flash_attn_qkvpacked_func
    q, k, v = (randn((1, 96, 2, 32), s, F32) for s in (12, 13, 14))
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True).cpu()
    assert out.dtype == F32
    ref, ref_lse, ref_p = ora.attention(to_np(q), to_np(k), to_np(v), causal=True)
    assert_close(to_np(out), ref, ATOL32, "flash_attn_func fp32")
    o2, lse2, p2 = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True,
                                   return_attn_probs=True)
    assert_close(to_np(o2.cpu()), ref, ATOL32, "probs path out")
    assert_close(lse2.cpu().numpy(), ref_lse, ATOL32, "probs path lse")
    assert_close(p2.cpu().numpy(), ref_p, 1e-6, "probs")
    qkv = torch.stack((q, k, v), dim=2)
    o3 = flash_attn_qkvpacked_func(qkv.to(DEV), causal=True).cpu()
    assert_close(to_np(o3), ref, ATOL32, "qkvpacked fp32")


def test_varlen():
    from flash_attn_triton.triton_kernel.attention_kernel import varlen_forward
    lq, lk = [1, 130, 0, 77], [3, 130, 40, 200]
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32)
    q = randn((sum(lq), 4, 64), 15, F32)
    k = randn((sum(lk), 2, 64), 16, F32)
    v = randn((sum(lk), 2, 64), 17, F32)
    for causal in (False, True):
        out, lse = varlen_forward(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                                  max(lq), max(lk), softmax_scale=0.125, causal=causal,
                                  return_lse=True)
        torch.cuda.synchronize()
        ref, ref_lse = ora.attention_varlen(to_np(q), to_np(k), to_np(v), cu_q.numpy(),
                                            cu_k.numpy(), 0.125, causal)
        assert_close(to_np(out.cpu()), ref, ATOL32, f"varlen fp32 causal={causal}")
        assert_close(lse.cpu().numpy(), ref_lse, ATOL32, "varlen fp32 lse")


@pytest.mark.parametrize("sq", [1, 5])
def test_paged_kvcache(sq):
    from flash_attn_triton import flash_attn_with_kvcache
    lengths = [1, 37, 256, 700]
    page, hq, hk, d = 256, 8, 2, 128
    pages = [(L + page - 1) // page for L in lengths]
    gen = torch.Generator().manual_seed(18)
    perm = torch.randperm(sum(pages), generator=gen)
    bt = torch.zeros((len(lengths), max(pages)), dtype=torch.int32)
    c = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[c:c + n]
        c += n
    kc = randn((sum(pages), page, hk, d), 19, F32)
    vc = randn((sum(pages), page, hk, d), 20, F32)
    q = randn((len(lengths), sq, hq, d), 21, F32)
    seqlens = torch.tensor(lengths, dtype=torch.int32)
    for causal in (False, True):
        out = flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV),
                                      cache_seqlens=seqlens.to(DEV), block_table=bt.to(DEV),
                                      causal=causal)
        torch.cuda.synchronize()
        ref, _, _, _ = ora.attention_kvcache(to_np(q), to_np(kc), to_np(vc), cache_seqlens=lengths,
                                             block_table=bt.numpy(), causal=causal)
        assert_close(to_np(out.cpu()), ref, ATOL32, f"paged fp32 causal={causal}")
