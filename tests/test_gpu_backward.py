"""Gradients of the HIP backward kernels (fa_bwd_dense / fa_bwd_varlen) against
the float64 oracle (oracle/attention.py attention_backward, pinned against
torch autograd and finite differences in tests/test_oracle.py).

Bars: the reference's own gradient tests compare fp16 against SDPA at
atol = rtol = 2e-2 (tests/test_compare_implementations.py:23-24,81-82).  Here
the comparison is against the exact float64 gradient, elementwise
|got - exact| <= GRAD_ATOL + GRAD_RTOL * |exact|: fp16 inputs carry P and dS
rounded to fp16 into fp32 accumulations, bf16 rounds them 8x coarser; fp32
inputs keep every product in fp32 (the fp32 matrix core), within 1e-4.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
GRAD_ATOL = {torch.float16: 5e-3, torch.bfloat16: 4e-2, torch.float32: 1e-4}
GRAD_RTOL = {torch.float16: 1e-2, torch.bfloat16: 4e-2, torch.float32: 1e-4}


def _check(name, got, exact, dtype):
    got = to_np(got.cpu())
    err = np.abs(got - exact)
    bound = GRAD_ATOL[dtype] + GRAD_RTOL[dtype] * np.abs(exact)
    worst = float(np.max(err - bound)) if err.size else -1.0
    assert np.all(np.isfinite(got)), f"{name}: non-finite gradient"
    assert worst <= 0, (f"{name}: max |err| {float(np.max(err)):.3e} exceeds the bar "
                        f"(max |exact| {float(np.max(np.abs(exact))):.3e})")


def _dense_case(B, Sq, Sk, Hq, Hk, D, dtype=torch.float16, seed=0, causal=False,
                window=(-1, -1), softcap=0.0, alibi=False, scale=None, api="func"):
    from flash_attn_triton import flash_attn_func, flash_attn_func_cross
    q = randn((B, Sq, Hq, D), seed + 1, dtype)
    k = randn((B, Sk, Hk, D), seed + 2, dtype)
    v = randn((B, Sk, Hk, D), seed + 3, dtype)
    do = randn((B, Sq, Hq, D), seed + 4, dtype)
    slopes = (torch.rand(Hq, generator=torch.Generator().manual_seed(seed + 5)) * 0.5
              if alibi else None)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    fn = flash_attn_func if (api == "func" and Sq == Sk) else flash_attn_func_cross
    out = fn(qd, kd, vd, causal=causal, window_size=window, softcap=softcap,
             alibi_slopes=None if slopes is None else slopes.to(DEV), softmax_scale=scale)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    ref = ora.attention_backward(to_np(q), to_np(k), to_np(v), to_np(do), scale, causal, window,
                                 softcap, None if slopes is None else slopes.double().numpy())
    for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), ref):
        _check(name, t.grad, r, dtype)
    return qd.grad, kd.grad, vd.grad


@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dims(d, causal):
    _dense_case(2, 200, 200, 4, 4, d, causal=causal, seed=d)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_ragged_lengths(dtype, causal):
    _dense_case(2, 333, 333, 8, 2, 128, dtype=dtype, causal=causal, seed=11)


@pytest.mark.parametrize("causal", [False, True])
def test_cross_lengths(causal):
    # Sq != Sk: flash_attn_func_cross, upper-left alignment.
    _dense_case(1, 70, 301, 4, 2, 64, causal=causal, seed=21)
    _dense_case(1, 257, 64, 4, 4, 128, causal=causal, seed=22)


@pytest.mark.parametrize("d", [64, 128])
def test_rows_without_visible_keys(d):
    # Window (8, 8) over 64 keys: query rows past 71 see no key (LSE -inf, zero
    # output and zero gradient); the dK/dV kernel masks every pair of them.
    _dense_case(1, 300, 64, 4, 2, d, causal=False, window=(8, 8), seed=23)
    _dense_case(2, 200, 40, 2, 2, d, causal=True, window=(4, -1), seed=24)


@pytest.mark.parametrize("d", [64, 128])
def test_window_alibi_softcap(d):
    _dense_case(2, 300, 300, 4, 2, d, causal=True, window=(64, 0), softcap=20.0, alibi=True,
                seed=31)
    _dense_case(1, 190, 190, 2, 1, d, causal=False, window=(16, 40), softcap=5.0, seed=32,
                scale=0.3)


def test_d256_generic():
    _dense_case(1, 150, 150, 2, 2, 256, causal=True, softcap=10.0, alibi=True, seed=41)


def test_reference_gradient_case():
    # tests/test_compare_implementations.py:86-91: B2 S17 H2 D16, scale 0.125.
    for causal in (False, True):
        _dense_case(2, 17, 17, 2, 2, 16, causal=causal, scale=0.125, seed=42)


def test_deterministic():
    a = _dense_case(1, 256, 256, 8, 2, 64, causal=True, seed=51)
    b = _dense_case(1, 256, 256, 8, 2, 64, causal=True, seed=51)
    for x, y in zip(a, b):
        assert torch.equal(x, y), "two identical backward calls differ"


def test_qkvpacked_and_low_level_attention():
    from flash_attn_triton import flash_attn_qkvpacked_func
    from flash_attn_triton.triton_kernel.attention_kernel import attention
    qkv = randn((1, 128, 3, 2, 64), 61).to(DEV).requires_grad_()
    do = randn((1, 128, 2, 64), 62).to(DEV)
    flash_attn_qkvpacked_func(qkv, causal=True).backward(do)
    q, k, v = (to_np(t) for t in qkv.detach().cpu().unbind(2))
    ref = ora.attention_backward(q, k, v, to_np(do.cpu()), None, True)
    for i in range(3):
        _check(f"dqkv[{i}]", qkv.grad[:, :, i], ref[i], torch.float16)
    # attention(): [B, H, S, D] views, the reference's low-level entry point.
    qh, kh, vh = (randn((1, 2, 128, 64), s).to(DEV).requires_grad_() for s in (63, 64, 65))
    attention(qh, kh, vh, causal=True).backward(do.transpose(1, 2))
    ref = ora.attention_backward(*(to_np(t.detach().cpu().transpose(1, 2)) for t in (qh, kh, vh)),
                                 to_np(do.cpu()), None, True)
    for name, t, r in zip(("dq", "dk", "dv"), (qh, kh, vh), ref):
        _check(name, t.grad.transpose(1, 2), r, torch.float16)


def test_probs_path_gradients():
    from flash_attn_triton import flash_attn_func
    q, k, v = (randn((1, 96, 2, 32), s).to(DEV).requires_grad_() for s in (71, 72, 73))
    do = randn((1, 96, 2, 32), 74)
    out, lse, probs = flash_attn_func(q, k, v, causal=True, return_attn_probs=True)
    assert not lse.requires_grad and not probs.requires_grad
    out.backward(do.to(DEV))
    ref = ora.attention_backward(*(to_np(t.detach().cpu()) for t in (q, k, v)), to_np(do),
                                 None, True)
    for name, t, r in zip(("dq", "dk", "dv"), (q, k, v), ref):
        _check(name, t.grad, r, torch.float16)


def _varlen_case(lq, lk, Hq=4, Hk=2, D=64, dtype=torch.float16, seed=0, causal=False,
                 window=(-1, -1), softcap=0.0, alibi=False):
    from flash_attn_triton import flash_attn_varlen_func
    cq = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32)
    ck = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32)
    q = randn((int(sum(lq)), Hq, D), seed + 1, dtype)
    k = randn((int(sum(lk)), Hk, D), seed + 2, dtype)
    v = randn((int(sum(lk)), Hk, D), seed + 3, dtype)
    do = randn((int(sum(lq)), Hq, D), seed + 4, dtype)
    slopes = (torch.rand(len(lq), Hq, generator=torch.Generator().manual_seed(seed + 5)) * 0.5
              if alibi else None)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = flash_attn_varlen_func(qd, kd, vd, cq.to(DEV), ck.to(DEV), max(lq), max(lk),
                                 causal=causal, window_size=window, softcap=softcap,
                                 alibi_slopes=None if slopes is None else slopes.to(DEV))
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    ref = ora.attention_varlen_backward(to_np(q), to_np(k), to_np(v), to_np(do), cq.numpy(),
                                        ck.numpy(), None, causal, window, softcap,
                                        None if slopes is None else slopes.double().numpy())
    for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), ref):
        _check(name, t.grad, r, dtype)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_ragged(causal):
    _varlen_case([1, 130, 64, 257, 5], [3, 130, 200, 100, 5], causal=causal, seed=80)


def test_varlen_empty_sequences_and_features():
    _varlen_case([0, 20, 33, 7], [5, 0, 40, 7], causal=True, seed=90)
    _varlen_case([300, 129, 64], [300, 129, 64], Hq=8, Hk=2, D=128, causal=True,
                 window=(64, 0), softcap=30.0, alibi=True, seed=91)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_kv_heads_over_xcds(causal):
    # 4 sequences x 2 K/V heads = 8 K/V heads: the launches deal them
    # round-robin over the 8 XCDs (GQA group 2 for dQ); ragged lengths.
    _varlen_case([300, 7, 129, 64], [300, 40, 129, 200], Hq=4, Hk=2, D=128, causal=causal,
                 seed=97)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_varlen_dtypes_d128(dtype):
    _varlen_case([200, 513], [200, 513], Hq=4, Hk=4, D=128, dtype=dtype, causal=True, seed=95)


def test_baseline_c2_sampled_heads():
    # BASELINE config 2 shape (B4 H32 S4096 D128 fp16, causal): the whole
    # backward runs; two (batch, head) slices are checked against the oracle.
    from flash_attn_triton import flash_attn_func
    B, S, H, D = 4, 4096, 32, 128
    gen = torch.Generator(device="cpu").manual_seed(1)
    q, k, v, do = (torch.randn((B, S, H, D), generator=gen).to(torch.float16) for _ in range(4))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    flash_attn_func(qd, kd, vd, causal=True).backward(do.to(DEV))
    torch.cuda.synchronize()
    for b, h in ((0, 0), (3, 31)):
        sl = (slice(b, b + 1), slice(None), slice(h, h + 1))
        ref = ora.attention_backward(to_np(q[sl]), to_np(k[sl]), to_np(v[sl]), to_np(do[sl]),
                                     None, True)
        for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), ref):
            _check(f"{name}[{b},{h}]", t.grad[sl], r, torch.float16)


def _kvcache_grad_case(paged, causal, rotary=False, alibi=False, window=(-1, -1), seed=300):
    # Gradients through flash_attn_with_kvcache against the float64 oracle
    # run per sequence on the gathered keys (the reference's own
    # computation, flash_attn_interface.py:494-525), the key gradients
    # scattered back into the cache's rows.
    from flash_attn_triton import flash_attn_with_kvcache
    B, Sq, Hq, Hk, D = 3, 4, 4, 2, 64
    lengths = [70, 131, 9]
    if paged:
        page = 64
        pages_per = [(L + page - 1) // page for L in lengths]
        n_pages = sum(pages_per) + 2
        perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(seed))
        bt = torch.zeros((B, max(pages_per)), dtype=torch.int32)
        pos = 0
        for b, n in enumerate(pages_per):
            bt[b, :n] = perm[pos:pos + n].to(torch.int32)
            pos += n
        kc = randn((n_pages, page, Hk, D), seed + 1)
        vc = randn((n_pages, page, Hk, D), seed + 2)
        rows, pads = None, [0] * B
    else:
        cap = 160
        kc = randn((B + 1, cap, Hk, D), seed + 1)
        vc = randn((B + 1, cap, Hk, D), seed + 2)
        rows, pads, bt = [2, 0, 3], [5, 0, 17], None
    q = randn((B, Sq, Hq, D), seed + 3)
    do = randn((B, Sq, Hq, D), seed + 4)
    slopes = (torch.rand(Hq, generator=torch.Generator().manual_seed(seed + 5)) * 0.3
              if alibi else None)
    cos = sin = None
    if rotary:
        ang = torch.arange(256, dtype=torch.float32)[:, None] * (
            1e-2 * torch.arange(1, D // 4 + 1, dtype=torch.float32))[None, :]
        cos, sin = torch.cos(ang), torch.sin(ang)
    qd, kcd, vcd = (t.to(DEV).requires_grad_() for t in (q, kc, vc))
    out = flash_attn_with_kvcache(
        qd, kcd, vcd, cache_seqlens=torch.tensor(lengths, dtype=torch.int32).to(DEV),
        block_table=None if bt is None else bt.to(DEV),
        cache_batch_idx=None if rows is None else torch.tensor(rows, dtype=torch.int32).to(DEV),
        cache_leftpad=None if paged else torch.tensor(pads, dtype=torch.int32).to(DEV),
        rotary_cos=None if cos is None else cos.to(DEV), rotary_sin=None if sin is None else sin.to(DEV),
        rotary_interleaved=False, causal=causal, window_size=window,
        alibi_slopes=None if slopes is None else slopes.to(DEV))
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D)
    dq_ref = np.zeros(q.shape)
    dk_ref, dv_ref = np.zeros(kc.shape), np.zeros(vc.shape)
    cos_h = None if cos is None else cos.half().double().numpy()
    sin_h = None if sin is None else sin.half().double().numpy()
    for b, L in enumerate(lengths):
        st = pads[b]
        if paged:
            page = kc.shape[1]
            j = np.arange(L)
            idx = (bt[b].numpy()[j // page].astype(np.int64), j % page)
        else:
            idx = (np.full(L, rows[b]), st + np.arange(L))
        kb, vb = to_np(kc)[idx][None], to_np(vc)[idx][None]
        qb = to_np(q[b:b + 1])
        pos = np.arange(Sq) + L - Sq + st
        if rotary:
            qb = ora.apply_rotary(qb, cos_h, sin_h, pos, False)
        dqb, dkb, dvb = ora.attention_backward(
            qb, kb, vb, to_np(do[b:b + 1]), scale, causal, window, 0.0,
            None if slopes is None else slopes.double().numpy(),
            causal_offset=(L - Sq) if causal else 0)
        if rotary:   # the rotation is orthogonal: back through it with the angle negated
            dqb = ora.apply_rotary(dqb, cos_h, -sin_h, pos, False)
        dq_ref[b] = dqb[0]
        np.add.at(dk_ref, idx, dkb[0])
        np.add.at(dv_ref, idx, dvb[0])
    _check("dq", qd.grad, dq_ref, torch.float16)
    _check("dk_cache", kcd.grad, dk_ref, torch.float16)
    _check("dv_cache", vcd.grad, dv_ref, torch.float16)


@pytest.mark.parametrize("paged", [True, False])
@pytest.mark.parametrize("causal", [False, True])
def test_kvcache_gradients(paged, causal):
    _kvcache_grad_case(paged, causal)


def test_kvcache_gradients_rotary_alibi_window():
    _kvcache_grad_case(True, True, rotary=True, alibi=True, window=(40, 0), seed=320)
    _kvcache_grad_case(False, False, rotary=True, window=(16, 8), seed=340)


@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_fp32_head_dims(d, causal):
    # D = 256: two passes over the output dims in both kernels, V rows read
    # again per query tile in the dK/dV kernel.
    _dense_case(2, 150, 150, 4, 2, d, dtype=torch.float32, causal=causal, seed=140 + d)


def test_fp32_head_dim_256_features():
    # D = 256 through the generic instantiations: cross lengths, window,
    # softcap, ALiBi; varlen with ragged sequences; attn_bias (dropout at
    # D = 256 in fp32: test_gpu_dropout.py).
    _dense_case(1, 70, 301, 4, 2, 256, dtype=torch.float32, causal=True, window=(64, 0),
                softcap=20.0, alibi=True, seed=410)
    _varlen_case([1, 130, 64, 97], [3, 130, 200, 97], Hq=4, Hk=2, D=256,
                 dtype=torch.float32, causal=True, seed=412)
    _bias_case((1, 4, 100, 100), Sq=100, Sk=100, D=256, dtype=torch.float32, causal=True,
               seed=413)


def test_fp32_cross_and_features():
    _dense_case(1, 70, 301, 4, 2, 64, dtype=torch.float32, causal=True, seed=150)
    _dense_case(2, 300, 300, 4, 2, 128, dtype=torch.float32, causal=True, window=(64, 0),
                softcap=20.0, alibi=True, seed=151)
    _dense_case(1, 190, 190, 2, 1, 32, dtype=torch.float32, causal=False, window=(16, 40),
                softcap=5.0, seed=152, scale=0.3)


def test_fp32_varlen():
    _varlen_case([1, 130, 64, 257, 5], [3, 130, 200, 100, 5], Hq=4, Hk=2, D=64,
                 dtype=torch.float32, causal=True, seed=160)
    _varlen_case([300, 129, 64], [300, 129, 64], Hq=8, Hk=2, D=128, dtype=torch.float32,
                 causal=True, window=(64, 0), softcap=30.0, alibi=True, seed=161)


def test_fp32_bias_gradients():
    _bias_case((1, 4, 120, 120), Sq=120, Sk=120, D=64, dtype=torch.float32, causal=True,
               softcap=10.0, seed=170)
    _bias_case((120, 120), Sq=120, Sk=120, D=128, dtype=torch.float32, causal=False, seed=171)


def _bias_case(bias_shape, B=2, Sq=150, Sk=190, Hq=4, Hk=2, D=64, dtype=torch.float16,
               seed=0, causal=False, softcap=0.0, alibi=False, bias_dtype=torch.float32,
               window=(-1, -1)):
    """Gradients through attn_bias: the reference's math path is differentiated
    by torch autograd, so d bias is dS summed over the bias's broadcast dims."""
    from flash_attn_triton import flash_attn_func
    q = randn((B, Sq, Hq, D), seed + 1, dtype)
    k = randn((B, Sk, Hk, D), seed + 2, dtype)
    v = randn((B, Sk, Hk, D), seed + 3, dtype)
    do = randn((B, Sq, Hq, D), seed + 4, dtype)
    bias = randn(bias_shape, seed + 5, torch.float32).to(bias_dtype)
    slopes = (torch.rand(Hq, generator=torch.Generator().manual_seed(seed + 6)) * 0.3
              if alibi else None)
    qd, kd, vd, bd = (t.to(DEV).requires_grad_() for t in (q, k, v, bias))
    out = flash_attn_func(qd, kd, vd, causal=causal, softcap=softcap, window_size=window,
                          alibi_slopes=None if slopes is None else slopes.to(DEV), attn_bias=bd)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    ref = ora.attention_backward(to_np(q), to_np(k), to_np(v), to_np(do), None, causal, window,
                                 softcap, None if slopes is None else slopes.double().numpy(),
                                 attn_bias=bias.double().numpy(), return_dbias=True)
    for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), ref):
        _check(name, t.grad, r, dtype)
    assert bd.grad.shape == bias.shape and bd.grad.dtype == bias_dtype
    # d bias sums dS over the broadcast dims: the bar scales with the count.
    summed = (B * Hq * Sq * Sk) // int(np.prod(bias_shape))
    got = to_np(bd.grad.float().cpu())
    err = np.abs(got - ref[3])
    bound = GRAD_ATOL[dtype] * math.sqrt(summed) + GRAD_RTOL[dtype] * np.abs(ref[3])
    print(f"dbias {tuple(bias_shape)}: max-abs err {float(np.max(err)):.3e} "
          f"(max |exact| {float(np.max(np.abs(ref[3]))):.3e})")
    assert np.all(np.isfinite(got)) and np.all(err <= bound), float(np.max(err - bound))


@pytest.mark.parametrize("bias_shape", [(2, 4, 150, 150), (1, 1, 150, 150), (150, 150),
                                        (2, 1, 1, 150), (4, 150, 1)])
def test_attn_bias_gradients(bias_shape):
    _bias_case(bias_shape, Sq=150, Sk=150, causal=True, seed=110)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attn_bias_gradients_with_features(dtype):
    # Softcap (the bias sits inside the tanh), ALiBi and a window; fp16 bias;
    # D = 128 and D = 32.
    _bias_case((2, 4, 200, 200), Sq=200, Sk=200, D=128, dtype=dtype, causal=True, softcap=15.0,
               alibi=True, window=(64, 0), seed=120, bias_dtype=torch.float16)
    _bias_case((1, 4, 96, 96), Sq=96, Sk=96, D=32, dtype=dtype, causal=False, softcap=0.0,
               seed=121)


def test_attn_bias_gradients_only_bias():
    # q, k, v without grad: the bias alone is differentiated.
    from flash_attn_triton import flash_attn_func
    q, k, v = (randn((1, 64, 2, 64), s).to(DEV) for s in (131, 132, 133))
    bias = randn((1, 2, 64, 64), 134, torch.float32).to(DEV).requires_grad_()
    do = randn((1, 64, 2, 64), 135)
    flash_attn_func(q, k, v, attn_bias=bias).backward(do.to(DEV))
    ref = ora.attention_backward(*(to_np(t.cpu()) for t in (q, k, v)), to_np(do), None, False,
                                 attn_bias=to_np(bias.detach().cpu()), return_dbias=True)
    np.testing.assert_allclose(to_np(bias.grad.cpu()), ref[3], atol=GRAD_ATOL[torch.float16],
                               rtol=GRAD_RTOL[torch.float16])
