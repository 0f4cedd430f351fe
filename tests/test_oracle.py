"""Pins the CPU oracle before anything is compared against it (CPU only).

Each oracle function is checked against something independent of its own
formula: torch's CPU ``scaled_dot_product_attention`` (the oracle of the
reference's tests, tests/test_compare_implementations.py:31-41, with window
and ALiBi expressed as SDPA masks/biases as at :97-105 and :208-211), closed
forms, a pure-Python brute force on tiny shapes, exact rational arithmetic
for the quantizer, and a second (C) implementation of the quantizer.
"""
import ctypes
import math
import os
import subprocess
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ora
from oracle import quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _sdpa(q, k, v, causal=False, scale=None, mask=None, gqa=False):
    """SDPA in float64 on [B,S,H,D] numpy inputs -> [B,S,H,D]."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).double().transpose(1, 2)
    out = F.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=mask, is_causal=causal,
                                         scale=scale, enable_gqa=gqa)
    return out.transpose(1, 2).numpy()


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


# ----------------------------------------------------------------- attention vs SDPA
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(17, 17), (7, 13), (13, 7), (64, 64)])
def test_attention_matches_sdpa(causal, sq, sk):
    q, k, v = _rand((2, sq, 3, 16), 1), _rand((2, sk, 3, 16), 2), _rand((2, sk, 3, 16), 3)
    out, lse, probs = ora.attention(q, k, v, 0.125, causal)
    np.testing.assert_allclose(out, _sdpa(q, k, v, causal, 0.125), atol=1e-12)
    # LSE is consistent with the probabilities: p = exp(s - lse) sums to one.
    np.testing.assert_allclose(probs.sum(-1), 1.0, atol=1e-12)


def test_attention_gqa_matches_sdpa():
    q, k, v = _rand((2, 20, 8, 32), 4), _rand((2, 20, 2, 32), 5), _rand((2, 20, 2, 32), 6)
    out, _, _ = ora.attention(q, k, v, None, True)
    np.testing.assert_allclose(out, _sdpa(q, k, v, True, 1 / math.sqrt(32), gqa=True), atol=1e-12)


def test_default_scale_is_inverse_sqrt_d():
    q, k, v = _rand((1, 9, 2, 64), 7), _rand((1, 9, 2, 64), 8), _rand((1, 9, 2, 64), 9)
    out, _, _ = ora.attention(q, k, v)
    np.testing.assert_allclose(out, _sdpa(q, k, v, False, 0.125), atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("window", [(3, 2), (0, 0), (5, -1), (-1, 1)])
def test_window_matches_sdpa_mask(causal, window):
    # Reference tests/test_compare_implementations.py:93-130 builds the same mask.
    q, k, v = _rand((1, 17, 2, 16), 10), _rand((1, 17, 2, 16), 11), _rand((1, 17, 2, 16), 12)
    pos = torch.arange(17)
    valid = torch.ones(17, 17, dtype=torch.bool)
    if window[0] >= 0:
        valid &= pos[None, :] >= pos[:, None] - window[0]
    if window[1] >= 0:
        valid &= pos[None, :] <= pos[:, None] + window[1]
    if causal:
        valid &= pos[None, :] <= pos[:, None]
    out, _, _ = ora.attention(q, k, v, None, causal, window)
    np.testing.assert_allclose(out, _sdpa(q, k, v, mask=valid), atol=1e-12)


def test_alibi_matches_sdpa_bias():
    # Reference tests/test_compare_implementations.py:204-212.
    q, k, v = _rand((2, 17, 2, 16), 13), _rand((2, 17, 2, 16), 14), _rand((2, 17, 2, 16), 15)
    slopes = np.abs(_rand((2, 2), 16)) * 0.1
    qp, kp = torch.arange(17)[:, None], torch.arange(17)[None, :]
    bias = -torch.from_numpy(slopes)[:, :, None, None] * (qp - kp).abs().double()
    out, _, _ = ora.attention(q, k, v, None, False, alibi_slopes=slopes)
    np.testing.assert_allclose(out, _sdpa(q, k, v, mask=bias), atol=1e-12)
    # (H,) slopes broadcast over the batch
    out1, _, _ = ora.attention(q, k, v, None, True, alibi_slopes=slopes[0])
    bias1 = bias[:1].expand(2, -1, -1, -1) + torch.where(qp >= kp, 0.0, -math.inf)
    np.testing.assert_allclose(out1, _sdpa(q, k, v, mask=bias1), atol=1e-12)


def test_attn_bias_matches_sdpa():
    # Reference tests/test_compare_implementations.py:171-178.
    q, k, v = _rand((2, 7, 2, 16), 17), _rand((2, 13, 2, 16), 18), _rand((2, 13, 2, 16), 19)
    bias = _rand((2, 2, 7, 13), 20) * 0.1
    out, _, _ = ora.attention(q, k, v, attn_bias=bias)
    np.testing.assert_allclose(out, _sdpa(q, k, v, mask=torch.from_numpy(bias)), atol=1e-12)


# ----------------------------------------------------------------- closed forms
def test_softcap_saturates_to_known_probabilities():
    # scores +-100 with cap 1: capped scores are tanh(+-100) = +-1 (to 1e-80), so
    # the two probabilities are e/(e + 1/e) and (1/e)/(e + 1/e).
    D = 4
    q = np.zeros((1, 1, 1, D)); q[..., 0] = 10.0
    k = np.zeros((1, 2, 1, D)); k[0, 0, 0, 0] = 10.0; k[0, 1, 0, 0] = -10.0
    v = np.zeros((1, 2, 1, D)); v[0, 0, 0, 1] = 1.0; v[0, 1, 0, 2] = 1.0
    out, lse, probs = ora.attention(q, k, v, softmax_scale=1.0, softcap=1.0)
    e = math.e
    np.testing.assert_allclose(probs[0, 0, 0], [e / (e + 1 / e), (1 / e) / (e + 1 / e)], rtol=1e-14)
    np.testing.assert_allclose(lse[0, 0, 0], math.log(e + 1 / e), rtol=1e-14)
    np.testing.assert_allclose(out[0, 0, 0, 1:3], probs[0, 0, 0], rtol=1e-14)


def test_huge_softcap_is_identity():
    q, k, v = _rand((1, 11, 2, 16), 21), _rand((1, 11, 2, 16), 22), _rand((1, 11, 2, 16), 23)
    out, _, _ = ora.attention(q, k, v, 0.25, True, softcap=1e7)
    np.testing.assert_allclose(out, _sdpa(q, k, v, True, 0.25), atol=1e-10)


def test_uniform_and_single_key_and_empty_rows():
    k, v = _rand((1, 8, 1, 4), 24), _rand((1, 8, 1, 4), 25)
    q = np.zeros((1, 8, 1, 4))
    # q = 0: uniform over the visible keys (causal: keys 0..i)
    out, lse, _ = ora.attention(q, k, v, causal=True)
    for i in range(8):
        np.testing.assert_allclose(out[0, i, 0], v[0, :i + 1, 0].mean(0), atol=1e-14)
        np.testing.assert_allclose(lse[0, 0, i], math.log(i + 1), atol=1e-14)
    # window (0, 0): every row sees only its own key
    q2 = _rand((1, 8, 1, 4), 26)
    out, lse, _ = ora.attention(q2, k, v, 0.5, window_size=(0, 0))
    np.testing.assert_allclose(out[0, :, 0], v[0, :, 0], atol=1e-14)
    np.testing.assert_allclose(lse[0, 0], 0.5 * np.einsum("sd,sd->s", q2[0, :, 0], k[0, :, 0]),
                               atol=1e-14)
    # causal with negative offset: the first rows see nothing -> out 0, lse -inf
    out, lse, probs = ora.attention(q2, k, v, causal=True, causal_offset=-3)
    assert np.all(out[0, :3] == 0) and np.all(np.isneginf(lse[0, 0, :3]))
    assert np.all(probs[0, 0, :3] == 0)


def _brute(q, k, v, scale, causal, window, softcap, slopes, offset):
    """Pure-Python loops: one score at a time, in the documented pipeline order."""
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    out = [[[[0.0] * D for _ in range(H)] for _ in range(Sq)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            kh = h // (H // Hk)
            for i in range(Sq):
                qp = i + offset
                scores = []
                for j in range(Sk):
                    ok = (not causal or qp >= j) and (window[0] < 0 or j >= qp - window[0]) \
                        and (window[1] < 0 or j <= qp + window[1])
                    if not ok:
                        continue
                    s = sum(float(q[b, i, h, d]) * float(k[b, j, kh, d]) for d in range(D)) * scale
                    if slopes is not None:
                        s -= float(slopes[b][h]) * abs(qp - j)
                    if softcap > 0:
                        s = softcap * math.tanh(s / softcap)
                    scores.append((j, s))
                if not scores:
                    continue
                m = max(s for _, s in scores)
                z = sum(math.exp(s - m) for _, s in scores)
                for d in range(D):
                    out[b][i][h][d] = sum(math.exp(s - m) / z * float(v[b, j, kh, d]) for j, s in scores)
    return np.array(out)


@pytest.mark.parametrize("case", range(4))
def test_brute_force_all_features(case):
    rng = np.random.default_rng(100 + case)
    B, Sq, Sk, H, Hk, D = 2, [5, 6, 4, 6][case], [5, 4, 7, 6][case], 4, [4, 2, 1, 2][case], 4
    q, k, v = rng.standard_normal((B, Sq, H, D)), rng.standard_normal((B, Sk, Hk, D)), \
        rng.standard_normal((B, Sk, Hk, D))
    causal = case % 2 == 1
    window = [(-1, -1), (2, 1), (1, -1), (3, 0)][case]
    softcap = [0.0, 0.7, 2.0, 0.3][case]
    slopes = rng.random((B, H)) * 0.5
    offset = [0, 1, 0, 2][case]
    out, _, _ = ora.attention(q * 1.5, k, v, 0.6, causal, window, softcap, slopes,
                              causal_offset=offset)
    ref = _brute(q * 1.5, k, v, 0.6, causal, window, softcap, slopes, offset)
    np.testing.assert_allclose(out, ref, atol=1e-12)


def test_alibi_is_applied_before_softcap():
    # The two orders disagree on this input; the reference adds ALiBi to the
    # score before softcap (flash_attn_interface.py:36-42, kernel :308-314).
    q = np.full((1, 1, 1, 1), 3.0)
    k = np.array([[[[1.0]], [[1.0]]]])
    v = np.array([[[[0.0]], [[1.0]]]])
    slopes = np.array([2.0])
    out, _, _ = ora.attention(q, k, v, 1.0, False, softcap=1.0, alibi_slopes=slopes,
                              causal_offset=0)
    # key 0: |0-0| = 0 -> tanh(3); key 1: |0-1| = 1 -> tanh(3 - 2) = tanh(1)
    a, b = math.tanh(3.0), math.tanh(1.0)
    expected = math.exp(b) / (math.exp(a) + math.exp(b))
    np.testing.assert_allclose(out[0, 0, 0, 0], expected, rtol=1e-14)


# ----------------------------------------------------------------- varlen / kv-cache
def test_varlen_matches_per_sequence_sdpa():
    # Reference tests/test_compare_implementations.py:140-159.
    lq, lk = [3, 5], [4, 6]
    q, k, v = _rand((8, 2, 16), 30), _rand((10, 2, 16), 31), _rand((10, 2, 16), 32)
    out, lse = ora.attention_varlen(q, k, v, [0, 3, 8], [0, 4, 10], causal=True)
    exp = np.concatenate([
        _sdpa(q[None, 0:3], k[None, 0:4], v[None, 0:4], True)[0],
        _sdpa(q[None, 3:8], k[None, 4:10], v[None, 4:10], True)[0]])
    np.testing.assert_allclose(out, exp, atol=1e-12)
    assert lse.shape == (8, 2)


def test_varlen_empty_sequences():
    q, k, v = _rand((5, 1, 4), 33), _rand((3, 1, 4), 34), _rand((3, 1, 4), 35)
    out, lse = ora.attention_varlen(q, k, v, [0, 0, 5], [0, 3, 3])
    # second sequence has 5 queries and no keys: zeros and -inf
    assert np.all(out == 0) and np.all(np.isneginf(lse))


def test_paged_gather_is_the_contiguous_sequence():
    rng = np.random.default_rng(40)
    page, L = 4, 11
    contiguous = rng.standard_normal((L, 2, 8))
    n_pages = 5
    perm = rng.permutation(n_pages)
    cache = rng.standard_normal((n_pages, page, 2, 8))
    for t in range(L):
        cache[perm[t // page], t % page] = contiguous[t]
    np.testing.assert_array_equal(ora.gather_paged_kv(cache, perm, L), contiguous)


def test_compact_varlen_paged_rebuilds_the_packed_keys():
    # Sequences written token by token into shuffled pages come back packed.
    rng = np.random.default_rng(42)
    page, lengths = 4, [5, 0, 9]
    packed = rng.standard_normal((sum(lengths), 2, 8))
    cache = rng.standard_normal((8, page, 2, 8))
    perm = rng.permutation(8)
    bt = np.zeros((3, 3), dtype=np.int64)
    used, start = 0, 0
    for b, L in enumerate(lengths):
        n = (L + page - 1) // page
        bt[b, :n] = perm[used:used + n]
        for t in range(L):
            cache[bt[b, t // page], t % page] = packed[start + t]
        used += n
        start += L
    cu = np.array([0, 5, 5, 14])
    q = rng.standard_normal((3, 2, 8))
    _, k, v, cu_q, cu_k = ora.compact_varlen(q, cache, cache, [0, 1, 2, 3], cu, block_table=bt)
    np.testing.assert_array_equal(k, packed)
    np.testing.assert_array_equal(cu_k, cu)


def test_compact_varlen_seqused_is_truncated_per_sequence_sdpa():
    # seqused keeps each sequence's first rows: the result is SDPA of the
    # truncated slices, concatenated; full counts change nothing.
    lq, lk, uq, uk = [4, 6, 3], [5, 7, 2], [2, 6, 0], [5, 3, 1]
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    q, k, v = _rand((13, 2, 8), 43), _rand((14, 2, 8), 44), _rand((14, 2, 8), 45)
    cq2, ck2 = ora.compact_varlen(q, k, v, cq, ck, lq, lk)[3:]
    np.testing.assert_array_equal(cq2, cq)
    np.testing.assert_array_equal(ck2, ck)
    out, _ = ora.attention_varlen(*ora.compact_varlen(q, k, v, cq, ck, uq, uk), causal=True)
    exp = []
    for b in range(3):
        qb = q[None, cq[b]:cq[b] + uq[b]]
        if uq[b] == 0:
            continue
        exp.append(_sdpa(qb, k[None, ck[b]:ck[b] + uk[b]], v[None, ck[b]:ck[b] + uk[b]], True)[0])
    np.testing.assert_allclose(out, np.concatenate(exp), atol=1e-12)
    assert out.shape[0] == sum(uq)


# ----------------------------------------------------------------- gradients
def _torch_math(q, k, v, scale, causal, window, softcap, slopes, offset, bias=None):
    """The reference's math path (flash_attn_interface.py:15-49) in float64 torch,
    for autograd: BSHD inputs, GQA by repeat_interleave."""
    rep = q.shape[2] // k.shape[2]
    k = k.repeat_interleave(rep, dim=2)
    v = v.repeat_interleave(rep, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) * scale
    qp = torch.arange(q.shape[1], dtype=torch.float64)[:, None] + offset
    kp = torch.arange(k.shape[1], dtype=torch.float64)[None, :]
    if slopes is not None:
        s = s - slopes[None, :, None, None] * (qp - kp).abs()
    if bias is not None:
        s = s + bias
    if softcap > 0:
        s = softcap * torch.tanh(s / softcap)
    keep = torch.ones_like(qp * kp, dtype=torch.bool)
    if causal:
        keep &= qp >= kp
    if window[0] >= 0:
        keep &= kp >= qp - window[0]
    if window[1] >= 0:
        keep &= kp <= qp + window[1]
    p = torch.nan_to_num(torch.softmax(s.masked_fill(~keep, float("-inf")), dim=-1))
    return torch.einsum("bhqk,bkhd->bqhd", p, v)


@pytest.mark.parametrize("case", [
    dict(causal=False, window=(-1, -1), softcap=0.0, alibi=False, offset=0, sq=9, sk=9),
    dict(causal=True, window=(-1, -1), softcap=0.0, alibi=False, offset=0, sq=9, sk=12),
    dict(causal=True, window=(3, 0), softcap=5.0, alibi=True, offset=3, sq=7, sk=10),
    dict(causal=False, window=(2, 1), softcap=2.0, alibi=True, offset=0, sq=8, sk=8),
])
def test_backward_matches_torch_autograd(case):
    rng = np.random.default_rng(50)
    B, Hq, Hk, D = 2, 4, 2, 8
    q = rng.standard_normal((B, case["sq"], Hq, D))
    k = rng.standard_normal((B, case["sk"], Hk, D))
    v = rng.standard_normal((B, case["sk"], Hk, D))
    do = rng.standard_normal((B, case["sq"], Hq, D))
    slopes = rng.uniform(0.1, 0.9, Hq) if case["alibi"] else None
    tq, tk, tv = (torch.from_numpy(x).requires_grad_() for x in (q, k, v))
    out = _torch_math(tq, tk, tv, 0.3, case["causal"], case["window"], case["softcap"],
                      None if slopes is None else torch.from_numpy(slopes), case["offset"])
    out.backward(torch.from_numpy(do))
    got = ora.attention_backward(q, k, v, do, 0.3, case["causal"], case["window"],
                                 case["softcap"], slopes, case["offset"])
    for g, t in zip(got, (tq, tk, tv)):
        np.testing.assert_allclose(g, t.grad.numpy(), atol=1e-12)


@pytest.mark.parametrize("shape", [(2, 4, 7, 10), (1, 4, 7, 10), (2, 1, 1, 10), (7, 10),
                                   (4, 1, 10)])
def test_backward_bias_gradient_matches_torch_autograd(shape):
    # attn_bias broadcast over batch / heads / rows: autograd sums dS over the
    # broadcast dims; with softcap the bias sits inside the tanh.
    rng = np.random.default_rng(52)
    B, Sq, Sk, Hq, Hk, D = 2, 7, 10, 4, 2, 8
    q = rng.standard_normal((B, Sq, Hq, D))
    k = rng.standard_normal((B, Sk, Hk, D))
    v = rng.standard_normal((B, Sk, Hk, D))
    do = rng.standard_normal((B, Sq, Hq, D))
    bias = rng.standard_normal(shape)
    for causal, softcap in ((True, 0.0), (False, 4.0)):
        tq, tk, tv, tb = (torch.from_numpy(x).requires_grad_() for x in (q, k, v, bias))
        out = _torch_math(tq, tk, tv, 0.3, causal, (-1, -1), softcap, None, 3, tb)
        out.backward(torch.from_numpy(do))
        got = ora.attention_backward(q, k, v, do, 0.3, causal, (-1, -1), softcap, None, 3,
                                     attn_bias=bias, return_dbias=True)
        assert got[3].shape == bias.shape
        for g, t in zip(got, (tq, tk, tv, tb)):
            np.testing.assert_allclose(g, t.grad.numpy(), atol=1e-12)


def test_backward_matches_finite_differences():
    # d/dx of sum(out * dout) by central differences, every input element.
    rng = np.random.default_rng(51)
    q, k, v = rng.standard_normal((1, 4, 2, 4)), rng.standard_normal((1, 5, 1, 4)), \
        rng.standard_normal((1, 5, 1, 4))
    do = rng.standard_normal((1, 4, 2, 4))
    kw = dict(softmax_scale=0.7, causal=True, window_size=(2, -1), softcap=3.0,
              alibi_slopes=np.array([0.25, 0.5]), causal_offset=1)
    grads = ora.attention_backward(q, k, v, do, **kw)
    f = lambda a, b, c: float(np.sum(ora.attention(a, b, c, **kw)[0] * do))
    h = 1e-6
    for idx, x in enumerate((q, k, v)):
        num = np.zeros_like(x)
        for pos in np.ndindex(x.shape):
            args = [q.copy(), k.copy(), v.copy()]
            args[idx][pos] += h
            fp = f(*args)
            args[idx][pos] -= 2 * h
            num[pos] = (fp - f(*args)) / (2 * h)
        np.testing.assert_allclose(grads[idx], num, atol=1e-7)


def test_varlen_backward_is_per_sequence_backward():
    rng = np.random.default_rng(52)
    q, k, v = rng.standard_normal((9, 2, 8)), rng.standard_normal((11, 2, 8)), \
        rng.standard_normal((11, 2, 8))
    do = rng.standard_normal((9, 2, 8))
    dq, dk, dv = ora.attention_varlen_backward(q, k, v, do, [0, 4, 4, 9], [0, 5, 6, 11],
                                               causal=True)
    g0 = ora.attention_backward(q[None, :4], k[None, :5], v[None, :5], do[None, :4], causal=True)
    g2 = ora.attention_backward(q[None, 4:], k[None, 6:], v[None, 6:], do[None, 4:], causal=True)
    np.testing.assert_allclose(dq, np.concatenate([g0[0][0], g2[0][0]]), atol=1e-14)
    np.testing.assert_allclose(dk, np.concatenate([g0[1][0], np.zeros((1, 2, 8)), g2[1][0]]),
                               atol=1e-14)
    np.testing.assert_allclose(dv[5], 0.0)


# ----------------------------------------------------------------- dropout
def test_philox_known_answers():
    # Random123 known-answer vectors for philox4x32, 10 rounds.
    kat = [((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
           ((0xffffffff,) * 4, (0xffffffff, 0xffffffff),
            (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
           ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
            (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1))]
    for ctr, key, want in kat:
        got = ora.philox4x32_10(np.array([ctr], dtype=np.uint64), key)[0]
        assert tuple(int(x) for x in got) == want


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_dropout_keep_rate_and_scale(p):
    f = ora.dropout_factors(1234, p, [0, 1], 4, 256, 256)
    kept = f > 0
    n = kept.size
    # Binomial: the kept fraction lies within 6 standard deviations of 1 - p.
    assert abs(kept.mean() - (1 - p)) < 6 * math.sqrt(p * (1 - p) / n)
    t16 = round(float(np.float32(p)) * 65536)
    np.testing.assert_allclose(f[kept], 65536.0 / (65536 - t16), rtol=1e-15)
    # The kept scale is within 2^-17 / (1 - p) of the reference's 1 / (1 - p).
    assert abs(f[kept][0] * (1 - float(np.float32(p))) - 1) <= 2 ** -17 / (1 - p) + 1e-12
    # Every (batch, head) draws its own mask: masks of different heads agree
    # on about p^2 + (1-p)^2 of the elements, not on all of them.
    agree = (kept[0, 0] == kept[1, 3]).mean()
    assert abs(agree - (p * p + (1 - p) ** 2)) < 0.01


@pytest.mark.parametrize("p", [1e-7, 2.0 ** -17, 3e-5, 0.25, 1 - 2.0 ** -12, 1 - 2.0 ** -16,
                               1 - 2.0 ** -18])
def test_dropout_mask_is_unbiased(p):
    # E[factor] = keep probability x kept scale must be exactly 1 for every
    # p the 16-bit draws can express, including the extremes: p below
    # 2^-17 keeps everything at scale 1, p = 1 - 2^-16 keeps one draw value
    # in 65536 at scale 65536, and so does p = 1 - 2^-18, whose threshold
    # would round to 65536 (nothing kept) and stops at 65535.
    t16 = min(65535, round(float(np.float32(p)) * 65536))
    f = ora.dropout_factors(99, p, [0, 1, 2, 3], 8, 128, 256)
    kept = f > 0
    if t16 == 0:
        np.testing.assert_array_equal(f, 1.0)
        return
    scale = f[kept].max() if kept.any() else 65536.0 / (65536 - t16)
    np.testing.assert_array_equal(f[kept], scale)
    assert scale * (65536 - t16) == 65536.0
    # The kept fraction is the keep probability (binomial, 6 sigma).
    q_keep = (65536 - t16) / 65536
    n = f.size
    assert abs(kept.mean() - q_keep) <= 6 * math.sqrt(q_keep * (1 - q_keep) / n) + 1.0 / n


def test_dropout_p_near_one_keeps_one_draw_value():
    # p = 1 - 2^-18 would round to t16 = 65536 (nothing kept); the threshold
    # stops at 65535, the threshold of p = 1 - 2^-16, so both give one mask.
    a = ora.dropout_factors(1, 1 - 2.0 ** -18, [0, 1], 4, 256, 256)
    b = ora.dropout_factors(1, 1 - 2.0 ** -16, [0, 1], 4, 256, 256)
    np.testing.assert_array_equal(a, b)
    assert set(np.unique(a)) <= {0.0, 65536.0}


def test_dropout_mask_is_seed_dependent_and_p0_is_identity():
    a = ora.dropout_factors(1, 0.5, [0], 2, 64, 64)
    b = ora.dropout_factors(2, 0.5, [0], 2, 64, 64)
    assert 0.4 < (a == b).mean() < 0.6
    np.testing.assert_array_equal(ora.dropout_factors(1, 0.0, [0], 2, 64, 64), 1.0)
    rng = np.random.default_rng(53)
    q, k, v = (rng.standard_normal((1, 20, 2, 8)) for _ in range(3))
    np.testing.assert_array_equal(ora.attention(q, k, v)[0],
                                  ora.attention(q, k, v, dropout_p=0.0, dropout_seed=9)[0])


def test_dropout_known_answer_single_key():
    # Reference tests/test_compare_implementations.py:161-168: q = k = 0,
    # v = 1, one key: the output is 1 / (1 - p) where kept, 0 where dropped.
    q = np.zeros((1, 1, 1, 16))
    v = np.ones((1, 1, 1, 16))
    seen = set()
    for seed in range(64):
        out = ora.attention(q, q, v, dropout_p=0.5, dropout_seed=seed)[0]
        assert np.all(out == out.flat[0]) and out.flat[0] in (0.0, 2.0)
        seen.add(float(out.flat[0]))
    assert seen == {0.0, 2.0}


def test_dropout_backward_matches_finite_differences():
    rng = np.random.default_rng(54)
    q, k, v = (rng.standard_normal((1, 6, 2, 4)) for _ in range(3))
    do = rng.standard_normal((1, 6, 2, 4))
    kw = dict(softmax_scale=0.6, causal=True, softcap=4.0, dropout_p=0.3, dropout_seed=77)
    grads = ora.attention_backward(q, k, v, do, **kw)
    f = lambda a, b, c: float(np.sum(ora.attention(a, b, c, **kw)[0] * do))
    h = 1e-6
    for idx, x in enumerate((q, k, v)):
        num = np.zeros_like(x)
        for pos in np.ndindex(x.shape):
            args = [q.copy(), k.copy(), v.copy()]
            args[idx][pos] += h
            fp = f(*args)
            args[idx][pos] -= 2 * h
            num[pos] = (fp - f(*args)) / (2 * h)
        np.testing.assert_allclose(grads[idx], num, atol=1e-7)


@pytest.mark.parametrize("causal", [False, True])
def test_kvcache_decode_matches_sdpa_bottom_right(causal):
    rng = np.random.default_rng(41)
    page, Sq, Hq, Hk, D = 4, 3, 4, 2, 8
    lengths = [9, 5]
    kc = rng.standard_normal((8, page, Hk, D))
    vc = rng.standard_normal((8, page, Hk, D))
    bt = np.array([[3, 0, 6], [5, 1, 2]])
    q = rng.standard_normal((2, Sq, Hq, D))
    out, _, _, _ = ora.attention_kvcache(q, kc, vc, cache_seqlens=lengths, block_table=bt,
                                         causal=causal)
    for b, L in enumerate(lengths):
        kb = ora.gather_paged_kv(kc, bt[b], L)[None]
        vb = ora.gather_paged_kv(vc, bt[b], L)[None]
        mask = torch.ones(Sq, L, dtype=torch.bool).tril(diagonal=L - Sq) if causal else None
        exp = _sdpa(q[b:b + 1], kb, vb, mask=mask, gqa=True, scale=1 / math.sqrt(D))
        np.testing.assert_allclose(out[b:b + 1], exp, atol=1e-12)


def test_kvcache_append_then_attend():
    rng = np.random.default_rng(42)
    kc = rng.standard_normal((2, 10, 1, 4))
    vc = rng.standard_normal((2, 10, 1, 4))
    kn, vn = rng.standard_normal((2, 2, 1, 4)), rng.standard_normal((2, 2, 1, 4))
    q = rng.standard_normal((2, 2, 1, 4))
    out, _, kc2, vc2 = ora.attention_kvcache(q, kc, vc, cache_seqlens=[3, 7], k_new=kn, v_new=vn,
                                             causal=True)
    np.testing.assert_array_equal(kc2[0, 3:5], kn[0])
    np.testing.assert_array_equal(kc2[1, 7:9], kn[1])
    np.testing.assert_array_equal(vc2[1, 7:9], vn[1])
    np.testing.assert_array_equal(kc2[0, :3], kc[0, :3])
    exp = _sdpa(q[:1], kc2[:1, :5], vc2[:1, :5],
                mask=torch.ones(2, 5, dtype=torch.bool).tril(diagonal=3))
    np.testing.assert_allclose(out[:1], exp, atol=1e-12)


@pytest.mark.parametrize("interleaved", [True, False])
def test_rotary_is_a_complex_rotation(interleaved):
    rng = np.random.default_rng(43)
    S, H, D, R = 5, 2, 8, 6
    x = rng.standard_normal((S, H, D))
    theta = rng.standard_normal((10, R // 2))
    pos = np.array([0, 3, 9, 4, 1])
    out = ora.apply_rotary(x, np.cos(theta), np.sin(theta), pos, interleaved)
    if interleaved:
        z = x[..., 0:R:2] + 1j * x[..., 1:R:2]
    else:
        z = x[..., :R // 2] + 1j * x[..., R // 2:R]
    zr = z * np.exp(1j * theta[pos])[:, None, :]
    if interleaved:
        np.testing.assert_allclose(out[..., 0:R:2], zr.real, atol=1e-14)
        np.testing.assert_allclose(out[..., 1:R:2], zr.imag, atol=1e-14)
    else:
        np.testing.assert_allclose(out[..., :R // 2], zr.real, atol=1e-14)
        np.testing.assert_allclose(out[..., R // 2:R], zr.imag, atol=1e-14)
    np.testing.assert_array_equal(out[..., R:], x[..., R:])


# ----------------------------------------------------------------- quantizer
def _f32(x: Fraction) -> Fraction:
    """Round an exact rational to the nearest binary32 value (ties to even)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


def _exact_quant_row(row, divide: bool):
    """Quantizer on exact rationals with explicit binary32 rounding after each op."""
    vals = [Fraction(float(x)) for x in row]
    amax = max(abs(x) for x in vals)
    s = _f32(max(amax, Fraction(1)) / 127)
    inv = _f32(1 / s)
    out = []
    for x in vals:
        y = _f32(x / s) if divide else _f32(x * inv)
        if y >= 0:
            t = _f32(y + Fraction(1, 2))
            r = t.numerator // t.denominator
        else:
            t = _f32(y - Fraction(1, 2))
            r = -((-t.numerator) // t.denominator)
        out.append(int(r))
    return out, float(s)


def _known_rows(D=32):
    rng = np.random.default_rng(50)
    rows = [np.zeros(D), np.linspace(-0.9, 0.9, D), rng.standard_normal(D),
            rng.standard_normal(D) * 8.0, np.full(D, 1.0), rng.standard_normal(D) * 300.0]
    tie = np.zeros(D)
    tie[0], tie[1], tie[2], tie[3] = 127.0, 0.5, -0.5, 2.5     # s = 1 exactly: x.5 ties
    rows.append(tie)
    return np.stack(rows).astype(np.float16)


def test_round_half_away_known_answers():
    x = np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, -0.49999997, 0.0, 126.5], np.float32)
    got = quant.round_half_away(x)
    # 0.49999997 + 0.5 rounds to 1.0 in binary32 (ties-to-even), so floor gives 1.
    np.testing.assert_array_equal(got, [1, -1, 2, 3, -3, 1, -1, 0, 127])


@pytest.mark.parametrize("divide", [False, True])
def test_quantizer_matches_exact_arithmetic(divide):
    rows = _known_rows()
    q8, s = (quant.quantize_q_rows if divide else quant.quantize_k_rows)(rows)
    for r, row in enumerate(rows):
        exp8, exp_s = _exact_quant_row(row, divide)
        assert q8[r].tolist() == exp8, f"row {r}"
        assert float(s[r]) == exp_s
    # known values: zero row -> scale 1/127, all zeros; the tie row has s = 1
    assert np.all(q8[0] == 0) and s[0] == np.float32(1.0) / np.float32(127.0)
    assert s[6] == 1.0 and q8[6][:4].tolist() == [127, 1, -1, 3]


def _c_oracle():
    lib = os.path.join(ROOT, "oracle", "libfa_oracle.so")
    if not os.path.exists(lib):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True,
                       capture_output=True)
    c = ctypes.CDLL(lib)
    for name in ("oracle_quantize_k_rows_f16", "oracle_quantize_q_rows_f16"):
        getattr(c, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.c_int64]
    return c


@pytest.mark.parametrize("divide", [False, True])
def test_numpy_and_c_quantizers_agree(divide):
    rng = np.random.default_rng(51)
    x = (rng.standard_normal((4000, 128)) * rng.choice([0.3, 1, 8, 100], (4000, 1))).astype(np.float16)
    x[:10] = _known_rows(128)[:7].repeat(2, axis=0)[:10]
    c = _c_oracle()
    k8 = np.empty(x.shape, np.int8)
    s = np.empty(x.shape[0], np.float32)
    fn = c.oracle_quantize_q_rows_f16 if divide else c.oracle_quantize_k_rows_f16
    fn(x.ctypes.data, k8.ctypes.data, s.ctypes.data, x.shape[0], x.shape[1])
    n8, ns = (quant.quantize_q_rows if divide else quant.quantize_k_rows)(x)
    np.testing.assert_array_equal(k8, n8)
    np.testing.assert_array_equal(s.view(np.uint32), ns.view(np.uint32))


def test_quantized_values_are_bounded_and_close():
    x = (np.random.default_rng(52).standard_normal((500, 64)) * 5).astype(np.float16)
    k8, s = quant.quantize_k_rows(x)
    assert np.abs(k8.astype(int)).max() <= 127
    err = np.abs(k8 * s[:, None].astype(np.float64) - x.astype(np.float64))
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-6))


def test_int8_attention_exact_when_quantization_is_lossless():
    # Integer-valued rows with amax 127 quantize with s = 1 exactly, so the INT8
    # oracle equals the float attention oracle on the same inputs.
    rng = np.random.default_rng(53)
    B, H, S, D = 1, 2, 8, 32
    q = rng.integers(-127, 128, (B, H, S, D)).astype(np.float16)
    k = rng.integers(-127, 128, (B, H, S, D)).astype(np.float16)
    q[..., 0] = 127
    k[..., 0] = -127
    v = rng.standard_normal((B, H, S, D))
    for causal in (False, True):
        o8, l8 = quant.attention_int8(q, k, v, causal, sm_scale=1e-3)
        of, lf, _ = ora.attention(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                                  v.transpose(0, 2, 1, 3), 1e-3, causal)
        np.testing.assert_allclose(o8, of.transpose(0, 2, 1, 3), atol=1e-12)
        np.testing.assert_allclose(l8, lf, atol=1e-12)


def test_round_half_away_trunc_form_matches_definition():
    # The GPU quantizers round with trunc(x + copysign(0.5, x)); the
    # reference's _round_i8 is x >= 0 ? floor(x + 0.5) : ceil(x - 0.5)
    # (attention_kernel_int8.py:27-39).  In fp32 arithmetic both take the same
    # single addition, so they agree bit for bit; checked on ties, signed
    # zeros, values just around ties and 10^6 random values over 12 binades.
    rng = np.random.default_rng(7)
    mags = np.float32(2.0) ** rng.uniform(-6, 6, 1_000_000).astype(np.float32)
    x = (mags * rng.choice(np.array([-1, 1], np.float32), mags.size)).astype(np.float32)
    ties = (np.arange(-200, 200, dtype=np.float32) + np.float32(0.5))
    near = np.concatenate([np.nextafter(ties, np.float32(np.inf)), np.nextafter(ties, np.float32(-np.inf))])
    special = np.array([0.0, -0.0, 0.49999997, -0.49999997, 127.0, -127.0, 126.5, -126.5],
                       dtype=np.float32)
    x = np.concatenate([x, ties, near, special]).astype(np.float32)
    half = np.float32(0.5)
    ref = np.where(x >= 0, np.floor(x + half), np.ceil(x - half)).astype(np.float32)
    got = np.trunc((x + np.copysign(half, x)).astype(np.float32)).astype(np.float32)
    assert np.array_equal(ref.view(np.uint32) & 0x7FFFFFFF, got.view(np.uint32) & 0x7FFFFFFF)
    assert np.array_equal(ref, got)
