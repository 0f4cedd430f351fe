"""INT8-QK path on the GPU: byte-exact K quantization and attention parity."""
import math

import numpy as np
import pytest
import torch

from _helpers import INT8_ATOL, assert_close, randn, to_np
from oracle import attention as ora
from oracle import quant

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _outlier_k(B, H, S, D, seed):
    """K ~ N(0,1) fp16 with 1% of token rows scaled x8."""
    k = randn((B, H, S, D), seed)
    gen = torch.Generator().manual_seed(seed + 1000)
    n_out = max(1, S // 100)
    for b in range(B):
        for h in range(H):
            rows = torch.randperm(S, generator=gen)[:n_out]
            k[b, h, rows] = (k[b, h, rows].float() * 8.0).half()
    return k


@pytest.mark.parametrize("head_dim", [32, 64, 128, 256])
def test_quant_k_byte_exact(head_dim):
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import quantize_k_int8
    k = _outlier_k(2, 3, 320, head_dim, 5)
    # add rows that hit the clamp, exact zeros and x.5 ties
    k[0, 0, 0] = 0
    k[0, 0, 1] = torch.linspace(-0.9, 0.9, head_dim).half()
    # amax 127 gives s = 1 exactly: every j + 0.5 is a tie, rounded away from
    # zero; signed zeros quantize to 0.
    ties = torch.arange(head_dim, dtype=torch.float32) - head_dim / 2 + 0.5
    ties[0], ties[1], ties[2] = 127.0, -0.0, 0.0
    k[1, 2, 5] = ties.half()
    k8, s_k = quantize_k_int8(k.to(DEV))
    torch.cuda.synchronize()
    ref8, refs = quant.quantize_k_rows(k.numpy().reshape(-1, 320, head_dim))
    assert np.array_equal(k8.cpu().numpy(), ref8)
    assert np.array_equal(s_k.cpu().numpy().view(np.uint32), refs.view(np.uint32))


@pytest.mark.parametrize("seqlen", [100, 63, 1])
def test_quant_k_lengths_not_multiple_of_64(seqlen):
    # The row-per-thread prepass (lengths that are not a multiple of 64).
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import quantize_k_int8
    k = _outlier_k(2, 3, seqlen, 128, 11)
    k8, s_k = quantize_k_int8(k.to(DEV))
    torch.cuda.synchronize()
    ref8, refs = quant.quantize_k_rows(k.numpy().reshape(-1, seqlen, 128))
    assert np.array_equal(k8.cpu().numpy(), ref8)
    assert np.array_equal(s_k.cpu().numpy().view(np.uint32), refs.view(np.uint32))


def test_quant_k_strided_input():
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import quantize_k_int8
    base = _outlier_k(2, 128, 4, 64, 9)            # [B, S, H, D] storage
    k = base.transpose(1, 2)                        # [B, H, S, D] view
    k8, s_k = quantize_k_int8(k.to(DEV))
    ref8, refs = quant.quantize_k_rows(k.contiguous().numpy().reshape(-1, 128, 64))
    assert np.array_equal(k8.cpu().numpy(), ref8)
    assert np.array_equal(s_k.cpu().numpy(), refs)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_int8_attention(causal, head_dim):
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import attention_int8
    B, H, S = 2, 2, 384
    q = randn((B, H, S, head_dim), 1)
    k = _outlier_k(B, H, S, head_dim, 2)
    v = randn((B, H, S, head_dim), 3)
    out = attention_int8(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal).cpu()
    # Parity bar: the INT8-QK semantics (per-token quantized Q and K, exact
    # integer QK^T, float64 softmax and PV) at 2e-2.
    ref, _ = quant.attention_int8(q.numpy(), k.numpy(), to_np(v), causal=causal)
    assert_close(to_np(out), ref, INT8_ATOL, "int8 vs INT8-semantics oracle", torch.float16)
    # The scheme itself moves the result away from unquantized attention: with
    # x8 outlier keys the oracle-vs-oracle distance reaches ~0.2 on some rows.
    # The kernel must not add to it beyond the fp16 bar.
    ref_f, _, _ = ora.attention(to_np(q.transpose(1, 2)), to_np(k.transpose(1, 2)),
                                to_np(v.transpose(1, 2)), causal=causal)
    scheme = np.abs(ref - ref_f.transpose(0, 2, 1, 3))
    kernel = np.abs(to_np(out) - ref_f.transpose(0, 2, 1, 3))
    assert np.max(kernel - scheme) <= 2e-3 + 1e-3


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lens", [(200, 250), (320, 128), (64, 320), (1, 320)])
def test_int8_partial_lengths(causal, lens):
    # seq_len_k masks keys >= seq_len_k (zero-filled past the end of a tile) and
    # places query row i at i + seq_len_k - seq_len_q; rows before the first
    # visible key come out as zeros.
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import attention_int8
    B, H, S, D = 1, 3, 320, 128
    q = randn((B, H, S, D), 11)
    k = _outlier_k(B, H, S, D, 12)
    v = randn((B, H, S, D), 13)
    out = attention_int8(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, seq_len_k=lens[0],
                         seq_len_q=lens[1]).cpu()
    ref, _ = quant.attention_int8(q.numpy(), k.numpy(), to_np(v), causal=causal,
                                  seq_len_k=lens[0], seq_len_q=lens[1])
    assert_close(to_np(out), ref, INT8_ATOL, f"lens={lens}", torch.float16)


def test_int8_reference_case():
    # Reference tests/test_compare_implementations.py:222-235 (forward part):
    # B=2, S=128, H=2, D=64, scale 0.125, causal and not.
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import attention_int8
    q, k, v = (randn((2, 128, 2, 64), s) for s in (42, 43, 44))
    for causal in (False, True):
        out = attention_int8(*(t.transpose(1, 2).contiguous().to(DEV) for t in (q, k, v)),
                             causal=causal, sm_scale=0.125).transpose(1, 2).cpu()
        ref, _, _ = ora.attention(to_np(q), to_np(k), to_np(v), 0.125, causal)
        assert_close(to_np(out), ref, INT8_ATOL, f"causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
def test_int8_baseline_c3_sampled(causal):
    # B=4, H=32, S=4096, D=128, 1% outlier K rows; sampled rows.
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import (attention_int8,
                                                                      quantize_k_int8)
    B, H, S, D = 4, 32, 4096, 128
    q = randn((B, H, S, D), 4)
    k = randn((B, H, S, D), 5)
    gen = torch.Generator().manual_seed(6)
    for b in range(B):
        for h in range(H):
            rows = torch.randperm(S, generator=gen)[:41]
            k[b, h, rows] = (k[b, h, rows].float() * 8.0).half()
    v = randn((B, H, S, D), 7)
    kd = k.to(DEV)
    k8, s_k = quantize_k_int8(kd)
    ref8, refs = quant.quantize_k_rows(k.numpy().reshape(B * H, S, D))
    assert np.array_equal(k8.cpu().numpy(), ref8)
    assert np.array_equal(s_k.cpu().numpy(), refs)
    out = attention_int8(q.to(DEV), kd, v.to(DEV), causal=causal).cpu()
    rng = np.random.default_rng(3)
    for _ in range(24):
        b, h, i = int(rng.integers(B)), int(rng.integers(H)), int(rng.integers(S))
        ref, _ = quant.attention_int8(q[b:b + 1, h:h + 1, i:i + 1].numpy(),
                                      k[b:b + 1, h:h + 1].numpy(), to_np(v[b:b + 1, h:h + 1]),
                                      causal=causal, q_positions=[i])
        assert_close(to_np(out[b, h, i]), ref[0, 0, 0], INT8_ATOL, f"b={b} h={h} i={i}",
                     torch.float16)


def _int8_torch_reference(q8, s_q, k8, s_k, v, causal, scale):
    """The INT8-QK semantics in fp32 torch on the GPU for one batch of heads:
    q8/k8 [H, S, D] int8 values (as float32), s_q/s_k [H, S]; the integer dot
    products (|sum| <= 128 * 127^2 < 2^24) are exact in fp32."""
    qk = torch.matmul(q8, k8.transpose(1, 2).contiguous())
    sc = qk * (s_q[:, :, None] * s_k[:, None, :]) * scale
    if causal:
        S = sc.shape[-1]
        i = torch.arange(S, device=sc.device)
        sc.masked_fill_(i[None, :] > i[:, None], float("-inf"))
    return torch.matmul(torch.softmax(sc, dim=-1), v)


def _int8_every_row(B, H, S, causal, seed, label):
    # Every output row against the INT8 semantics in fp32 torch (Q quantized
    # by the oracle's fp32 restatement, K8 / s_k from the kernel's prepass,
    # which the sampled test above checks byte for byte); the torch reference
    # is checked against the float64 oracle first.  1 % of K's token rows are
    # scaled by 8 (per-token scale outliers).
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import (attention_int8,
                                                                      quantize_k_int8)
    D = 128
    scale = 1.0 / math.sqrt(D)
    q = randn((B, H, S, D), seed)
    k = randn((B, H, S, D), seed + 1)
    gen = torch.Generator().manual_seed(seed + 2)
    for b in range(B):
        for h in range(H):
            rows = torch.randperm(S, generator=gen)[:max(1, S // 100)]
            k[b, h, rows] = (k[b, h, rows].float() * 8.0).half()
    v = randn((B, H, S, D), seed + 3)
    kd = k.to(DEV)
    k8, s_k = quantize_k_int8(kd)
    out = attention_int8(q.to(DEV), kd, v.to(DEV), causal=causal)
    q8n, s_qn = quant.quantize_q_rows(q.numpy())
    q8 = torch.from_numpy(q8n.astype(np.float32)).to(DEV)
    s_q = torch.from_numpy(s_qn.astype(np.float32)).to(DEV)
    k8f = k8.to(torch.float32).reshape(B, H, S, D)
    s_kf = s_k.reshape(B, H, S)
    # The reference on one head's first 256 rows and keys against the oracle.
    small = _int8_torch_reference(q8[0, :1, :256], s_q[0, :1, :256], k8f[0, :1, :256],
                                  s_kf[0, :1, :256], v[0, :1, :256].to(DEV).float(), causal, scale)
    ora_small, _ = quant.attention_int8(q[0:1, 0:1, :256].numpy(), k[0:1, 0:1, :256].numpy(),
                                        to_np(v[0:1, 0:1, :256]), causal=causal)
    assert np.max(np.abs(to_np(small.cpu()) - ora_small[0])) < 1e-5
    vd = v.to(DEV).float()
    worst = 0.0
    for b in range(B):
        ref = _int8_torch_reference(q8[b], s_q[b], k8f[b], s_kf[b], vd[b], causal, scale)
        worst = max(worst, float((out[b].float() - ref).abs().max()))
        assert_close(to_np(out[b].cpu()), to_np(ref.cpu()), INT8_ATOL, f"int8 b={b}", torch.float16)
        del ref
    print(f"{label} causal={causal}: raw max-abs error {worst:.3e}")
    assert worst <= INT8_ATOL, f"{label}: raw max-abs error {worst:.3e} > 2e-2"


@pytest.mark.parametrize("causal", [True, False])
def test_int8_baseline_c3_every_row(causal):
    # BASELINE config 3 in full (the persistent INT8 kernel, eight row blocks
    # per workgroup).
    _int8_every_row(4, 32, 4096, causal, 4, "C3 full")


@pytest.mark.parametrize("causal", [True, False])
def test_int8_persistent_long_rows(causal):
    # A longer sequence on the persistent path: 32 (batch, head) groups of
    # 32 row blocks each (16 causal pairs), four rounds per workgroup.
    _int8_every_row(2, 16, 8192, causal, 60, "S=8192")


def _int8_grad_check(name, got, exact):
    # The reference's INT8 gradient bars against unquantized attention
    # (tests/test_compare_implementations.py:27-28, :221-235): the INT8
    # forward's output and LSE feed the fp16 dense backward.
    got = to_np(got.cpu())
    err = np.abs(got - exact)
    bound = 5e-2 + 2e-2 * np.abs(exact)
    print(f"int8 backward {name}: max-abs err {float(np.max(err)):.3e}")
    assert np.all(np.isfinite(got)) and np.all(err <= bound), (
        f"{name}: max |err| {float(np.max(err)):.3e}")


@pytest.mark.parametrize("causal", [False, True])
def test_int8_gradients(causal):
    # The reference's case: B2 H2 S128 D64, scale 0.125, two query and two
    # key blocks per head.
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import attention_int8
    q, k, v, do = (randn((2, 2, 128, 64), s) for s in (201, 202, 203, 204))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = attention_int8(qd, kd, vd, causal=causal, sm_scale=0.125)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    ref = ora.attention_backward(*(to_np(t.transpose(1, 2)) for t in (q, k, v, do)), 0.125, causal)
    for name, t, r in zip(("dq", "dk", "dv"), (qd, kd, vd), ref):
        _int8_grad_check(name, t.grad.transpose(1, 2), r)


def test_int8_gradients_with_short_key_length():
    # seq_len_k = 100 of 128 keys visible, query row i at position
    # i + seq_len_k - seq_len_q: keys 100.. get exactly zero gradients.
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import attention_int8
    q, k, v, do = (randn((1, 2, 128, 64), s) for s in (211, 212, 213, 214))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = attention_int8(qd, kd, vd, causal=True, seq_len_k=100, seq_len_q=128)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert torch.count_nonzero(kd.grad[:, :, 100:]) == 0
    assert torch.count_nonzero(vd.grad[:, :, 100:]) == 0
    ref = ora.attention_backward(*(to_np(t.transpose(1, 2)) for t in (q, k[:, :, :100], v[:, :, :100],
                                                                         do)),
                                 None, True, causal_offset=100 - 128)
    for name, t, r in zip(("dq", "dk", "dv"), (qd.grad, kd.grad[:, :, :100], vd.grad[:, :, :100]),
                          ref):
        _int8_grad_check(name, t.transpose(1, 2), r)
