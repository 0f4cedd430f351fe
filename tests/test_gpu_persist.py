"""Full-output parity of the persistent ping-pong prefill (large dense launches).

The persistent kernel runs one workgroup per CU over a list of row blocks
whose key tiles stream through one LDS ring, so a mistake at a block hand-over
(a stale Q row, O^T not cleared, a running max carried over, a tile of the
wrong block, an output written to the wrong rows) shows up in whole blocks.
These tests therefore check every output row and LSE of launches that take
the persistent path, against an fp32 torch reference computed on the GPU
(scores, mask, logsumexp, softmax, product with V; TF32 off), which is itself
checked against the float64 oracle on sampled rows.  Shapes: D = 128, B * H a
multiple of 8, sequence lengths a multiple of 512 (causal) / 256, and enough
row blocks for two or more per workgroup on a 256-CU MI355X.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import ATOL, assert_close, randn, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _torch_ref(q, k, v, causal, scale):
    """fp32 attention on the GPU: out [B, S, Hq, D] and natural-log LSE [B, Hq, S]."""
    torch.backends.cuda.matmul.allow_tf32 = False
    B, S, Hq, D = q.shape
    Hk = k.shape[2]
    qf = q.float().permute(0, 2, 1, 3).contiguous()
    kf = k.float().permute(0, 2, 1, 3).repeat_interleave(Hq // Hk, dim=1).contiguous()
    vf = v.float().permute(0, 2, 1, 3).repeat_interleave(Hq // Hk, dim=1).contiguous()
    out = torch.empty((B, Hq, S, D), dtype=torch.float32, device=q.device)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool, device=q.device), 1) if causal else None
    for b in range(B):
        s = torch.matmul(qf[b], kf[b].transpose(-1, -2).contiguous()) * scale
        if mask is not None:
            s.masked_fill_(mask, float("-inf"))
        lse[b] = torch.logsumexp(s, dim=-1)
        out[b] = torch.matmul(torch.softmax(s, dim=-1), vf[b])
        del s
    return out.permute(0, 2, 1, 3).contiguous(), lse


def _case(B, S, Hq, Hk, causal, dtype=torch.float16, seed=0, oracle_rows=6):
    from flash_attn_triton.triton_kernel.attention_kernel import dense_forward
    D = 128
    q = randn((B, S, Hq, D), seed + 1, dtype)
    k = randn((B, S, Hk, D), seed + 2, dtype)
    v = randn((B, S, Hk, D), seed + 3, dtype)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out, lse = dense_forward(qd, kd, vd, softmax_scale=scale, causal=causal, return_lse=True)
    ref_out, ref_lse = _torch_ref(qd, kd, vd, causal, scale)
    torch.cuda.synchronize()
    # The torch reference against the float64 oracle on a few rows.
    rng = np.random.default_rng(seed)
    ref_np = ref_out.cpu().numpy()
    for _ in range(oracle_rows):
        b, h, i = int(rng.integers(B)), int(rng.integers(Hq)), int(rng.integers(S))
        kh = h // (Hq // Hk)
        exp, _, _ = ora.attention(to_np(q[b:b + 1, i:i + 1, h:h + 1]), to_np(k[b:b + 1, :, kh:kh + 1]),
                                  to_np(v[b:b + 1, :, kh:kh + 1]), softmax_scale=scale,
                                  causal=causal, causal_offset=i)
        assert np.max(np.abs(ref_np[b, i, h] - exp[0, 0, 0])) < 1e-5, (b, h, i)
    got = to_np(out.cpu())
    err = float(np.max(np.abs(got - ref_np)))
    print(f"persistent B={B} S={S} Hq={Hq} Hk={Hk} causal={causal} {dtype}: max-abs err {err:.3e}")
    if dtype == torch.float16:
        # The north star's literal bar on the raw difference, output rounding
        # included (assert_close below allows half an fp16 ulp on top).
        assert err <= ATOL[dtype], f"raw max-abs error {err:.3e} > {ATOL[dtype]:.0e}"
    assert_close(got, ref_np, ATOL[dtype], "out (every row)", dtype)
    assert_close(lse.cpu().numpy(), ref_lse.cpu().numpy(), 1e-3, "lse (every row)")


@pytest.mark.parametrize("causal", [True, False])
def test_persistent_every_row(causal):
    # 64 groups x 8 row blocks: 32 causal pairs / 64 blocks per XCD, two row
    # blocks per workgroup.
    _case(4, 2048, 16, 16, causal, seed=10)


def test_persistent_gqa_bf16():
    _case(2, 2048, 32, 8, True, dtype=torch.bfloat16, seed=20)
    _case(2, 2048, 32, 8, False, dtype=torch.bfloat16, seed=30)


@pytest.mark.parametrize("causal", [True, False])
def test_persistent_baseline_config_c2_every_row(causal):
    # BASELINE config 2 at full size (B=4, H=32, S=4096, D=128): eight row
    # blocks per workgroup, every output row and LSE checked.
    _case(4, 4096, 32, 32, causal, seed=40)


@pytest.mark.parametrize("causal", [True, False])
def test_persistent_long_sequence(causal):
    # S = 8192: 32 row blocks per (batch, head) group, 16 groups, two rounds
    # per workgroup; causal pairs span 8192 keys.
    _case(1, 8192, 16, 16, causal, seed=50)


def test_persistent_causal_odd_groups_per_xcd():
    # 24 (batch, head) groups: 3 per XCD, an odd count, so the causal list
    # keeps both row blocks of a pair in one group (the two-group pairing
    # needs an even count); 24 workgroups per XCD, two row blocks each.
    _case(1, 4096, 24, 24, True, seed=60)



def test_persistent_causal_three_pairs_per_workgroup():
    # B=3, H=32, S=4096: 12 groups per XCD, 96 row-block pairs over 32
    # workgroups: three causal pairs (six row blocks) per workgroup.
    _case(3, 4096, 32, 32, True, seed=70)


def test_persistent_causal_gqa_bf16_long():
    # S = 8192: 32 row blocks per group, grouped KV heads, bf16.
    _case(2, 8192, 32, 8, True, dtype=torch.bfloat16, seed=80)


def test_persistent_causal_repeats_streams_and_graph():
    # Every row block is computed the same way whichever workgroup takes it
    # and whenever it runs: repeated launches, launches on two streams at
    # once, and replays of a captured graph (with eager launches between the
    # replays) give bitwise the same output and LSE.
    from flash_attn_triton.triton_kernel.attention_kernel import dense_forward
    B, S, H, D = 4, 4096, 32, 128
    q, k, v = (randn((B, S, H, D), s, torch.float16).to(DEV) for s in (91, 92, 93))
    scale = 1.0 / math.sqrt(D)

    def run():
        return dense_forward(q, k, v, softmax_scale=scale, causal=True, return_lse=True)

    out0, lse0 = run()
    for _ in range(3):
        out, lse = run()
        assert torch.equal(out, out0) and torch.equal(lse, lse0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    res = []
    for st in (s1, s2, s1, s2):
        with torch.cuda.stream(st):
            res.append(run())
    torch.cuda.synchronize()
    for out, lse in res:
        assert torch.equal(out, out0) and torch.equal(lse, lse0)
    del res
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, lse_g = run()
    for _ in range(3):
        out_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out0) and torch.equal(lse_g, lse0)
        out, lse = run()
        torch.cuda.synchronize()
        assert torch.equal(out, out0) and torch.equal(lse, lse0)
