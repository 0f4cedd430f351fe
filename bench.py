"""Benchmark of the gfx950 FlashAttention-2 forward (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--prewarm SECONDS] [--workload NAME]

A "step" is one call of the public entry point on one batch of synthetic
input already resident in HBM.  The default workload is BASELINE config 2,
the metric's headline shape: dense FP16 causal forward, B=4, H=32,
S_q=S_k=4096, D=128 (``flash_attn_func(q, k, v, causal=True)``).  Other
workloads (``--workload``): ``dense`` (same shape, non-causal),
``int8_causal`` / ``int8`` (config 3, ``attention_int8``, quantization
prepass included), ``decode`` (config 4, paged GQA decode through
``flash_attn_with_kvcache``), ``varlen`` (config 5) and ``bwd_causal`` /
``bwd`` (the backward of config 2: dq, dk, dv; 2.5 x the forward's FLOPs).

FLOP convention (reference README.md:226-229): causal 2*B*H*D*S*(S+1),
non-causal 4*B*H*D*S^2; varlen counts 4*H*D per unmasked (q, k) pair; decode
is measured in algorithmic bytes (K/V rows read + q + out + block table).

Before the W warmup steps every measurement runs untimed steps for
``--prewarm`` seconds (default 0.5) so that the timed steps see settled GPU
clocks; the line reports how many (``prewarm_steps``).  The timed region of
the whole-job value is exactly K steps, with nothing else between its two
synchronizations.

The JSON line carries ``roofline`` and ``cpu_baseline``.  ``roofline.achieved``
is the algorithmic work of one launch divided by the mean duration of the
C-ABI launch of the dominant kernel (HIP events recorded on the launch stream
around every such call in a second timed run of the same K steps; for decode
the split and combine kernels together), against the MI355X published peak.
The events are a run of their own because they are packets on the stream
between the launches and slow the whole job down (by about 13 us per 200 us
decode step).
``roofline.traffic`` is HBM bytes per launch from two ``rocprofv3 --pmc`` child
runs (FETCH_SIZE, WRITE_SIZE), each scaled by what the same counter reads for
a 1 GiB device copy; ``--traffic off`` skips them.  ``cpu_baseline`` is the
CPU SDPA path the metric names: ``torch.nn.functional.scaled_dot_product_attention``
in fp32 on the host's cores (at most 16 threads), timed on a bounded sample
of the same workload (decode: block-table gather + SDPA with ``enable_gqa``
per sequence, gather included; varlen: the same score pipeline per sequence
in fp32 torch math, since softcap is not an SDPA mask; backward: autograd of
SDPA).

The default run (the headline, dense FP16 causal) also measures the other
targets of the metric in the same line, under ``extra`` (``--extras off``
skips them): dense FP16 non-causal, INT8-QK causal and non-causal (BASELINE
config 3, with their speed ratio to FP16 at the same shape and mask, per
launch and whole job) and paged decode GB/s (config 4).  Each extra carries
its whole-job value, mean launch time, roofline fraction and CPU baseline.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-attn-triton_amd"))
sys.path.insert(0, ROOT)

# Host threads for the CPU baseline: the box's CPU share for one GPU.
CPU_THREADS = min(16, os.cpu_count() or 1)

PEAK = {"fp16": 2500.0, "int8_mixed": 1.0 / (0.5 / 5000.0 + 0.5 / 2500.0), "hbm": 8000.0}


def _randn(torch, shape, seed, dtype, device):
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32).to(dtype)


# ----------------------------------------------------------------------------- CPU baseline
def _median_time(fn, reps=3):
    """1 untimed run, then the median of ``reps`` timed runs (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _cpu_heads(torch, tensors, n_heads, head_axis):
    """fp32 CPU copies [1, n, S, D] of the first ``n_heads`` (batch, head) pairs
    of BSHD (head_axis 2) or BHSD (head_axis 1) tensors."""
    out = []
    for t in tensors:
        x = t.transpose(1, 2) if head_axis == 2 else t   # -> [B, H, S, D]
        B, H = x.shape[0], x.shape[1]
        x = x.reshape(B * H, x.shape[2], x.shape[3])[:n_heads]
        out.append(x.float().cpu().unsqueeze(0).contiguous())
    return out


def cpu_sdpa_dense(torch, tensors, head_axis, causal, flops_per_head, n_total, budget_s,
                   what, backward=False, dout=None):
    """fp32 SDPA (or its autograd backward) on the host over a sample of
    (batch, head) pairs sized to about ``budget_s`` seconds of work."""
    import torch.nn.functional as F
    torch.set_num_threads(CPU_THREADS)

    def run(n):
        q, k, v = _cpu_heads(torch, tensors, n, head_axis)
        if not backward:
            return lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        (g,) = _cpu_heads(torch, [dout], n, head_axis)
        q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)

        def bwd():
            out = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
            out.backward(g)
            q.grad = k.grad = v.grad = None
        return bwd

    t1 = _median_time(run(1), reps=1)
    n = int(max(1, min(n_total, budget_s / 4.0 / max(t1, 1e-6))))
    dt = _median_time(run(n))
    flops = flops_per_head * n
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": CPU_THREADS,
            "kind": "torch_sdpa_cpu",
            "sample": f"torch.nn.functional.scaled_dot_product_attention fp32 on CPU "
                      f"({'autograd backward of ' if backward else ''}{what}), {n} of {n_total} "
                      f"(batch, head) pairs as one [1, {n}, S, D] call, median of 3 after 1 "
                      f"warmup: {dt * 1e3:.1f} ms; torch.set_num_threads({CPU_THREADS})"}


# ----------------------------------------------------------------------------- workloads
def make_dense(torch, causal):
    from flash_attn_triton import flash_attn_func
    B, S, H, D = 4, 4096, 32, 128
    q, k, v = (_randn(torch, (B, S, H, D), s, torch.float16, "cuda") for s in (1, 2, 3))
    flops = 2.0 * B * H * D * S * (S + 1) if causal else 4.0 * B * H * D * S * S

    def step():
        return flash_attn_func(q, k, v, causal=causal)

    def cpu(budget_s):
        return cpu_sdpa_dense(torch, (q, k, v), 2, causal, flops / (B * H), B * H, budget_s,
                              f"S=4096, D=128, causal={causal}")

    cfg = {"workload": f"dense_fp16_{'causal' if causal else 'noncausal'}_b{B}_h{H}_s{S}_d{D}",
           "batch": B, "heads": H, "seqlen": S, "head_dim": D, "causal": causal,
           "layout": "BSHD contiguous"}
    return dict(step=step, work=flops, unit="TFLOP/s", scale=1e12, dtype="fp16",
                metric="attn fwd TFLOP/s (FP16) S=4096 D=128", bound="mfma", peak=PEAK["fp16"],
                peak_unit="TFLOP/s", config=cfg, cpu=cpu, native="fwd_dense",
                kernels=KERNELS["dense"], alg_bytes=4 * B * S * H * D * 2)


def make_bwd(torch, causal):
    """Backward of config 2 (dq, dk, dv from dout, given the forward's output and
    LSE).  FLOPs by the usual convention: 2.5 x the forward's (five products per
    visible pair)."""
    from flash_attn_triton.triton_kernel.attention_kernel import dense_backward, dense_forward
    B, S, H, D = 4, 4096, 32, 128
    q, k, v, do = (_randn(torch, (B, S, H, D), s, torch.float16, "cuda") for s in (1, 2, 3, 8))
    scale = 1.0 / math.sqrt(D)
    out, lse = dense_forward(q, k, v, softmax_scale=scale, causal=causal, return_lse=True)
    fwd = 2.0 * B * H * D * S * (S + 1) if causal else 4.0 * B * H * D * S * S
    flops = 2.5 * fwd

    def step():
        return dense_backward(q, k, v, out, do, lse, softmax_scale=scale, causal=causal)

    def cpu(budget_s):
        # The timed CPU call is forward + backward (autograd has no backward
        # alone); its rate counts the backward's 2.5x FLOPs, so it flatters the
        # CPU by the forward's share.
        return cpu_sdpa_dense(torch, (q, k, v), 2, causal, flops / (B * H), B * H, budget_s,
                              f"S=4096, D=128, causal={causal}; forward included in the time",
                              backward=True, dout=do)

    cfg = {"workload": f"dense_bwd_fp16_{'causal' if causal else 'noncausal'}_b{B}_h{H}_s{S}_d{D}",
           "batch": B, "heads": H, "seqlen": S, "head_dim": D, "causal": causal,
           "layout": "BSHD contiguous", "flop_convention": "2.5 x forward"}
    return dict(step=step, work=flops, unit="TFLOP/s", scale=1e12, dtype="fp16",
                metric="attn bwd TFLOP/s (FP16) S=4096 D=128", bound="mfma", peak=PEAK["fp16"],
                peak_unit="TFLOP/s", config=cfg, cpu=cpu, native="bwd_dense",
                kernels=KERNELS["bwd"], alg_bytes=8 * B * S * H * D * 2 + 2 * B * H * S * 4)


def make_int8(torch, causal):
    from flash_attn_triton.triton_kernel.attention_kernel_int8 import attention_int8
    B, H, S, D = 4, 32, 4096, 128
    q, k, v = (_randn(torch, (B, H, S, D), s, torch.float16, "cuda") for s in (4, 5, 6))
    gen = torch.Generator(device="cuda").manual_seed(7)
    n_out = S // 100
    idx = torch.argsort(torch.rand(B * H, S, generator=gen, device="cuda"), dim=1)[:, :n_out]
    kf = k.view(B * H, S, D)
    rows = torch.arange(B * H, device="cuda")[:, None].expand(-1, n_out)
    kf[rows, idx] = (kf[rows, idx].float() * 8.0).half()
    flops = 2.0 * B * H * D * S * (S + 1) if causal else 4.0 * B * H * D * S * S

    def step():
        return attention_int8(q, k, v, causal=causal)

    def cpu(budget_s):
        # The host has no INT8 attention: fp32 SDPA of the same shape and mask.
        return cpu_sdpa_dense(torch, (q, k, v), 1, causal, flops / (B * H), B * H, budget_s,
                              f"S=4096, D=128, causal={causal}, same inputs as the INT8 run")

    cfg = {"workload": f"int8qk_{'causal' if causal else 'noncausal'}_b{B}_h{H}_s{S}_d{D}",
           "batch": B, "heads": H, "seqlen": S, "head_dim": D, "causal": causal,
           "k_outliers": "1% of token rows x8", "layout": "BHSD contiguous"}
    return dict(step=step, work=flops, unit="TFLOP/s", scale=1e12, dtype="int8+fp16",
                metric="attn fwd TFLOP/s (INT8-QK) S=4096 D=128", bound="mfma",
                peak=PEAK["int8_mixed"], peak_unit="TFLOP/s", config=cfg, cpu=cpu,
                native="fwd_int8", kernels=KERNELS["int8"],
                alg_bytes=B * H * S * (3 * D * 2 + D + 4))


def make_decode(torch):
    from flash_attn_triton import flash_attn_with_kvcache
    B, Hq, Hk, D, page = 64, 32, 8, 128, 256
    gen = torch.Generator().manual_seed(0)
    lengths = torch.randint(512, 8193, (B,), generator=gen)
    pages_per = ((lengths + page - 1) // page).tolist()
    n_pages = sum(pages_per)
    perm = torch.randperm(n_pages, generator=gen)
    bt = torch.zeros((B, 32), dtype=torch.int32)
    pos = 0
    for b, n in enumerate(pages_per):
        bt[b, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    kc = _randn(torch, (n_pages, page, Hk, D), 11, torch.float16, "cuda")
    vc = _randn(torch, (n_pages, page, Hk, D), 12, torch.float16, "cuda")
    q = _randn(torch, (B, 1, Hq, D), 13, torch.float16, "cuda")
    seqlens = lengths.to(torch.int32).cuda()
    btd = bt.cuda()
    total_tokens = int(lengths.sum())
    nbytes = (total_tokens * Hk * D * 2 * 2 + q.numel() * 2 * 2 + sum(pages_per) * 4 + B * 4)

    def step():
        return flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens, block_table=btd)

    def cpu(budget_s):
        # Per sequence: gather its pages through the block table, then SDPA with
        # enable_gqa (the gather is inside the timing).  The host caches are
        # fp32, so the CPU reads twice the fp16 bytes the rate is quoted in.
        import torch.nn.functional as F
        torch.set_num_threads(CPU_THREADS)
        kh, vh, qh = kc.float().cpu(), vc.float().cpu(), q.float().cpu()
        btl = bt.long()

        def one(b):
            L = int(lengths[b])
            pg = btl[b, :pages_per[b]]
            k = kh[pg].reshape(-1, Hk, D)[:L].transpose(0, 1).unsqueeze(0)
            v = vh[pg].reshape(-1, Hk, D)[:L].transpose(0, 1).unsqueeze(0)
            return F.scaled_dot_product_attention(qh[b:b + 1].transpose(1, 2), k, v,
                                                  enable_gqa=True)

        one(0)
        done, b, t0 = 0, 0, time.perf_counter()
        while b < B and (time.perf_counter() - t0) < budget_s:
            one(b)
            done += int(lengths[b]) * Hk * D * 2 * 2 + Hq * D * 2 * 2 + pages_per[b] * 4 + 4
            b += 1
        dt = time.perf_counter() - t0
        return {"value": round(done / dt / 1e9, 4), "unit": "GB/s", "cores": CPU_THREADS,
                "kind": "torch_sdpa_cpu",
                "sample": f"per sequence: block-table gather + "
                          f"torch.nn.functional.scaled_dot_product_attention(enable_gqa=True), "
                          f"fp32 on CPU, {b} of {B} sequences in {dt:.2f} s (gather included); "
                          f"rate in the fp16 algorithmic bytes; "
                          f"torch.set_num_threads({CPU_THREADS})"}

    cfg = {"workload": "paged_decode_b64_hq32_hk8_d128_page256", "batch": B, "heads_q": Hq,
           "heads_k": Hk, "head_dim": D, "page_size": page, "total_cache_tokens": total_tokens,
           "cache_lengths": "U[512, 8192], seed 0", "block_table": "random page permutation"}
    return dict(step=step, work=nbytes, unit="GB/s", scale=1e9, dtype="fp16",
                metric="paged decode GB/s", bound="hbm", peak=PEAK["hbm"], peak_unit="GB/s",
                config=cfg, cpu=cpu, native="fwd_kvcache", kernels=KERNELS["decode"],
                alg_bytes=nbytes)


def make_varlen(torch):
    from flash_attn_triton import flash_attn_varlen_func
    H, D = 16, 128
    gen = torch.Generator().manual_seed(0)
    lengths = torch.randint(128, 4097, (32,), generator=gen)
    cu = torch.zeros(33, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0).to(torch.int32)
    T = int(cu[-1])
    q, k, v = (_randn(torch, (T, H, D), s, torch.float16, "cuda") for s in (21, 22, 23))
    slopes = (2.0 ** (-8.0 * (torch.arange(H) + 1) / H)).float().cuda()
    cud = cu.cuda()
    max_len = int(lengths.max())
    left, cap = 1024, 30.0

    def pairs(L):
        i = torch.arange(L, dtype=torch.float64)
        return float(torch.clamp(i, max=left).sum() + L)

    n_pairs = sum(pairs(int(L)) for L in lengths)
    flops = 4.0 * H * D * n_pairs

    def step():
        return flash_attn_varlen_func(q, k, v, cud, cud, max_len, max_len, causal=True,
                                      window_size=(left, 0), softcap=cap, alibi_slopes=slopes)

    def cpu(budget_s):
        # softcap is not an additive mask, so the host runs SDPA's math as
        # fp32 torch ops per sequence: scores, ALiBi, softcap, causal + window
        # mask, softmax, product with V.
        torch.set_num_threads(CPU_THREADS)
        qh, kh, vh = (t.float().cpu() for t in (q, k, v))
        sl = slopes.cpu()
        scale = 1.0 / math.sqrt(D)

        def one(b):
            s, e = int(cu[b]), int(cu[b + 1])
            L = e - s
            qs, ks, vs = (t[s:e].transpose(0, 1) for t in (qh, kh, vh))   # [H, L, D]
            sc = torch.matmul(qs, ks.transpose(1, 2)) * scale
            i = torch.arange(L)
            dist = (i[:, None] - i[None, :]).float()
            sc = sc - sl[:, None, None] * dist.abs()
            sc = cap * torch.tanh(sc / cap)
            keep = (dist >= 0) & (dist <= left)
            sc = sc.masked_fill(~keep, float("-inf"))
            return torch.matmul(torch.softmax(sc, dim=-1), vs)

        one(0)
        done, b, t0 = 0.0, 0, time.perf_counter()
        while b < 32 and (time.perf_counter() - t0) < budget_s:
            one(b)
            done += 4.0 * H * D * pairs(int(cu[b + 1] - cu[b]))
            b += 1
        dt = time.perf_counter() - t0
        return {"value": round(done / dt / 1e12, 5), "unit": "TFLOP/s", "cores": CPU_THREADS,
                "kind": "torch_math_cpu",
                "sample": f"SDPA math in fp32 torch ops on CPU per sequence (scores, ALiBi, "
                          f"softcap, causal + window mask, softmax, PV), {b} of 32 sequences "
                          f"in {dt:.2f} s; torch.set_num_threads({CPU_THREADS})"}

    cfg = {"workload": "varlen_fp16_32seq_h16_d128_causal_win1024_alibi_softcap30",
           "sequences": 32, "total_tokens": T, "heads": H, "head_dim": D,
           "unmasked_pairs": n_pairs}
    return dict(step=step, work=flops, unit="TFLOP/s", scale=1e12, dtype="fp16",
                metric="varlen attn fwd TFLOP/s (FP16, causal+window+ALiBi+softcap)",
                bound="mfma", peak=PEAK["fp16"], peak_unit="TFLOP/s", config=cfg, cpu=cpu,
                native="fwd_varlen", kernels=KERNELS["varlen"], alg_bytes=4 * T * H * D * 2)


def make_copy(torch):
    """Calibration leg for the HBM traffic counters: a device-to-device copy of
    1 GiB (torch's copy kernel) moves exactly 1 GiB in and 1 GiB out, so
    FETCH_SIZE / WRITE_SIZE per dispatch of this kernel give the counter's
    scale factor."""
    n = 1 << 29
    src = torch.ones(n, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    nbytes = 2 * src.numel() * 2

    def step():
        dst.copy_(src)
        return dst

    cfg = {"workload": "copy_1GiB_fp16", "bytes_read": src.numel() * 2,
           "bytes_written": src.numel() * 2}
    return dict(step=step, work=nbytes, unit="GB/s", scale=1e9, dtype="fp16",
                metric="device copy GB/s (traffic-counter calibration)", bound="hbm",
                peak=PEAK["hbm"], peak_unit="GB/s", config=cfg, cpu=None, native=None,
                kernels=KERNELS["copy"], alg_bytes=nbytes)


# The dominant kernel(s) of each workload as rocprofv3 names them; the first
# one is launched once per step.
KERNELS = {
    "dense_causal": ("fa::prefill_persist_kernel",),
    "dense": ("fa::prefill_persist_kernel",),
    "bwd_causal": ("fa::bwd_dq_kernel", "fa::bwd_dkdv_split_kernel"),
    "bwd": ("fa::bwd_dq_kernel", "fa::bwd_dkdv_split_kernel"),
    "int8_causal": ("fa::int8_persist_kernel",),
    "int8": ("fa::int8_persist_kernel",),
    "decode": ("fa::decode_kernel", "fa::decode_combine_kernel"),
    "varlen": ("fa::prefill_kernel",),
    "copy": ("__amd_rocclr_copyBuffer",),
}

WORKLOADS = {
    "dense_causal": lambda torch: make_dense(torch, True),
    "dense": lambda torch: make_dense(torch, False),
    "bwd_causal": lambda torch: make_bwd(torch, True),
    "bwd": lambda torch: make_bwd(torch, False),
    "int8_causal": lambda torch: make_int8(torch, True),
    "int8": lambda torch: make_int8(torch, False),
    "decode": make_decode,
    "varlen": make_varlen,
    "copy": make_copy,
}


# ----------------------------------------------------------------------------- traffic
def _counter_per_dispatch(csv_path, counter, kernels):
    """Mean of ``counter`` (KiB) per launch of ``kernels[0]``, summed over every
    dispatch of every kernel in ``kernels`` (rocprofv3 counter_collection.csv)."""
    import csv
    total, primary = 0.0, 0
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            name = row["Kernel_Name"]
            hit = [k for k in kernels if k in name]
            if not hit:
                continue
            total += float(row["Counter_Value"])
            primary += hit[0] == kernels[0]
    return total / primary if primary else None


def _pmc_pass(workload, counter, kernels, outdir):
    """One ``rocprofv3 --pmc <counter>`` run of this script (a child process,
    started before this process touches the GPU) -> KiB per dispatch."""
    import glob
    import subprocess
    d = os.path.join(outdir, f"{workload}_{counter}")
    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "pmc", "--",
           sys.executable, os.path.abspath(__file__), "--workload", workload, "--steps", "2",
           "--warmup", "1", "--prewarm", "0", "--cpu-budget", "0", "--traffic", "off",
           "--extras", "off"]
    subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=180,
                   check=True)
    found = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not found:
        raise RuntimeError(f"rocprofv3 wrote no counter file under {d}")
    return _counter_per_dispatch(found[0], counter, kernels)


def measure_traffic(workload, kernels, keep_dir=None):
    """HBM bytes per launch of the dominant kernel(s) from FETCH_SIZE and
    WRITE_SIZE, each scaled by what the same counter reads for a 1 GiB
    device copy (1 GiB read, 1 GiB written)."""
    import shutil
    import tempfile
    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not found"
    copy_kernels = ("__amd_rocclr_copyBuffer",)
    gib = float(1 << 30)
    out = {}
    with tempfile.TemporaryDirectory(prefix="fa_pmc_") as tmp:
        if keep_dir:
            os.makedirs(keep_dir, exist_ok=True)
            tmp = keep_dir
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            cal = _pmc_pass("copy", counter, copy_kernels, tmp)
            val = _pmc_pass(workload, counter, kernels, tmp)
            if not cal or val is None:
                return None, f"{counter}: no matching dispatches"
            factor = gib / (cal * 1024.0)
            out[counter] = (val * 1024.0 * factor, factor)
    return out, None


class _HipEvents:
    """Timing events of the HIP runtime this process runs on, created with
    ``hipEventReleaseToDevice``: recording one then ends with a device-scope
    release instead of the default system-scope one (the runtime's flag for
    precise timings of the commands between events).  torch's events use the
    default flags; around every decode call their system-scope releases cost
    about 13 us of GPU time per step (measured on MI355X, 197.5 -> 211 us)."""

    RELEASE_TO_DEVICE = 0x40000000

    def __init__(self):
        path = next((l.split()[-1] for l in open("/proc/self/maps") if "libamdhip64" in l),
                    "libamdhip64.so.7")
        hip = ctypes.CDLL(path)
        hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                            ctypes.c_void_p]
        hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        for f in ("hipEventCreateWithFlags", "hipEventRecord", "hipEventElapsedTime",
                  "hipEventDestroy"):
            getattr(hip, f).restype = ctypes.c_int
        self.hip = hip

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def create(self):
        ev = ctypes.c_void_p()
        self._ok(self.hip.hipEventCreateWithFlags(ctypes.byref(ev), self.RELEASE_TO_DEVICE),
                 "hipEventCreateWithFlags")
        return ev

    def record(self, ev, stream_handle):
        self._ok(self.hip.hipEventRecord(ev, ctypes.c_void_p(stream_handle)), "hipEventRecord")

    def elapsed_ms(self, start, stop):
        ms = ctypes.c_float()
        self._ok(self.hip.hipEventElapsedTime(ctypes.byref(ms), start, stop),
                 "hipEventElapsedTime")
        return ms.value

    def destroy(self, ev):
        self.hip.hipEventDestroy(ev)


class _LaunchTimer:
    """Records HIP events on the launch stream around every call of one C-ABI
    entry point (``fa_<name>``, the launch of the dominant kernel).  The
    events bracket the library call itself, so the Python wrapper's argument
    preparation, which the GPU would otherwise wait out when its queue is
    empty (the KV-cache path synchronizes once per call to check its
    arguments), stays outside the window.  The events are created before the
    timed region (``_HipEvents``: device-scope release)."""

    def __init__(self, torch, name, calls):
        self.torch, self.name, self.pairs, self.used = torch, name, [], 0
        self.orig = self.lib = None
        self.calls = calls

    def __enter__(self):
        from flash_attn_triton import _native
        if self.name is None:
            return self
        self.ev = _HipEvents()
        self.pairs = [(self.ev.create(), self.ev.create()) for _ in range(self.calls)]
        self.lib = _native.load()
        self.cname = "fa_" + self.name
        self.orig = getattr(self.lib, self.cname)
        torch, orig, ev = self.torch, self.orig, self.ev

        def timed(*a):
            if self.used == len(self.pairs):
                self.pairs.append((ev.create(), ev.create()))
            s, e = self.pairs[self.used]
            self.used += 1
            stream = torch.cuda.current_stream().cuda_stream
            ev.record(s, stream)
            r = orig(*a)
            ev.record(e, stream)
            return r

        setattr(self.lib, self.cname, timed)
        return self

    def __exit__(self, *exc):
        if self.orig is not None:
            setattr(self.lib, self.cname, self.orig)
        return False

    def mean_s(self):
        if not self.used:
            return None
        ms = [self.ev.elapsed_ms(s, e) for s, e in self.pairs[:self.used]]
        for s, e in self.pairs:
            self.ev.destroy(s)
            self.ev.destroy(e)
        return sum(ms) / len(ms) / 1e3


def prewarm(torch, step, seconds):
    """Untimed steps for about ``seconds`` of wall time, in batches of 8 with a
    synchronization after each, before the counted warmup: the GPU's clocks
    take on the order of 100 ms of continuous load to settle (the C2 causal
    launch measured 660 us after 3 warmup steps, 571 us after 30 and 546 us
    after 200 on one MI355X)."""
    n, t0 = 0, time.perf_counter()
    while seconds > 0 and time.perf_counter() - t0 < seconds and n < 100000:
        for _ in range(8):
            step()
        n += 8
        torch.cuda.synchronize()
    return n


def measure(torch, wl, steps, warmup, prewarm_s=0.0):
    """Whole-job time of ``steps`` steps after the clock pre-warm and ``warmup``
    untimed steps, and the mean launch time of the dominant kernel.

    Two timed regions of ``steps`` steps each: the first, with nothing but the
    steps between its two synchronizations, gives the whole-job value; the
    second records HIP events around every launch of the dominant kernel and
    gives its mean launch time.  Events between launches are packets of their
    own on the stream: around every decode call (a 200 us step) they added
    about 13 us per step to the whole job, whichever release scope they use."""
    step = wl["step"]
    n_pre = prewarm(torch, step, prewarm_s)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    with _LaunchTimer(torch, wl["native"], steps) as timer:
        t1 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        wall_events = time.perf_counter() - t1
    avg_launch_s = timer.mean_s()
    if avg_launch_s is None:   # copy calibration: no native entry point
        avg_launch_s = wall / steps
    achieved = wl["work"] / avg_launch_s / wl["scale"]
    return {
        "wall": wall,
        "ms_per_step": wall / steps * 1e3,
        "value": wl["work"] / (wall / steps) / wl["scale"],
        "avg_launch_s": avg_launch_s,
        "achieved": achieved,
        "frac": achieved / wl["peak"],
        "prewarm_steps": n_pre,
        "ms_per_step_with_events": wall_events / steps * 1e3,
    }


def run_cpu(torch, wl, budget):
    if budget <= 0 or wl["cpu"] is None:
        return None
    from threadpoolctl import threadpool_limits
    with threadpool_limits(limits=CPU_THREADS):
        return wl["cpu"](budget)


# The other targets of the metric, and the backward of the headline
# configuration, measured with the headline in the default run.
EXTRAS = ("dense", "int8_causal", "int8", "decode", "varlen", "bwd_causal")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--prewarm", type=float, default=0.5,
                    help="seconds of untimed steps before the warmup steps, for the GPU clocks "
                         "to settle (0 = none)")
    ap.add_argument("--workload", default="dense_causal", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-budget", type=float, default=8.0,
                    help="seconds of host work for each CPU baseline sample (0 = skip)")
    ap.add_argument("--traffic", default="auto", choices=("auto", "off"),
                    help="auto: two rocprofv3 --pmc child runs (FETCH_SIZE, WRITE_SIZE) plus a "
                         "copy calibration give roofline.traffic; off: traffic null")
    ap.add_argument("--traffic-dir", default=None,
                    help="keep the counter runs' rocprofv3 output under this directory")
    ap.add_argument("--extras", default="auto", choices=("auto", "off"),
                    help="auto: the default workload also measures " + ", ".join(EXTRAS))
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; every box in this pipeline has one GPU and "
              "the attention forward needs no cross-GPU exchange (heads and batches shard across "
              "GPUs without communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    # Counter passes run first, as child processes, while this process has not
    # touched the GPU yet.
    traffic, traffic_note = None, None
    if args.traffic == "auto" and args.workload != "copy":
        try:
            traffic, traffic_note = measure_traffic(args.workload, KERNELS[args.workload],
                                                    args.traffic_dir)
        except Exception as exc:  # counters are optional: the line is still printed
            traffic, traffic_note = None, f"counter pass failed: {exc}"

    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    wl = WORKLOADS[args.workload](torch)
    m = measure(torch, wl, args.steps, args.warmup, args.prewarm)
    cpu = run_cpu(torch, wl, args.cpu_budget)

    roof = {
        "bound": wl["bound"],
        "achieved": round(m["achieved"], 3),
        "peak": round(wl["peak"], 1),
        "unit": wl["peak_unit"],
        "frac": round(m["frac"], 4),
        "traffic": None,
        "kernel": " + ".join(wl["kernels"]),
        "avg_launch_us": round(m["avg_launch_s"] * 1e6, 2),
        "launch_timing": "HIP events (device-scope release) around every launch in a second "
                         "timed run of the same steps",
        "ms_per_step_with_events": round(m["ms_per_step_with_events"], 4),
    }
    if traffic is not None:
        fetch, ffac = traffic["FETCH_SIZE"]
        write, wfac = traffic["WRITE_SIZE"]
        roof["traffic"] = round(fetch + write)
        roof["traffic_detail"] = {"read_bytes": round(fetch), "write_bytes": round(write),
                                  "fetch_factor": round(ffac, 4), "write_factor": round(wfac, 4),
                                  "algorithmic_bytes": wl.get("alg_bytes")}
    elif traffic_note is not None:
        roof["traffic_note"] = traffic_note
    line = {
        "metric": wl["metric"],
        "value": round(m["value"], 3),
        "unit": wl["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_steps": m["prewarm_steps"],
        "ms_per_step": round(m["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic (seeded N(0,1))",
        "config": wl["config"],
        "roofline": roof,
        "cpu_baseline": cpu,
    }

    if args.extras == "auto" and args.workload == "dense_causal":
        extra = {}
        del wl
        runs = {"dense_causal": m}
        for name in EXTRAS:
            xw = WORKLOADS[name](torch)
            xm = measure(torch, xw, args.steps, args.warmup, args.prewarm)
            runs[name] = xm
            extra[name] = {
                "metric": xw["metric"], "value": round(xm["value"], 3), "unit": xw["unit"],
                "ms_per_step": round(xm["ms_per_step"], 4), "prewarm_steps": xm["prewarm_steps"],
                "dtype": xw["dtype"],
                "config": xw["config"],
                "roofline": {"bound": xw["bound"], "achieved": round(xm["achieved"], 3),
                             "peak": round(xw["peak"], 1), "unit": xw["peak_unit"],
                             "frac": round(xm["frac"], 4),
                             "kernel": " + ".join(xw["kernels"]),
                             "avg_launch_us": round(xm["avg_launch_s"] * 1e6, 2)},
                "cpu_baseline": run_cpu(torch, xw, args.cpu_budget),
            }
            if name.startswith("int8"):
                fp16 = runs["dense_causal" if name == "int8_causal" else "dense"]
                # Same FLOPs on both sides: the speed ratio is the time ratio.
                extra[name]["speedup_vs_fp16"] = {
                    "whole_job": round(fp16["ms_per_step"] / xm["ms_per_step"], 4),
                    "per_launch": round(fp16["avg_launch_s"] / xm["avg_launch_s"], 4),
                    "fp16_frac_of_fp16_peak": round(fp16["frac"], 4),
                    "int8_frac_of_fp16_peak": round(xm["achieved"] / PEAK["fp16"], 4),
                    "target": 1.3}
            del xw
            torch.cuda.empty_cache()
        line["extra"] = extra
    print(json.dumps(line))


if __name__ == "__main__":
    main()
