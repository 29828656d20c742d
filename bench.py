"""Benchmark of the smooth-attn hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

A step is one forward + backward pass of the causal squareplus
normalisation over config 2 at L=4096 (x = randn/sqrt(128) and
dy = randn, bf16 [4,16,4096,4096], family alpha=2, theta=0.5, p=2), run
through the public autograd API.  ``value`` is algorithmic HBM bytes per
step / step time.  Algorithmic bytes: the forward reads the causal triangle
of x and writes the full output; the backward reads the triangle of x and
dy and writes the full dx (2 bytes per element).  HIP events around the
forward and backward launches inside the timed steps give the per-launch
durations behind ``roofline``.

Every other figure follows one protocol: the median of 100 launches, each
timed by its own HIP event pair on the launch stream and preceded by a read
of 512 MiB of unrelated memory (which evicts the inputs from L2 and the
256 MB Infinity Cache), after 20 warm-up launches.  The line carries the
fused-attention figures the metric also names (config 3 forward and
backward, TFLOP/s over the causal triangle), config 4 (fp8), config 5
(paged decode), config 2 at L = 1024 / 2048 with its row-wise fp32 variant,
config 1's shape on the GPU, the rows built after the hot path (RoPE
attention, softmax baselines, paged-KV append), and the CPU baselines: the
reference's eager CPU path restated in oracle/ (fp32 torch on the host
cores), each on a bounded, stated sample of its config.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "smooth-attn_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
FP8_PEAK_TFLOPS = 5033.2
FP32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA
# HBM bytes per launch of the causal-norm kernels on this workload, measured
# with rocprofv3 FETCH_SIZE and WRITE_SIZE passes over this script
# (--copy-calibration) and scaled by what the same counters read for a plain
# 1 GiB device copy: FETCH_SIZE x 2.000, WRITE_SIZE x 1.000.  The counter
# summary and commands are kept under profiles/.
NORM_TRAFFIC_BYTES = {"fwd": 3.2393e9, "bwd": 4.3325e9}
METRIC = "causal-norm fwd+bwd HBM GB/s (% peak); fused attn TFLOP/s, L=4096 D=128"


def tri(n):
    return n * (n + 1) // 2


def norm_bytes(B, H, L, elem=2):
    fwd = B * H * elem * (tri(L) + L * L)
    bwd = B * H * elem * (2 * tri(L) + L * L)
    return fwd, bwd


def attn_flops(B, H, L, D):
    return 4 * B * H * D * tri(L)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def time_events(torch, fn, iters):
    """Per-launch durations (ms) from HIP events on the current stream."""
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for a, b in evs:
        a.record(st)
        fn()
        b.record(st)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


FLUSH_BYTES = 512 << 20
KERNEL_ITERS = 100
KERNEL_WARMUP = 20
_flush_buf = None


def flush_caches(torch):
    """Read 512 MiB of unrelated memory: evicts earlier data from the 4 MB
    L2s and the 256 MB Infinity Cache, and (being a read) leaves no dirty
    lines whose write-back would land in the next timed launch."""
    global _flush_buf
    if _flush_buf is None:
        _flush_buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device="cuda:0")
    _flush_buf.sum()


def time_kernel(torch, fn, iters=KERNEL_ITERS, warmup=KERNEL_WARMUP, flush=True):
    """BASELINE protocol for one launch ``fn``: ``warmup`` untimed launches,
    then ``iters`` launches each bracketed by its own HIP event pair on the
    current (launch) stream and preceded by a cache flush outside the
    events.  Returns the median, mean and p10/p90 in microseconds."""
    for _ in range(warmup):
        if flush:
            flush_caches(torch)
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for a, b in evs:
        if flush:
            flush_caches(torch)
        a.record(st)
        fn()
        b.record(st)
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    n = len(us)
    return {"median": us[n // 2], "mean": sum(us) / n, "p10": us[n // 10], "p90": us[(9 * n) // 10], "n": n}


def time_rotating(torch, fns, iters=KERNEL_ITERS, warmup=KERNEL_WARMUP):
    """Back-to-back launches cycling over ``fns`` (closures over separate
    input/output copies, so each launch's inputs were last touched
    len(fns) - 1 launches earlier and, with at least 3 copies larger than
    the 256 MB Infinity Cache together, come from HBM), ``iters`` of them
    between one HIP event pair: the average per launch, without the fixed
    cost of an event pair per launch.  Returns microseconds."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for i in range(iters):
        fns[i % len(fns)]()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / iters


def bench_norm(torch, sa, steps, warmup):
    """Config 2 at L=4096: the per-kernel protocol on the forward and the
    backward launch, then the timed steps (W untimed, K timed) with HIP
    events around each launch inside them."""
    from smooth_attn import FamilyConfig, kernels

    B, H, L = 4, 16, 4096
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(2)
    x = (torch.randn(B, H, L, L, generator=gen, device=dev) / math.sqrt(128)).to(torch.bfloat16)
    dy = torch.randn(B, H, L, L, generator=gen, device=dev).to(torch.bfloat16)
    fam = FamilyConfig()
    fwd_b, bwd_b = norm_bytes(B, H, L)

    out = torch.empty_like(x)
    kf = time_kernel(torch, lambda: sa.softplus_norm_causal_triton_out(out, x, family=fam))
    kb = time_kernel(torch, lambda: kernels._softplus_norm_causal_backward(x, dy, fam))
    del out

    xg = x.detach().requires_grad_(True)
    st = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]

    def step(e=None):
        if e is not None:
            e[0].record(st)
        y = sa.softplus_norm_causal(xg, family=fam)
        if e is not None:
            e[1].record(st)
        (dx,) = torch.autograd.grad(y, xg, dy)
        if e is not None:
            e[2].record(st)
        return dx

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(ev[i])
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    fwd_avg = sum(e[0].elapsed_time(e[1]) for e in ev) / steps  # ms
    bwd_avg = sum(e[1].elapsed_time(e[2]) for e in ev) / steps
    sample = x[0, 0].cpu(), dy[0, 0].cpu()
    del x, dy, xg
    torch.cuda.empty_cache()
    return {
        "shape": [B, H, L, L],
        "ms_per_step": ms_per_step,
        "gbs": (fwd_b + bwd_b) / (ms_per_step * 1e-3) / 1e9,
        "fwd_bytes": fwd_b,
        "bwd_bytes": bwd_b,
        "fwd_us": fwd_avg * 1e3,
        "bwd_us": bwd_avg * 1e3,
        "fwd_gbs": fwd_b / (fwd_avg * 1e-3) / 1e9,
        "bwd_gbs": bwd_b / (bwd_avg * 1e-3) / 1e9,
        "kernel_fwd": kf,
        "kernel_bwd": kb,
        "sample": sample,
    }


def _rounded(d, nd=2):
    return {k: (round(v, nd) if isinstance(v, float) else v) for k, v in d.items()}


def bench_attention(torch, sa):
    """Config 3: forward and backward of the fused bf16 attention."""
    from smooth_attn import kernels

    B, H, L, D = 4, 32, 4096, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(B, H, L, D, generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn(B, H, L, D, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(B, H, L, D, generator=gen, device=dev).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    kf = time_kernel(torch, lambda: kernels._sp2norm_flash_fwd(q, k, v, scale))
    flops = attn_flops(B, H, L, D)
    # Backward (dQ + delta kernel, then dK/dV kernel) on the forward's o and
    # row sums with a seeded upstream gradient.  FLOPs counted as 2.5 x the
    # forward's (the usual convention: dQ, dK, dV, dP and one S product); the
    # two-kernel scheme executes 3.5 x (S and dP are recomputed in both).
    do = torch.randn(B, H, L, D, generator=gen, device=dev).to(torch.bfloat16)
    o, rs = kernels._sp2norm_flash_fwd(q, k, v, scale)
    kb = time_kernel(torch, lambda: kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, scale))
    bflops = 2.5 * flops
    us, bus = kf["median"], kb["median"]
    # Sustained: back to back over 3 input copies (1.1 GB of q/k/v, 2.6 GB
    # with the backward's o/dO, against a 256 MB Infinity Cache), as a
    # training step runs them; the clock then settles lower than between
    # the flushed launches above.
    copies = [(q, k, v, o, do, rs)] + [tuple(t.clone() for t in (q, k, v, o, do, rs)) for _ in range(2)]
    sus = time_rotating(torch, [lambda c=c: kernels._sp2norm_flash_fwd(c[0], c[1], c[2], scale) for c in copies])
    bsus = time_rotating(torch, [lambda c=c: kernels._sp2norm_flash_bwd(*c, scale) for c in copies])
    sample = q[0, :4].cpu(), k[0, :4].cpu(), v[0, :4].cpu()
    del q, k, v, do, o, rs, copies
    torch.cuda.empty_cache()
    return {
        "config": "config3 fused causal attention fwd bf16 [4,32,4096,128]",
        "us": round(us, 2),
        "tflops": round(flops / us / 1e6, 1),
        "frac_bf16_peak": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
        "flops": flops,
        "fwd_times_us": _rounded(kf),
        "bwd_us": round(bus, 2),
        "bwd_tflops": round(bflops / bus / 1e6, 1),
        "bwd_frac_bf16_peak": round(bflops / bus / 1e6 / BF16_PEAK_TFLOPS, 4),
        "bwd_flops": bflops,
        "bwd_times_us": _rounded(kb),
        "sustained_us": round(sus, 2),
        "sustained_frac_bf16_peak": round(flops / sus / 1e6 / BF16_PEAK_TFLOPS, 4),
        "bwd_sustained_us": round(bsus, 2),
        "bwd_sustained_frac_bf16_peak": round(bflops / bsus / 1e6 / BF16_PEAK_TFLOPS, 4),
        "sustained_protocol": "100 back-to-back launches over 3 input copies between one HIP event pair, "
                              "after 20 warm-up launches",
    }, sample


def bench_fp8(torch):
    """Config 4: fp8 e4m3fn Q/K (per-tensor scales), bf16 V, GQA 32/8, L=8192.
    Kernel-only timing on pre-quantised inputs (as tests/bench_fp8_kernel.py
    times the reference), plus the full entry point with device quantisation."""
    import smooth_attn
    from smooth_attn import kernels

    B, Hq, Hkv, L, D = 2, 32, 8, 8192, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(B, Hq, L, D, generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, D, generator=gen, device=dev).to(torch.bfloat16)
    q8, qs = kernels._quantize_to_fp8_device(q)
    k8, ks = kernels._quantize_to_fp8_device(k)
    scale = 1.0 / math.sqrt(D)
    kt = time_kernel(torch, lambda: kernels._sp2norm_fp8_flash_fwd(q8, k8, v, qs, ks, None, scale, Hq // Hkv))
    full = time_kernel(torch, lambda: smooth_attn.sp2norm_fp8_flash_attention(q, k, v, quantize_v=False),
                       iters=30, warmup=5)
    qk_flops = 2 * B * Hq * D * tri(L)
    ideal_us = qk_flops / (FP8_PEAK_TFLOPS * 1e12) * 1e6 + qk_flops / (BF16_PEAK_TFLOPS * 1e12) * 1e6
    us = kt["median"]
    # Sustained: back to back over 4 copies of the kernel's inputs (4 x 112 MiB)
    copies = [(q8, k8, v)] + [(q8.clone(), k8.clone(), v.clone()) for _ in range(3)]
    sus = time_rotating(torch, [lambda c=c: kernels._sp2norm_fp8_flash_fwd(c[0], c[1], c[2], qs, ks, None, scale,
                                                                           Hq // Hkv) for c in copies])
    del copies
    sample = (q8[0, 0].cpu(), k8[0, 0].cpu(), v[0, 0].cpu(), float(qs), float(ks))
    del q, k, v, q8, k8
    torch.cuda.empty_cache()
    return {
        "config": "config4 fp8 e4m3fn QK^T + bf16 PV, GQA 32/8, [2,32|8,8192,128]",
        "us": round(us, 2),
        "tflops_total": round(2 * qk_flops / us / 1e6, 1),
        "frac_of_mfma_roofline": round(ideal_us / us, 4),
        "ideal_us": round(ideal_us, 2),
        "times_us": _rounded(kt),
        "entry_point_us_incl_quantisation": round(full["median"], 2),
        "sustained_us": round(sus, 2),
        "sustained_frac_of_mfma_roofline": round(ideal_us / sus, 4),
        "sustained_protocol": "100 back-to-back launches over 4 input copies between one HIP event pair, "
                              "after 20 warm-up launches",
    }, sample


def config5_inputs(torch):
    """Config 5's seeded layout: 64 sequences, ctx ~ U[512, 16384], page 16,
    the block table a seeded permutation of all pages handed out in order."""
    B, P = 64, 16
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(512, 16385, (B,), generator=g)
    npg_seq = [(int(c) + P - 1) // P for c in lens]
    n_pages = sum(npg_seq)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    table = torch.zeros(B, max(npg_seq), dtype=torch.int32)
    pos = 0
    for i, n in enumerate(npg_seq):
        table[i, :n] = perm[pos:pos + n]
        pos += n
    return lens, table, n_pages


def paged_bytes(lens, P=16, B=64, Hq=32, D=128):
    tot = int(lens.sum())
    npg = sum((int(c) + P - 1) // P for c in lens)
    return 4096 * tot + 4 * npg + B * Hq * D * 2 * 2 + 4 * B


def bench_paged(torch):
    """Config 5: 64 sequences, ctx ~ U[512, 16384] (seeded), Hq 32 / Hkv 8,
    D 128, page 16, block table a seeded permutation of all pages."""
    import smooth_attn as sa

    B, Hq, Hkv, D, P = 64, 32, 8, 128, 16
    lens, table, n_pages = config5_inputs(torch)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)
    kc = torch.randn(n_pages, Hkv, P, D, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(n_pages, Hkv, P, D, generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, D, generator=gen, device=dev).to(torch.bfloat16)
    table_d = table.to(dev)
    lens_d = lens.to(torch.int32).to(dev)
    kt = time_kernel(torch, lambda: sa.sp2norm_paged_attention(q, kc, vc, table_d, lens_d, block_size=P))
    nbytes = paged_bytes(lens)
    us = kt["median"]
    # the CPU leg gathers its sequences' pages from these device caches
    sample = (q.cpu(), kc, vc, table, lens)
    res = {
        "config": "config5 paged decode, 64 seqs ctx~U[512,16384], Hq32/Hkv8, D128, page16",
        "us": round(us, 2),
        "bytes": nbytes,
        "gbs": round(nbytes / us / 1e3, 1),
        "frac_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
        "times_us": _rounded(kt),
        "sum_ctx": int(lens.sum()),
    }
    return res, sample


def bench_next_rows(torch):
    """The rows built after the hot path, each timed by the same protocol:
    - fp32 fused attention forward and backward on config 3's shape (fp32
      MFMA, against the 157.3 TFLOP/s dense fp32 peak), and at head dims 256
      ([4,16,2048,256]) and 512 ([4,8,2048,512]);
    - bf16 attention forward and backward at head dim 256, [4,16,4096,256],
      and at head dim 512, [4,8,4096,512] (both config 3's FLOPs), and paged decode at head dim 256 on config 5's
      layout with Hq 16 / Hkv 4 (config 5's bytes), at head dim 512 with
      Hq 8 / Hkv 2 and at 1024 with Hq 8 / Hkv 1 (the same bytes), and paged decode over
      fp32 caches (and fp32 q over bf16 and e4m3fn caches, bf16 q over e4m3fn
      caches) on config 5's layout;
    - the bf16 attention backward over long rows and few KV heads
      ([1, 32, 8192, 128] with 8 KV heads, and [1, 16, 16384, 256] with 2),
      with its dK/dV key blocks split over their query tiles (the public
      path) and unsplit;
    - RoPE-fused attention forward on config 3's shape (K rotated once by a
      streaming kernel, Q in registers; the time includes the rotation),
      and the RoPE + W_o projection variant (RoPE forward plus one fp32-
      accumulating GEMM O[B*T, H*D] x W_o[H, D, D_model] viewed as
      [H*D, D_model], D_model = H*D);
    - row-wise and causal softmax (the comparison baselines) on config 2's
      largest shapes: causal bf16 [4,16,4096,4096] (reads the triangle,
      writes the full matrix), row-wise fp32 [64*4096, 4096];
    - the paged-KV writer on config 5's cache: a 1-token decode append and
      a 512-token chunk append for all 64 sequences."""
    import smooth_attn as sa

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    out = {}

    def med(fn, **kw):
        return time_kernel(torch, fn, **kw)["median"]

    B, H, L, D = 4, 32, 4096, 128
    q, k, v = (torch.randn(B, H, L, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(3))
    cos, sin = sa.precompute_rope_cos_sin(D, L, device=dev)
    us = med(lambda: sa.sp2norm_rope_flash_attention(q, k, v, cos, sin))
    fl = attn_flops(B, H, L, D)
    out["rope_attention"] = {"shape": [B, H, L, D], "us": round(us, 1), "tflops": round(fl / us / 1e6, 1),
                             "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                             "note": "includes the K rotation (read + write of K)"}
    d_model = H * D
    w_o = (torch.randn(H, D, d_model, generator=gen, device=dev) / math.sqrt(H * D)).to(torch.bfloat16)
    us = med(lambda: sa.sp2norm_rope_flash_attention_proj(q, k, v, w_o, cos, sin))
    fl_proj = 2 * B * L * (H * D) * d_model
    out["rope_attention_proj"] = {"shape": [B, H, L, D], "d_model": d_model, "us": round(us, 1),
                                  "tflops": round((fl + fl_proj) / us / 1e6, 1),
                                  "frac_bf16_peak": round((fl + fl_proj) / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                                  "flops": fl + fl_proj}
    del q, k, v, w_o
    torch.cuda.empty_cache()

    q, k, v, do = (torch.randn(B, H, L, D, generator=gen, device=dev) for _ in range(4))
    o, rs = sa.kernels._sp2norm_flash_fwd(q, k, v, 1 / math.sqrt(D))
    us_f = med(lambda: sa.kernels._sp2norm_flash_fwd(q, k, v, 1 / math.sqrt(D)))
    us_b = med(lambda: sa.kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, 1 / math.sqrt(D)))
    out["attention_fp32"] = {"shape": [B, H, L, D], "fwd_us": round(us_f, 1), "bwd_us": round(us_b, 1),
                             "fwd_tflops": round(fl / us_f / 1e6, 1), "bwd_tflops": round(2.5 * fl / us_b / 1e6, 1),
                             "fwd_frac_fp32_peak": round(fl / us_f / 1e6 / FP32_PEAK_TFLOPS, 4),
                             "bwd_frac_fp32_peak": round(2.5 * fl / us_b / 1e6 / FP32_PEAK_TFLOPS, 4)}
    del q, k, v, do, o, rs
    torch.cuda.empty_cache()

    # fp32 at head dims 256 and 512 ([4,16,2048,256], [4,8,2048,512]: half of
    # config 3's FLOPs each; their 16-row kernels load tiles straight into LDS)
    for Bf, Hf, Lf, Df in ((4, 16, 2048, 256), (4, 8, 2048, 512)):
        q, k, v, do = (torch.randn(Bf, Hf, Lf, Df, generator=gen, device=dev) for _ in range(4))
        o, rs = sa.kernels._sp2norm_flash_fwd(q, k, v, 1 / math.sqrt(Df))
        us_f = med(lambda: sa.kernels._sp2norm_flash_fwd(q, k, v, 1 / math.sqrt(Df)))
        us_b = med(lambda: sa.kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, 1 / math.sqrt(Df)))
        flf = attn_flops(Bf, Hf, Lf, Df)
        out[f"attention_fp32_d{Df}"] = {"shape": [Bf, Hf, Lf, Df], "fwd_us": round(us_f, 1), "bwd_us": round(us_b, 1),
                                        "fwd_frac_fp32_peak": round(flf / us_f / 1e6 / FP32_PEAK_TFLOPS, 4),
                                        "bwd_frac_fp32_peak": round(2.5 * flf / us_b / 1e6 / FP32_PEAK_TFLOPS, 4)}
        del q, k, v, do, o, rs
        torch.cuda.empty_cache()

    # head dim 256 (its own one-wave-per-SIMD kernels): [4,16,4096,256] has config 3's FLOPs
    q, k, v, do = (torch.randn(4, 16, L, 256, generator=gen, device=dev).to(torch.bfloat16) for _ in range(4))
    o, rs = sa.kernels._sp2norm_flash_fwd(q, k, v, 1 / 16)
    us_f = med(lambda: sa.kernels._sp2norm_flash_fwd(q, k, v, 1 / 16))
    us_b = med(lambda: sa.kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, 1 / 16))
    fl256 = attn_flops(4, 16, L, 256)
    out["attention_d256"] = {"shape": [4, 16, L, 256], "fwd_us": round(us_f, 1), "bwd_us": round(us_b, 1),
                             "fwd_frac_bf16_peak": round(fl256 / us_f / 1e6 / BF16_PEAK_TFLOPS, 4),
                             "bwd_frac_bf16_peak": round(2.5 * fl256 / us_b / 1e6 / BF16_PEAK_TFLOPS, 4)}
    del q, k, v, do, o, rs
    torch.cuda.empty_cache()

    # head dim 512 (4-wave blocks, one wave per SIMD): [4,8,4096,512] has config 3's FLOPs
    q, k, v, do = (torch.randn(4, 8, L, 512, generator=gen, device=dev).to(torch.bfloat16) for _ in range(4))
    sc512 = 1 / math.sqrt(512)
    o, rs = sa.kernels._sp2norm_flash_fwd(q, k, v, sc512)
    us_f = med(lambda: sa.kernels._sp2norm_flash_fwd(q, k, v, sc512), iters=20, warmup=3)
    us_b = med(lambda: sa.kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, sc512), iters=20, warmup=3)
    fl512 = attn_flops(4, 8, L, 512)
    out["attention_d512"] = {"shape": [4, 8, L, 512], "fwd_us": round(us_f, 1), "bwd_us": round(us_b, 1),
                             "fwd_frac_bf16_peak": round(fl512 / us_f / 1e6 / BF16_PEAK_TFLOPS, 4),
                             "bwd_frac_bf16_peak": round(2.5 * fl512 / us_b / 1e6 / BF16_PEAK_TFLOPS, 4)}
    del q, k, v, do, o, rs
    torch.cuda.empty_cache()

    # long rows over few KV heads: bf16 backward at B 1, Hq 32, Hkv 8,
    # T 8192 (512 dK/dV key blocks), with the dK/dV blocks split over their
    # query tiles (the public path) and unsplit (sa_flash_bwd)
    Bl, Hl, Hkl, Tl = 1, 32, 8, 8192
    q, do = (torch.randn(Bl, Hl, Tl, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(Bl, Hkl, Tl, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    sc = 1 / math.sqrt(D)
    o, rs = sa.kernels._sp2norm_flash_fwd(q, k, v, sc, Hl // Hkl)
    us_s = med(lambda: sa.kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, sc, Hl // Hkl), iters=20, warmup=3)
    lib = sa._lib.load()
    grads = [torch.empty_like(t) for t in (q, k, v)]
    delta = torch.empty(Bl, Hl, Tl, device=dev)

    def unsplit():
        st = lib.sa_flash_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), rs.data_ptr(),
                              grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(), delta.data_ptr(), Bl, Hl,
                              Hkl, Tl, D, *(sa._lib.strides(t) for t in (q, k, v, o, do, *grads)), sc, 0, 0,
                              sa._lib.SA_BF16, torch.cuda.current_stream().cuda_stream)
        sa._lib.check(st, "sa_flash_bwd")

    us_u = med(unsplit, iters=20, warmup=3)
    n_split = lib.sa_flash_bwd_workspace_size(Bl, Hl, Hkl, Tl, D, 0, sa._lib.SA_BF16) // (2 * Bl * Hkl * Tl * D * 4)
    fl_l = 2.5 * attn_flops(Bl, Hl, Tl, D)
    out["attention_bwd_long_rows"] = {"shape_q": [Bl, Hl, Tl, D], "kv_heads": Hkl, "n_split": int(n_split),
                                      "bwd_us": round(us_s, 1), "bwd_unsplit_us": round(us_u, 1),
                                      "bwd_frac_bf16_peak": round(fl_l / us_s / 1e6 / BF16_PEAK_TFLOPS, 4),
                                      "bwd_unsplit_frac_bf16_peak": round(fl_l / us_u / 1e6 / BF16_PEAK_TFLOPS, 4)}
    del q, k, v, do, o, rs, grads, delta
    torch.cuda.empty_cache()

    # the same at head dim 256: B 1, Hq 16, Hkv 2, T 16384 (256 dV and 256 dK
    # key blocks of 128 keys), split (the public path) and unsplit
    Bw, Hw, Hkw, Tw, Dw = 1, 16, 2, 16384, 256
    q, do = (torch.randn(Bw, Hw, Tw, Dw, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    k, v = (torch.randn(Bw, Hkw, Tw, Dw, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2))
    sc = 1 / math.sqrt(Dw)
    o, rs = sa.kernels._sp2norm_flash_fwd(q, k, v, sc, Hw // Hkw)
    us_s = med(lambda: sa.kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, sc, Hw // Hkw), iters=10, warmup=2)
    grads = [torch.empty_like(t) for t in (q, k, v)]
    delta = torch.empty(Bw, Hw, Tw, device=dev)

    def unsplit_w():
        st = lib.sa_flash_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), rs.data_ptr(),
                              grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(), delta.data_ptr(), Bw, Hw,
                              Hkw, Tw, Dw, *(sa._lib.strides(t) for t in (q, k, v, o, do, *grads)), sc, 0, 0,
                              sa._lib.SA_BF16, torch.cuda.current_stream().cuda_stream)
        sa._lib.check(st, "sa_flash_bwd")

    us_u = med(unsplit_w, iters=10, warmup=2)
    n_split = lib.sa_flash_bwd_workspace_size(Bw, Hw, Hkw, Tw, Dw, 0, sa._lib.SA_BF16) // (Bw * Hkw * Tw * Dw * 4)
    fl_w = 2.5 * attn_flops(Bw, Hw, Tw, Dw)
    out["attention_bwd_long_rows_d256"] = {"shape_q": [Bw, Hw, Tw, Dw], "kv_heads": Hkw, "n_split": int(n_split),
                                           "bwd_us": round(us_s, 1), "bwd_unsplit_us": round(us_u, 1),
                                           "bwd_frac_bf16_peak": round(fl_w / us_s / 1e6 / BF16_PEAK_TFLOPS, 4),
                                           "bwd_unsplit_frac_bf16_peak": round(fl_w / us_u / 1e6 / BF16_PEAK_TFLOPS, 4)}
    del q, k, v, do, o, rs, grads, delta
    torch.cuda.empty_cache()

    # paged decode at head dim 256 on config 5's layout with Hq 16 / Hkv 4
    # (the same 4 KB of K and V per token as config 5)
    lens, table, n_pages = config5_inputs(torch)
    kc = torch.randn(n_pages, 4, 16, 256, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(n_pages, 4, 16, 256, generator=gen, device=dev).to(torch.bfloat16)
    qd = torch.randn(64, 16, 1, 256, generator=gen, device=dev).to(torch.bfloat16)
    table_d, lens_d = table.to(dev), lens.to(torch.int32).to(dev)
    us = med(lambda: sa.sp2norm_paged_attention(qd, kc, vc, table_d, lens_d))
    nb = paged_bytes(lens, Hq=16, D=256)
    out["paged_decode_d256"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    del kc, vc, qd
    torch.cuda.empty_cache()

    # paged decode at head dim 512 on config 5's layout with Hq 8 / Hkv 2
    # (the same 4 KB of K and V per token; two waves per block split the columns)
    kc = torch.randn(n_pages, 2, 16, 512, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(n_pages, 2, 16, 512, generator=gen, device=dev).to(torch.bfloat16)
    qd = torch.randn(64, 8, 1, 512, generator=gen, device=dev).to(torch.bfloat16)
    us = med(lambda: sa.sp2norm_paged_attention(qd, kc, vc, table_d, lens_d))
    nb = paged_bytes(lens, Hq=8, D=512)
    out["paged_decode_d512"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    del kc, vc, qd
    torch.cuda.empty_cache()

    # paged decode at head dim 1024 on config 5's layout with Hq 8 / Hkv 1
    # (the same 4 KB of K and V per token; four waves per block split the columns)
    kc = torch.randn(n_pages, 1, 16, 1024, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(n_pages, 1, 16, 1024, generator=gen, device=dev).to(torch.bfloat16)
    qd = torch.randn(64, 8, 1, 1024, generator=gen, device=dev).to(torch.bfloat16)
    us = med(lambda: sa.sp2norm_paged_attention(qd, kc, vc, table_d, lens_d))
    nb = paged_bytes(lens, Hq=8, D=1024)
    out["paged_decode_d1024"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                 "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    del kc, vc, qd
    torch.cuda.empty_cache()

    # paged decode over fp32 caches on config 5's layout (8 KB of K and V
    # per token): fp32 q and fp32 q over the bf16 caches
    kc = torch.randn(n_pages, 8, 16, 128, generator=gen, device=dev)
    vc = torch.randn(n_pages, 8, 16, 128, generator=gen, device=dev)
    qd = torch.randn(64, 32, 1, 128, generator=gen, device=dev)
    us = med(lambda: sa.sp2norm_paged_attention(qd, kc, vc, table_d, lens_d))
    n_pg = sum((int(c) + 15) // 16 for c in lens)
    nb = 8192 * int(lens.sum()) + 4 * n_pg + 64 * 32 * 128 * (4 + 2) + 4 * 64  # fp32 K/V and q, bf16 output
    out["paged_decode_fp32"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    us = med(lambda: sa.sp2norm_paged_attention(qd, kc, vc, table_d, lens_d))
    nb = paged_bytes(lens) + 64 * 32 * 128 * 2  # config 5's bytes with a 4-byte q
    out["paged_decode_fp32_q_bf16_cache"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                             "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    # e4m3fn caches (2 KB of K and V per token), read unscaled as the reference reads them
    kc, vc = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
    us = med(lambda: sa.sp2norm_paged_attention(qd, kc, vc, table_d, lens_d))
    nb = 2048 * int(lens.sum()) + 4 * n_pg + 64 * 32 * 128 * (4 + 2) + 4 * 64
    out["paged_decode_fp8_cache"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                     "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    # the same caches under a bf16 q (taken as it is, no fp32 split)
    qb = qd.to(torch.bfloat16)
    us = med(lambda: sa.sp2norm_paged_attention(qb, kc, vc, table_d, lens_d))
    nb = 2048 * int(lens.sum()) + 4 * n_pg + 64 * 32 * 128 * (2 + 2) + 4 * 64
    out["paged_decode_bf16_q_fp8_cache"] = {"us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                            "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    del kc, vc, qd, qb
    torch.cuda.empty_cache()

    Bn, Hn, Ln = 4, 16, 4096
    x = (torch.randn(Bn, Hn, Ln, Ln, generator=gen, device=dev) / math.sqrt(128)).to(torch.bfloat16)
    y = torch.empty_like(x)
    us = med(lambda: sa.softmax_causal_triton_out(y, x))
    nb = Bn * Hn * 2 * (tri(Ln) + Ln * Ln)
    out["softmax_causal_bf16"] = {"shape": [Bn, Hn, Ln, Ln], "us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                  "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    del x, y
    torch.cuda.empty_cache()
    xr = torch.randn(Bn * Hn * Ln, Ln, generator=gen, device=dev)
    yr = torch.empty_like(xr)
    us = med(lambda: sa.softmax_triton_out(yr, xr))
    nb = 2 * xr.numel() * 4
    out["softmax_rowwise_fp32"] = {"shape": list(xr.shape), "us": round(us, 1), "GBs": round(nb / us / 1e3, 1),
                                   "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
    del xr, yr
    torch.cuda.empty_cache()

    Bp, Hkv, P = 64, 8, 16
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(512, 16385, (Bp,), generator=g)
    n_max = 512
    npg = [(int(c) + n_max + P - 1) // P for c in lens]
    n_pages = sum(npg)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    table = torch.zeros(Bp, max(npg), dtype=torch.int32)
    pos = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[pos:pos + n]
        pos += n
    kc = torch.zeros(n_pages, Hkv, P, D, device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    table_d = table.to(dev)
    lens_d = lens.to(torch.int32).to(dev)
    for n_new in (1, n_max):
        kn = torch.randn(Bp, Hkv, n_new, D, generator=gen, device=dev).to(torch.bfloat16)
        vn = torch.randn(Bp, Hkv, n_new, D, generator=gen, device=dev).to(torch.bfloat16)
        us = med(lambda: sa.sp2norm_paged_kv_append(kc, vc, kn, vn, table_d, lens_d, block_size=P))
        nb = 2 * 2 * kn.numel() * 2  # K and V rows, read once and written once
        out[f"paged_append_{n_new}"] = {"seqs": Bp, "n_new": n_new, "us": round(us, 2),
                                        "GBs": round(nb / us / 1e3, 1),
                                        "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
        del kn, vn
    del kc, vc
    torch.cuda.empty_cache()
    return out


def bench_norm_sizes(torch, sa):
    """Config 2 at the other lengths (causal bf16, L = 1024, 2048), its
    row-wise fp32 variant (x, dy fp32 [64 L, L], L = 1024, 2048, 4096) and
    config 1's shape on the GPU: per-kernel medians (caches flushed before
    every launch, so the 128 MiB inputs at L = 1024 come from HBM)."""
    from smooth_attn import FamilyConfig, kernels

    fam = FamilyConfig()
    dev = torch.device("cuda:0")
    out = {"causal_bf16": [], "rowwise_fp32": []}
    for L in (1024, 2048):
        gen = torch.Generator(device=dev).manual_seed(20 + L)
        x = (torch.randn(4, 16, L, L, generator=gen, device=dev) / math.sqrt(128)).to(torch.bfloat16)
        dy = torch.randn(4, 16, L, L, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty_like(x)
        fus = time_kernel(torch, lambda: sa.softplus_norm_causal_triton_out(y, x, family=fam))["median"]
        bus = time_kernel(torch, lambda: kernels._softplus_norm_causal_backward(x, dy, fam))["median"]
        fb, bb = norm_bytes(4, 16, L)
        out["causal_bf16"].append({"L": L, "fwd_us": round(fus, 2), "bwd_us": round(bus, 2),
                                   "GBs": round((fb + bb) / ((fus + bus) * 1e-6) / 1e9, 1),
                                   "frac_hbm_peak": round((fb + bb) / ((fus + bus) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del x, dy, y
    for L in (1024, 2048, 4096):
        gen = torch.Generator(device=dev).manual_seed(30 + L)
        x = torch.randn(64 * L, L, generator=gen, device=dev) / math.sqrt(128)
        dy = torch.randn(64 * L, L, generator=gen, device=dev)
        y = torch.empty_like(x)
        dx = torch.empty_like(x)
        fus = time_kernel(torch, lambda: sa.softplus_norm_triton_out(y, x, family=fam))["median"]
        bus = time_kernel(torch, lambda: kernels._norm_bwd_2d(x, dy, dx, fam, causal=False))["median"]
        fb, bb = 64 * 8 * L * L, 64 * 12 * L * L
        out["rowwise_fp32"].append({"L": L, "fwd_us": round(fus, 2), "bwd_us": round(bus, 2),
                                    "GBs": round((fb + bb) / ((fus + bus) * 1e-6) / 1e9, 1),
                                    "frac_hbm_peak": round((fb + bb) / ((fus + bus) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del x, dy, y, dx
    torch.cuda.empty_cache()
    gen = torch.Generator(device=dev).manual_seed(1)
    x1 = torch.randn(2, 8, 512, 512, generator=gen, device=dev).to(torch.bfloat16)
    y1 = torch.empty_like(x1)
    us1 = time_kernel(torch, lambda: sa.softplus_norm_causal_triton_out(y1, x1, family=fam))["median"]
    b1 = 16 * (2 * tri(512) + 2 * 512 * 512)
    out["config1_gpu_fwd"] = {"shape": [2, 8, 512, 512], "us": round(us1, 2), "bytes": b1,
                              "GBs": round(b1 / (us1 * 1e-6) / 1e9, 1)}
    return out


def bench_norm_rotating(torch, sa):
    """Config 2 at L = 1024 and 2048 (causal bf16), the same kernels as
    ``norm_other_sizes.causal_bf16`` timed back to back over 4 copies of x,
    dy, y and dx (4 x 512 MiB at L = 1024, so each launch's inputs come from
    HBM): 100 launches between one event pair after 100 warm-up launches, the
    median of three such runs.  Runs after the other GPU legs, whose
    allocations it would otherwise reshuffle."""
    from smooth_attn import FamilyConfig, kernels

    fam = FamilyConfig()
    dev = torch.device("cuda:0")
    out = []
    for L in (1024, 2048):
        gen = torch.Generator(device=dev).manual_seed(20 + L)
        copies = []
        for _ in range(4):
            x = (torch.randn(4, 16, L, L, generator=gen, device=dev) / math.sqrt(128)).to(torch.bfloat16)
            dy = torch.randn(4, 16, L, L, generator=gen, device=dev).to(torch.bfloat16)
            copies.append((x, dy, torch.empty_like(x), torch.empty_like(x)))
        fwd_fns = [lambda c=c: sa.softplus_norm_causal_triton_out(c[2], c[0], family=fam) for c in copies]
        bwd_fns = [lambda c=c: kernels._norm_bwd_2d(c[0].view(-1, L), c[1].view(-1, L), c[3].view(-1, L), fam,
                                                    causal=True) for c in copies]
        # median of three timed runs of 100 launches, each after 100 warm-up launches
        fr = sorted(time_rotating(torch, fwd_fns, warmup=100) for _ in range(3))[1]
        br = sorted(time_rotating(torch, bwd_fns, warmup=100) for _ in range(3))[1]
        fb, bb = norm_bytes(4, 16, L)
        out.append({"L": L, "fwd_us": round(fr, 2), "bwd_us": round(br, 2),
                    "GBs": round((fb + bb) / ((fr + br) * 1e-6) / 1e9, 1),
                    "frac_hbm_peak": round((fb + bb) / ((fr + br) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "protocol": "100 back-to-back launches over 4 input/output copies between one event pair, "
                                "after 100 warm-up launches; median of 3"})
        del copies
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# CPU baselines: the reference's eager CPU path, restated in oracle/ (fp32
# torch), on the host cores of the GPU box.
# ---------------------------------------------------------------------------
def cpu_threads(torch):
    """Threads for the CPU legs: the cores this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS when the environment sets
    it (the GPU box grants one GPU's job 16 threads and sets it so).
    Returns the thread count used and a description of the host."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    n = affinity
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    torch.set_num_threads(n)
    return n, {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity, "omp_num_threads": env,
               "torch_threads": torch.get_num_threads(), "cpu_model": cpu_model()}


def _median_wall(fn, budget_s, max_runs=5):
    """Median wall time (s) of fn after one warm-up run: at most max_runs
    runs, fewer when the budget is spent (at least one)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_runs and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_config1(torch, budget_s=10.0):
    """Config 1: the reference's CPU eager forward at full shape
    ([2,8,512,512] bf16), the oracle restatement."""
    from oracle import eager

    x = torch.randn(2, 8, 512, 512, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    med, n = _median_wall(lambda: eager.softplus_norm_causal_cpu_path(x), budget_s, max_runs=7)
    b1 = 16 * (2 * tri(512) + 2 * 512 * 512)
    return {"shape": [2, 8, 512, 512], "ms": round(med * 1e3, 3), "GBs": round(b1 / med / 1e9, 3), "runs": n,
            "threads": torch.get_num_threads()}


def cpu_baseline(torch, sample, threads, budget_s=20.0):
    """Config 2: the reference's eager CPU path (oracle restatement, fp32
    torch) on one [L, L] matrix of the benchmark input: forward + autograd
    backward."""
    from oracle import eager

    x, dy = sample
    L = x.shape[-1]

    def run():
        xr = x.detach().clone().requires_grad_(True)
        y = eager.softplus_norm_causal_eager(xr.float()).to(x.dtype)
        y.backward(dy)
        return xr.grad

    med, n = _median_wall(run, budget_s)
    fwd_b, bwd_b = norm_bytes(1, 1, L)
    return {
        "value": round((fwd_b + bwd_b) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"1 of the 64 [{L},{L}] bf16 matrices of the benchmark input, eager fp32 fwd + autograd bwd, "
                  f"median of {n} runs ({med * 1e3:.0f} ms each); throughput per matrix, which is the "
                  f"whole-config rate since the 64 matrices are independent",
    }


def cpu_attention(torch, sample, threads, budget_s=20.0):
    """Config 3 on the CPU: the restated sp2norm_flash_attention_eager
    (kernels.py:2053-2084) in fp32 on four (b, h) heads of the benchmark's
    inputs (it runs one head at a time); TFLOP/s over the causal triangle,
    as for the GPU figure."""
    from oracle import eager

    q, k, v = (t.float()[None] for t in sample)
    H, L, D = q.shape[1], q.shape[-2], q.shape[-1]
    med, n = _median_wall(lambda: eager.flash_attention_eager(q, k, v), budget_s, max_runs=3)
    fl = attn_flops(1, H, L, D)
    return {"value": round(fl / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{H} of the 128 (b, h) heads of config 3, eager fp32, median of {n} runs "
                      f"({med * 1e3:.0f} ms each; the full config would take about {128 / H * med:.0f} s)"}


def cpu_fp8(torch, sample, threads, budget_s=20.0):
    """Config 4 on the CPU: the restated eager attention in fp32 on the
    dequantised Q/K codes of one query head (and its KV head), bf16 V."""
    from oracle import eager

    q8, k8, v, qs, ks = sample
    qd, kd = (q8.float() * qs)[None, None], (k8.float() * ks)[None, None]
    vd = v.float()[None, None]
    L, D = qd.shape[-2], qd.shape[-1]
    med, n = _median_wall(lambda: eager.flash_attention_eager(qd, kd, vd), budget_s, max_runs=3)
    fl = 2 * 2 * D * tri(L)
    return {"value": round(fl / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"1 of the 64 query heads of config 4 on dequantised fp8 Q/K, eager fp32, median of {n} "
                      f"runs ({med * 1e3:.0f} ms each; about {64 * med:.0f} s for the full config)"}


def cpu_paged(torch, sample, threads, budget_s=30.0):
    """Config 5 on the CPU: the restated decode reference
    (tests/test_paged_long_context.py:39-65, oracle.eager.paged_decode_eager)
    over all 64 sequences, gathering pages through the same block table;
    GB/s over the config's algorithmic bytes."""
    from oracle import eager

    q, kc, vc, table, lens = sample
    kh, vh = kc.cpu(), vc.cpu()
    med, n = _median_wall(lambda: eager.paged_decode_eager(q, kh, vh, table, lens), budget_s, max_runs=3)
    nbytes = paged_bytes(lens)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole config (64 sequences, {int(lens.sum())} context tokens), eager fp32 page "
                      f"gather + decode, median of {n} runs ({med * 1e3:.0f} ms each)"}


def copy_calibration(torch, nbytes=1 << 30):
    """Three plain device-to-device copies of ``nbytes``: under a counter
    profiler their FETCH_SIZE / WRITE_SIZE per dispatch give the scale between
    the counters and bytes moved (each copy reads and writes ``nbytes``)."""
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"bench: copy calibration, 3 copies of {nbytes} bytes")
    del src, dst
    torch.cuda.empty_cache()


def profile_attention(torch, reps=3):
    """The workload of the attention counter profiles: config 3's forward
    and backward and config 4's fp8 forward, ``reps`` launches each on the
    bench's inputs, then the head-dim-256 ([4,16,4096,256] bf16) and fp32
    (config 3's shape) forward and backward, nothing else timed."""
    from smooth_attn import kernels

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    B, H, L, D = 4, 32, 4096, 128
    q, k, v, do = (torch.randn(B, H, L, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    for _ in range(reps):
        o, rs = kernels._sp2norm_flash_fwd(q, k, v, scale)
    for _ in range(reps):
        kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, scale)
    del q, k, v, do, o, rs
    B, Hq, Hkv, L = 2, 32, 8, 8192
    q = torch.randn(B, Hq, L, D, generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, D, generator=gen, device=dev).to(torch.bfloat16)
    q8, qs = kernels._quantize_to_fp8_device(q)
    k8, ks = kernels._quantize_to_fp8_device(k)
    for _ in range(reps):
        kernels._sp2norm_fp8_flash_fwd(q8, k8, v, qs, ks, None, scale, Hq // Hkv)
    del q, k, v, q8, k8
    for (B, H, L, D), dt in (((4, 16, 4096, 256), torch.bfloat16), ((4, 32, 4096, 128), torch.float32)):
        q, k, v, do = (torch.randn(B, H, L, D, generator=gen, device=dev).to(dt) for _ in range(4))
        scale = 1.0 / math.sqrt(D)
        for _ in range(reps):
            o, rs = kernels._sp2norm_flash_fwd(q, k, v, scale)
        for _ in range(reps):
            kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, scale)
        del q, k, v, do, o, rs
    torch.cuda.synchronize()
    log(f"bench: profile workload done ({reps} launches each of flash fwd, flash bwd, fp8 fwd, "
        "head-dim-256 and fp32 fwd and bwd)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 20 untimed steps (about 25 ms): after only 3, the next 20 steps ran
    # about 3% slower than the 20 after them (same kernels, no gaps between
    # launches), so a short warmup times a transient
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run three plain 1 GiB device copies (reference point for HBM counters)")
    ap.add_argument("--profile-attention", action="store_true",
                    help="only launch the attention kernels of configs 3 and 4, head dim 256 and fp32 a few times "
                         "(counter profiles)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the smooth-attn hot path has no multi-GPU component "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    import smooth_attn as sa

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)

    if args.profile_attention:
        profile_attention(torch)
        return
    if args.copy_calibration:
        copy_calibration(torch)
    log("bench: causal norm fwd+bwd [4,16,4096,4096] bf16")
    norm = bench_norm(torch, sa, args.steps, args.warmup)
    log(f"bench: norm {norm['ms_per_step']:.3f} ms/step, fwd {norm['fwd_us']:.1f} us, bwd {norm['bwd_us']:.1f} us")
    attn = fp8 = paged = sizes = nxt = None
    samples = {}
    if not args.no_extra:
        log("bench: fused attention config 3")
        attn, samples["attn"] = bench_attention(torch, sa)
        log(f"bench: attention {attn}")
        log("bench: fp8 attention config 4")
        fp8, samples["fp8"] = bench_fp8(torch)
        log(f"bench: fp8 {fp8}")
        log("bench: paged decode config 5")
        paged, samples["paged"] = bench_paged(torch)
        log(f"bench: paged {paged}")
        log("bench: config 2 other lengths, row-wise fp32, config 1 shape")
        sizes = bench_norm_sizes(torch, sa)
        log(f"bench: sizes {sizes}")
        log("bench: RoPE attention, softmax baselines, paged-KV append")
        nxt = bench_next_rows(torch)
        log(f"bench: next rows {nxt}")
        log("bench: config 2 at L = 1024 / 2048 back to back over rotating copies")
        sizes["causal_bf16_rotating"] = bench_norm_rotating(torch, sa)
        log(f"bench: rotating {sizes['causal_bf16_rotating']}")
    cpu = host = None
    if not args.no_cpu:
        threads, host = cpu_threads(torch)
        log(f"bench: cpu baselines on {threads} threads ({host})")
        cpu = cpu_baseline(torch, norm["sample"], threads)
        log(f"bench: cpu config 2 {cpu['value']} GB/s")
        if sizes is not None:
            sizes["config1_cpu_eager_fwd"] = cpu_config1(torch)
        if attn is not None:
            attn["cpu_baseline"] = cpu_attention(torch, samples["attn"], threads)
            log(f"bench: cpu config 3 {attn['cpu_baseline']}")
        if fp8 is not None:
            fp8["cpu_baseline"] = cpu_fp8(torch, samples["fp8"], threads)
            log(f"bench: cpu config 4 {fp8['cpu_baseline']}")
        if paged is not None:
            paged["cpu_baseline"] = cpu_paged(torch, samples["paged"], threads)
            log(f"bench: cpu config 5 {paged['cpu_baseline']}")
        cpu["host"] = host

    dominant = "bwd" if norm["bwd_us"] >= norm["fwd_us"] else "fwd"
    achieved = norm[f"{dominant}_gbs"]
    line = {
        "metric": METRIC,
        "value": round(norm["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(norm["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "config2: causal squareplus-norm fwd+bwd, bf16 [4,16,4096,4096], alpha=2 theta=0.5 p=2",
            "algorithmic_bytes_per_step": norm["fwd_bytes"] + norm["bwd_bytes"],
            "fwd_us": round(norm["fwd_us"], 2),
            "bwd_us": round(norm["bwd_us"], 2),
            "fwd_GBs": round(norm["fwd_gbs"], 1),
            "bwd_GBs": round(norm["bwd_gbs"], 1),
            "frac_hbm_peak_step": round(norm["gbs"] / HBM_PEAK_GBS, 4),
            "kernel_fwd_us": _rounded(norm["kernel_fwd"]),
            "kernel_bwd_us": _rounded(norm["kernel_bwd"]),
            "kernel_fwd_bwd_frac_hbm_peak": round(
                (norm["fwd_bytes"] + norm["bwd_bytes"]) /
                ((norm["kernel_fwd"]["median"] + norm["kernel_bwd"]["median"]) * 1e3) / HBM_PEAK_GBS, 4),
            "compute_dtype": "f32",
        },
        "roofline": {
            "kernel": f"norm_{dominant}_split<R=4> (causal, bf16, L=4096)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": NORM_TRAFFIC_BYTES[dominant],
        },
        "cpu_baseline": cpu,
        "attention": attn,
        "fp8_attention": fp8,
        "paged_decode": paged,
        "norm_other_sizes": sizes,
        "next_rows": nxt,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
