"""Benchmark harness and command line of smooth-attn — reference
kernels.py:2841-3132 (suites, backward validation, reports, argparse, main;
console script ``smooth-attn = smooth_attn.kernels:main``, pyproject.toml:36-37).

Every timed column runs a gfx950 HIP kernel of this package except the
``F.softmax`` / eager columns, which are torch's own GPU kernels (the
comparison the reference makes).  Timing: one HIP event pair per launch,
median (kernels.py:322-336).  Run as ``python -m smooth_attn [args]``.
"""
from __future__ import annotations

import argparse
import math

import torch
import torch.nn.functional as F

from .kernels import (
    DEFAULT_FAMILY,
    SUPPORTED_DTYPES,
    CausalBenchmarkResult,
    FamilyConfig,
    RowwiseBenchmarkResult,
    bench,
    bench_out,
    softmax_causal_eager,
    softmax_causal_triton_out,
    softmax_triton_out,
    softplus_norm_causal,
    softplus_norm_causal_eager,
    softplus_norm_causal_triton_out,
    softplus_norm_triton_out,
)

# kernels.py:30-55
DEFAULT_ROWWISE_SHAPES = (
    (256, 256), (256, 512), (256, 1024), (1024, 256), (1024, 512), (1024, 1024),
    (4096, 128), (4096, 256), (4096, 512), (4096, 1024), (8192, 256), (8192, 512),
    (8192, 1024), (16384, 128), (16384, 256), (16384, 512), (32768, 256), (32768, 512),
    (32, 512), (32, 1024), (32, 2048), (128, 512), (128, 1024), (128, 2048),
)
# kernels.py:56
DEFAULT_CAUSAL_LENGTHS = (128, 256, 512, 1024)


def _current_device_index():
    """kernels.py:123-126."""
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required for these kernels")
    return torch.cuda.current_device()


def _dtype_label(dtype):
    """kernels.py:143-147."""
    for label, candidate in SUPPORTED_DTYPES.items():
        if candidate == dtype:
            return label
    return str(dtype).replace("torch.", "")


def _parse_dtype_list(text):
    """kernels.py:150-157: comma-separated fp32/fp16/bf16."""
    labels = [tok.strip().lower() for tok in text.split(",") if tok.strip()]
    if not labels:
        raise ValueError("at least one dtype must be provided")
    out = []
    for label in labels:
        if label not in SUPPORTED_DTYPES:
            raise ValueError(f"unsupported dtype label: {label}")
        out.append(SUPPORTED_DTYPES[label])
    return out


def _parse_int_list(text):
    """kernels.py:160-164."""
    vals = [tok.strip() for tok in text.split(",") if tok.strip()]
    if not vals:
        raise ValueError("at least one integer must be provided")
    return [int(v) for v in vals]


def benchmark_rowwise_suite(family, shapes=None, warmup=50, iters=200):
    """F.softmax vs the HIP softmax vs the HIP family norm on fp32 rows —
    kernels.py:2841-2867."""
    results = []
    for rows, cols in tuple(shapes or DEFAULT_ROWWISE_SHAPES):
        x = torch.randn(rows, cols, device="cuda")
        out_sm, out_fam = torch.empty_like(x), torch.empty_like(x)
        t_torch = bench(lambda z: F.softmax(z, dim=-1), x, warmup=warmup, iters=iters)
        t_sm = bench_out(softmax_triton_out, out_sm, x, warmup=warmup, iters=iters)
        t_fam = bench_out(lambda o, z: softplus_norm_triton_out(o, z, family=family), out_fam, x,
                          warmup=warmup, iters=iters)
        results.append(RowwiseBenchmarkResult(shape=(rows, cols), torch_softmax_us=t_torch,
                                              triton_softmax_us=t_sm, family_us=t_fam))
    return results


def benchmark_causal_suite(family, dtypes, lengths, batch=2, heads=8, warmup=50, iters=200):
    """Causal [batch, heads, T, T]: eager torch softmax vs the HIP causal
    softmax vs the HIP causal family norm, with errors against fp32 eager and
    row-sum checks — kernels.py:2870-2932."""
    results = []
    for dtype in dtypes:
        for seq_len in lengths:
            x = torch.randn(batch, heads, seq_len, seq_len, device="cuda", dtype=dtype)
            ref_sm = softmax_causal_eager(x.float())
            ref_fam = softplus_norm_causal_eager(x.float(), family=family)
            out_sm, out_fam = torch.empty_like(x), torch.empty_like(x)
            our_sm, sm_meta = softmax_causal_triton_out(out_sm, x, return_meta=True)
            our_fam, fam_meta = softplus_norm_causal_triton_out(out_fam, x, family=family, return_meta=True)
            atol = 1e-4 if dtype == torch.float32 else 5e-3
            ones = torch.ones(batch, heads, seq_len, device=x.device)
            t_torch = bench(softmax_causal_eager, x, warmup=warmup, iters=iters)
            t_sm = bench_out(softmax_causal_triton_out, out_sm, x, warmup=warmup, iters=iters)
            t_fam = bench_out(lambda o, z: softplus_norm_causal_triton_out(o, z, family=family), out_fam, x,
                              warmup=warmup, iters=iters)
            results.append(CausalBenchmarkResult(
                dtype=dtype, batch=batch, heads=heads, seq_len=seq_len,
                torch_softmax_us=t_torch, triton_softmax_us=t_sm, family_us=t_fam,
                softmax_err=float((ref_sm - our_sm.float()).abs().max()),
                family_err=float((ref_fam - our_fam.float()).abs().max()),
                softmax_sums_ok=bool(torch.allclose(our_sm.float().sum(-1), ones, atol=atol)),
                family_sums_ok=bool(torch.allclose(our_fam.float().sum(-1), ones, atol=atol)),
                softmax_meta=sm_meta, family_meta=fam_meta,
            ))
    return results


def validate_causal_backward(family, dtypes, seq_len=128, batch=2, heads=4):
    """Fused causal backward vs autograd of the fp32 eager forward —
    kernels.py:2935-2967."""
    results = []
    for dtype in dtypes:
        x = torch.randn(batch, heads, seq_len, seq_len, device="cuda", dtype=dtype, requires_grad=True)
        up = torch.randn(batch, heads, seq_len, seq_len, device="cuda", dtype=torch.float32)
        (softplus_norm_causal(x, family=family, implementation="triton").float() * up).sum().backward()
        g_hip = x.grad.detach().clone()
        x_ref = x.detach().clone().requires_grad_(True)
        (softplus_norm_causal_eager(x_ref.float(), family=family) * up).sum().backward()
        g_ref = x_ref.grad.detach()
        fp32 = dtype == torch.float32
        results.append({
            "dtype": dtype,
            "max_abs_grad_err": float((g_hip.float() - g_ref.float()).abs().max()),
            "grad_close": bool(torch.allclose(g_hip.float(), g_ref.float(), atol=1e-4 if fp32 else 5e-3,
                                              rtol=1e-3 if fp32 else 5e-2)),
        })
    return results


def _geo_mean(values):
    return math.exp(sum(math.log(v) for v in values) / len(values))


def _print_header(title):
    print("=" * 80)
    print(title)
    print("=" * 80)


def _print_launch_meta(label, meta):
    """kernels.py:2970-2980; every meta of this package carries the launch
    keys, so the reference's KeyError on tiered meta cannot occur."""
    line = (f"  {label}: BLOCK={meta['block_size']} warps={meta['num_warps']} "
            f"stages={meta['num_stages']} progs={meta['num_programs']}")
    if "variant" in meta:
        line += f" variant={meta['variant']}"
    print(line)


def print_rowwise_report(results):
    """kernels.py:2983-3008."""
    print("\n--- Legacy Rowwise Benchmark ---")
    print("  HIP columns use reusable output buffers.")
    print(f"  {'Shape':>18s} {'F.softmax':>10s} {'sm_hip':>10s} {'fam_hip':>11s} {'fam/F.sm':>9s} {'fam/sm_hip':>10s}")
    print("  " + "-" * 74)
    r_torch, r_sm = [], []
    for row in results:
        r_torch.append(row.family_us / row.torch_softmax_us)
        r_sm.append(row.family_us / row.triton_softmax_us)
        print(f"  {str(row.shape):>18s} {row.torch_softmax_us:8.1f}us {row.triton_softmax_us:8.1f}us"
              f" {row.family_us:9.1f}us {r_torch[-1]:7.2f}x {r_sm[-1]:8.2f}x")
    print(f"\n  Geo mean fam_hip / F.softmax:  {_geo_mean(r_torch):.3f}x")
    print(f"  Geo mean fam_hip / softmax_hip: {_geo_mean(r_sm):.3f}x")


def print_causal_report(results, family):
    """kernels.py:3011-3058."""
    print("\n--- Production Causal Benchmark ---")
    print("  HIP columns use reusable output buffers and fp32 arithmetic.")
    print(f"  Family: {family.label}")
    print(f"  {'dtype':>6s} {'B,H,T':>12s} {'torch.sm':>10s} {'sm_hip':>10s} {'fam_hip':>10s}"
          f" {'fam/torch':>10s} {'fam/sm':>8s} {'sm_err':>10s} {'fam_err':>10s}")
    print("  " + "-" * 100)
    grouped = {}
    for row in results:
        label = _dtype_label(row.dtype)
        g = grouped.setdefault(label, ([], []))
        g[0].append(row.family_us / row.torch_softmax_us)
        g[1].append(row.family_us / row.triton_softmax_us)
        print(f"  {label:>6s} {f'{row.batch}x{row.heads}x{row.seq_len}':>12s} {row.torch_softmax_us:8.1f}us"
              f" {row.triton_softmax_us:8.1f}us {row.family_us:8.1f}us {g[0][-1]:8.2f}x {g[1][-1]:7.2f}x"
              f" {row.softmax_err:10.2e} {row.family_err:10.2e}")
    print("\n  Correctness:")
    for row in results:
        print(f"  {_dtype_label(row.dtype):>6s} T={row.seq_len:<4d} softmax_sum={row.softmax_sums_ok}"
              f" family_sum={row.family_sums_ok}")
    print("\n  Geo means by dtype:")
    for label, (vt, vs) in grouped.items():
        print(f"  {label:>6s} fam/torch={_geo_mean(vt):.3f}x fam/sm_hip={_geo_mean(vs):.3f}x")


def parse_args(argv=None):
    """kernels.py:3061-3075 (same options and defaults)."""
    p = argparse.ArgumentParser(description="smooth-attn squareplus benchmark harness (MI355X)")
    p.add_argument("--mode", choices=("causal", "rowwise", "all"), default="causal")
    p.add_argument("--dtypes", default="bf16", help="comma-separated: fp32,fp16,bf16")
    p.add_argument("--lengths", default=",".join(map(str, DEFAULT_CAUSAL_LENGTHS)),
                   help="comma-separated causal sequence lengths")
    p.add_argument("--batch", type=int, default=2)
    p.add_argument("--heads", type=int, default=8)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--iters", type=int, default=200)
    p.add_argument("--alpha", type=float, default=DEFAULT_FAMILY.alpha)
    p.add_argument("--theta", type=float, default=DEFAULT_FAMILY.theta)
    p.add_argument("--power", type=int, default=DEFAULT_FAMILY.power)
    p.add_argument("--quick", action="store_true", help="smaller sweep for iteration speed")
    p.add_argument("--check-backward", action="store_true", help="validate the fused autograd backward")
    return p.parse_args(argv)


def main(argv=None):
    """kernels.py:3078-3128."""
    args = parse_args(argv)
    family = FamilyConfig(alpha=args.alpha, theta=args.theta, power=args.power)
    dtypes = _parse_dtype_list(args.dtypes)
    lengths = _parse_int_list(args.lengths)
    if args.quick:
        lengths = lengths[: min(2, len(lengths))]
        args.warmup = min(args.warmup, 20)
        args.iters = min(args.iters, 100)

    _print_header("SMOOTH-ATTN SQUAREPLUS BENCHMARK (gfx950 HIP)")
    print(f"GPU: {torch.cuda.get_device_name(_current_device_index())}")
    print(f"Family: {family.label}")

    if args.mode in ("rowwise", "all"):
        print_rowwise_report(benchmark_rowwise_suite(family=family, warmup=args.warmup, iters=args.iters))

    if args.mode in ("causal", "all"):
        res = benchmark_causal_suite(family=family, dtypes=dtypes, lengths=lengths, batch=args.batch,
                                     heads=args.heads, warmup=args.warmup, iters=args.iters)
        if res:
            print("\n--- Causal Launch Meta (first case) ---")
            _print_launch_meta("softmax", res[0].softmax_meta)
            _print_launch_meta("family", res[0].family_meta)
        print_causal_report(res, family)

    if args.check_backward:
        print("\n--- Backward Validation ---")
        for row in validate_causal_backward(family=family, dtypes=dtypes, seq_len=lengths[0],
                                            batch=min(args.batch, 2), heads=min(args.heads, 4)):
            print(f"  {_dtype_label(row['dtype']):>6s} grad_close={row['grad_close']}"
                  f" max_abs_grad_err={row['max_abs_grad_err']:.2e}")
    print("\n" + "=" * 80)
