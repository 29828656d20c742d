"""Benchmark command line of smooth-attn on MI355X: ``python -m smooth_attn``.

The flags and their defaults, and the three benchmark functions with their
signatures and result types, are the reference's interface
(kernels.py:2841-2967, :3061-3128; console script ``smooth-attn``,
pyproject.toml:36-37), so scripts written against it keep working.

What the harness measures and prints is this package's own.  Each case is a
small table of *columns*: the package's HIP launches (writing into a
preallocated output) and torch's own kernel for the same operation.  Every
column is timed the same way (median of per-launch HIP event pairs,
``kernels.bench``), and every HIP column is reported against the bound these
kernels are built for: algorithmic HBM bytes per launch (read x once, only
its causal triangle for causal rows; write the whole output once), the
GB/s that gives, and the fraction of MI355X's 8 TB/s HBM peak.  The torch
column gives the speed ratio, and the causal table adds each HIP output's
error against fp32 eager and whether its rows sum to one.
"""
from __future__ import annotations

import argparse
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .kernels import (
    DEFAULT_FAMILY,
    SUPPORTED_DTYPES,
    CausalBenchmarkResult,
    FamilyConfig,
    RowwiseBenchmarkResult,
    bench,
    softmax_causal_eager,
    softmax_causal_triton,
    softmax_causal_triton_out,
    softmax_triton_out,
    softplus_norm_causal,
    softplus_norm_causal_eager,
    softplus_norm_causal_triton,
    softplus_norm_causal_triton_out,
    softplus_norm_triton_out,
)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E

# The reference's default sweeps (kernels.py:30-56): the row-wise shapes and
# the causal lengths.
DEFAULT_ROWWISE_SHAPES = (
    (256, 256), (256, 512), (256, 1024), (1024, 256), (1024, 512), (1024, 1024),
    (4096, 128), (4096, 256), (4096, 512), (4096, 1024), (8192, 256), (8192, 512),
    (8192, 1024), (16384, 128), (16384, 256), (16384, 512), (32768, 256), (32768, 512),
    (32, 512), (32, 1024), (32, 2048), (128, 512), (128, 1024), (128, 2048),
)
DEFAULT_CAUSAL_LENGTHS = (128, 256, 512, 1024)

# Row sums of a normalised output are 1 up to the rounding of its dtype (the
# bound the result fields *_sums_ok report); gradients are compared with
# allclose at these (atol, rtol).
_SUM_ATOL = {torch.float32: 1e-4, torch.float16: 5e-3, torch.bfloat16: 5e-3}
_GRAD_TOL = {torch.float32: (1e-4, 1e-3), torch.float16: (5e-3, 5e-2), torch.bfloat16: (5e-3, 5e-2)}


def _current_device_index():
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required for these kernels")
    return torch.cuda.current_device()


def _dtype_label(dtype):
    """fp32 / fp16 / bf16, or torch's own name for anything else."""
    names = {v: k for k, v in SUPPORTED_DTYPES.items()}
    return names.get(dtype, str(dtype).replace("torch.", ""))


def _parse_dtype_list(text):
    """Comma-separated dtype labels (case and spaces ignored)."""
    labels = [tok.strip().lower() for tok in text.split(",") if tok.strip()]
    if not labels:
        raise ValueError("at least one dtype must be provided")
    unknown = [lab for lab in labels if lab not in SUPPORTED_DTYPES]
    if unknown:
        raise ValueError(f"unsupported dtype label: {unknown[0]}")
    return [SUPPORTED_DTYPES[lab] for lab in labels]


def _parse_int_list(text):
    vals = [int(tok) for tok in text.split(",") if tok.strip()]
    if not vals:
        raise ValueError("at least one integer must be provided")
    return vals


# ---------------------------------------------------------------------------
# Byte model and columns
# ---------------------------------------------------------------------------
def rowwise_bytes(rows, cols, dtype):
    """Algorithmic HBM bytes of one row-wise launch: read x, write y."""
    return 2 * rows * cols * torch.finfo(dtype).bits // 8


def causal_bytes(n_matrices, seq_len, dtype):
    """Algorithmic HBM bytes of one causal launch over n [L, L] matrices:
    read the causal triangle of x, write the whole output (zeros included)."""
    elem = torch.finfo(dtype).bits // 8
    return n_matrices * elem * (seq_len * (seq_len + 1) // 2 + seq_len * seq_len)


@dataclass
class _Column:
    """One timed launch of a case; ``nbytes`` is set for the HIP columns
    (reported against the HBM roofline) and None for torch's."""

    label: str
    launch: object
    nbytes: int | None = None
    us: float = float("nan")

    def gbs(self):
        return self.nbytes / self.us / 1e3

    def cell(self):
        if self.nbytes is None:
            return f"{self.us:9.1f}"
        return f"{self.us:9.1f} {self.gbs():7.0f} {100 * self.gbs() / HBM_PEAK_GBS:5.1f}%"


def _time_columns(columns, warmup, iters):
    for col in columns:
        col.us = bench(col.launch, warmup=warmup, iters=iters)
    return {col.label: col for col in columns}


# ---------------------------------------------------------------------------
# Suites (signatures and result types of kernels.py:2841-2967)
# ---------------------------------------------------------------------------
_LAST_COLUMNS = {}  # (suite, index) -> timed columns, for the reports


def benchmark_rowwise_suite(family, shapes=None, warmup=50, iters=200):
    """fp32 rows: torch F.softmax, the HIP softmax and the HIP family
    normalisation, each into its own buffer (RowwiseBenchmarkResult per
    shape, times in microseconds)."""
    results = []
    for i, (rows, cols) in enumerate(tuple(shapes or DEFAULT_ROWWISE_SHAPES)):
        x = torch.randn(rows, cols, device="cuda")
        y = torch.empty_like(x)
        nb = rowwise_bytes(rows, cols, x.dtype)
        cols_t = _time_columns([
            _Column("torch", lambda: F.softmax(x, dim=-1)),
            _Column("softmax", lambda: softmax_triton_out(y, x), nb),
            _Column("family", lambda: softplus_norm_triton_out(y, x, family=family), nb),
        ], warmup, iters)
        _LAST_COLUMNS[("rowwise", i)] = cols_t
        results.append(RowwiseBenchmarkResult(shape=(rows, cols), torch_softmax_us=cols_t["torch"].us,
                                              triton_softmax_us=cols_t["softmax"].us,
                                              family_us=cols_t["family"].us))
    return results


def _rows_sum_to_one(y, dtype):
    return bool(((y.float().sum(-1) - 1.0).abs() <= _SUM_ATOL[dtype]).all())


def benchmark_causal_suite(family, dtypes, lengths, batch=2, heads=8, warmup=50, iters=200):
    """Causal [batch, heads, T, T] scores: torch's eager causal softmax, the
    HIP causal softmax and the HIP causal family normalisation.  Accuracy
    (max |HIP - fp32 eager|, rows summing to one) and the launch metadata
    come from one untimed call of each HIP entry point."""
    results = []
    for dtype in dtypes:
        for seq_len in lengths:
            x = torch.randn(batch, heads, seq_len, seq_len, device="cuda", dtype=dtype)
            sm, sm_meta = softmax_causal_triton(x, return_meta=True)
            fam, fam_meta = softplus_norm_causal_triton(x, family=family, return_meta=True)
            sm_err = float((sm.float() - softmax_causal_eager(x.float())).abs().max())
            fam_err = float((fam.float() - softplus_norm_causal_eager(x.float(), family=family)).abs().max())
            sums = (_rows_sum_to_one(sm, dtype), _rows_sum_to_one(fam, dtype))
            del sm, fam
            y = torch.empty_like(x)
            nb = causal_bytes(batch * heads, seq_len, dtype)
            cols_t = _time_columns([
                _Column("torch", lambda: softmax_causal_eager(x)),
                _Column("softmax", lambda: softmax_causal_triton_out(y, x), nb),
                _Column("family", lambda: softplus_norm_causal_triton_out(y, x, family=family), nb),
            ], warmup, iters)
            _LAST_COLUMNS[("causal", len(results))] = cols_t
            results.append(CausalBenchmarkResult(
                dtype=dtype, batch=batch, heads=heads, seq_len=seq_len,
                torch_softmax_us=cols_t["torch"].us, triton_softmax_us=cols_t["softmax"].us,
                family_us=cols_t["family"].us, softmax_err=sm_err, family_err=fam_err,
                softmax_sums_ok=sums[0], family_sums_ok=sums[1], softmax_meta=sm_meta, family_meta=fam_meta))
    return results


def validate_causal_backward(family, dtypes, seq_len=128, batch=2, heads=4):
    """The fused causal backward (through the autograd entry point) against
    autograd of the fp32 eager forward, for the same upstream gradient: a
    dict per dtype with ``dtype``, ``max_abs_grad_err`` and ``grad_close``."""
    out = []
    for dtype in dtypes:
        x = torch.randn(batch, heads, seq_len, seq_len, device="cuda", dtype=dtype)
        upstream = torch.randn(batch, heads, seq_len, seq_len, device="cuda")
        grads = []
        for fwd in (lambda t: softplus_norm_causal(t, family=family, implementation="triton").float(),
                    lambda t: softplus_norm_causal_eager(t.float(), family=family)):
            leaf = x.detach().clone().requires_grad_(True)
            (fwd(leaf) * upstream).sum().backward()
            grads.append(leaf.grad.float())
        atol, rtol = _GRAD_TOL[dtype]
        out.append({"dtype": dtype, "max_abs_grad_err": float((grads[0] - grads[1]).abs().max()),
                    "grad_close": bool(torch.allclose(grads[0], grads[1], atol=atol, rtol=rtol))})
    return out


# ---------------------------------------------------------------------------
# Reports
# ---------------------------------------------------------------------------
def _geomean(values):
    return math.exp(sum(map(math.log, values)) / len(values)) if values else float("nan")


def _kernel_label(meta):
    """The HIP kernel a launch ran: element, one wave per row, or split over
    several waves per row."""
    kind = meta.get("kernel") or "-"
    return f"{kind} x{meta.get('waves_per_row', 1)}"


_HIP_HEAD = f"{'us':>9s} {'GB/s':>7s} {'%HBM':>6s}"


def report_rowwise(results):
    """One line per shape: torch F.softmax time, then each HIP launch as
    time, algorithmic GB/s and fraction of the HBM peak; then how the
    squareplus family compares with F.softmax over the sweep."""
    print("\nrow-wise fp32 (read x + write y per launch)")
    print(f"  {'rows x cols':>13s} | {'torch us':>9s} | softmax {_HIP_HEAD} | family  {_HIP_HEAD} | vs torch")
    speedups = []
    for i, row in enumerate(results):
        cols = _LAST_COLUMNS.get(("rowwise", i))
        if cols is None:  # results not produced by this process's suite: times only
            cols = {"torch": _Column("torch", None, None, row.torch_softmax_us),
                    "softmax": _Column("softmax", None, rowwise_bytes(*row.shape, torch.float32),
                                       row.triton_softmax_us),
                    "family": _Column("family", None, rowwise_bytes(*row.shape, torch.float32), row.family_us)}
        speedups.append(row.torch_softmax_us / row.family_us)
        shape = f"{row.shape[0]} x {row.shape[1]}"
        print(f"  {shape:>13s} | {cols['torch'].cell()} | {cols['softmax'].cell()} | "
              f"{cols['family'].cell()} | {speedups[-1]:5.2f}x")
    print(f"  squareplus family vs torch softmax: geometric mean {_geomean(speedups):.2f}x "
          f"(range {min(speedups):.2f}x .. {max(speedups):.2f}x)")


def report_causal(results, family):
    """Per dtype: one line per length with the torch time, each HIP launch's
    time / GB/s / fraction of the HBM peak, the kernel it ran, its max error
    against fp32 eager and whether its rows sum to one."""
    print(f"\ncausal [B, H, T, T] (read the causal triangle + write all of y per launch); {family.label}")
    by_dtype = {}
    for i, row in enumerate(results):
        by_dtype.setdefault(_dtype_label(row.dtype), []).append((i, row))
    for label, rows in by_dtype.items():
        print(f"  {label}: {'B x H x T':>12s} | {'torch us':>9s} | softmax {_HIP_HEAD} | family  {_HIP_HEAD} | "
              f"{'kernel':>8s} | {'sm err':>8s} {'fam err':>8s} | sums ok | vs torch")
        speedups, fracs = [], []
        for i, row in rows:
            cols = _LAST_COLUMNS.get(("causal", i))
            if cols is None:
                nb = causal_bytes(row.batch * row.heads, row.seq_len, row.dtype)
                cols = {"torch": _Column("torch", None, None, row.torch_softmax_us),
                        "softmax": _Column("softmax", None, nb, row.triton_softmax_us),
                        "family": _Column("family", None, nb, row.family_us)}
            speedups.append(row.torch_softmax_us / row.family_us)
            fracs.append(cols["family"].gbs() / HBM_PEAK_GBS)
            shape = f"{row.batch} x {row.heads} x {row.seq_len}"
            ok = "yes" if row.softmax_sums_ok and row.family_sums_ok else "NO"
            print(f"  {'':{len(label)}s}  {shape:>12s} | {cols['torch'].cell()} | {cols['softmax'].cell()} | "
                  f"{cols['family'].cell()} | {_kernel_label(row.family_meta):>8s} | {row.softmax_err:8.1e} "
                  f"{row.family_err:8.1e} | {ok:>7s} | {speedups[-1]:5.2f}x")
        print(f"  {label}: squareplus family vs torch softmax: geometric mean {_geomean(speedups):.2f}x; "
              f"family at {100 * _geomean(fracs):.1f}% of the HBM peak (geometric mean)")


def report_backward(rows):
    print("\nfused causal backward vs autograd of the fp32 eager forward")
    for row in rows:
        print(f"  {_dtype_label(row['dtype']):>5s}: max |grad err| {row['max_abs_grad_err']:.2e}, "
              f"close: {'yes' if row['grad_close'] else 'NO'}")


# Names of the reference's report functions (kernels.py:2983-3058), kept for
# callers that print results themselves.
def print_rowwise_report(results):
    report_rowwise(results)


def print_causal_report(results, family):
    report_causal(results, family)


# ---------------------------------------------------------------------------
# Command line (flags and defaults of kernels.py:3061-3075)
# ---------------------------------------------------------------------------
def parse_args(argv=None):
    p = argparse.ArgumentParser(description="smooth-attn squareplus benchmark harness (MI355X, HIP)")
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
    args = parse_args(argv)
    family = FamilyConfig(alpha=args.alpha, theta=args.theta, power=args.power)
    dtypes = _parse_dtype_list(args.dtypes)
    lengths = _parse_int_list(args.lengths)
    warmup, iters = args.warmup, args.iters
    if args.quick:  # the first two lengths, shorter timing loops
        lengths = lengths[:2]
        warmup, iters = min(warmup, 20), min(iters, 100)
    dev = _current_device_index()
    print(f"smooth-attn benchmark on {torch.cuda.get_device_name(dev)} (HIP kernels for gfx950); "
          f"HBM peak {HBM_PEAK_GBS / 1000:.0f} TB/s; median of {iters} launches after {warmup} warm-up")
    if args.mode in ("rowwise", "all"):
        report_rowwise(benchmark_rowwise_suite(family, warmup=warmup, iters=iters))
    if args.mode in ("causal", "all"):
        report_causal(benchmark_causal_suite(family, dtypes, lengths, batch=args.batch, heads=args.heads,
                                             warmup=warmup, iters=iters), family)
    if args.check_backward:
        report_backward(validate_causal_backward(family, dtypes, seq_len=lengths[0], batch=min(args.batch, 2),
                                                 heads=min(args.heads, 4)))
