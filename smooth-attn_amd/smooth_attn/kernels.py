"""Public API of smooth-attn on MI355X: same names, signatures, argument
meaning and error behaviour as the reference's ``src/smooth_attn/kernels.py``,
backed by hand-written gfx950 HIP kernels through the C ABI
(include/smooth_attn_amd.h).  There is no Triton and no fallback path: if the
HIP library is missing every GPU entry point raises ``RuntimeError``.

Citations are ``path:line`` into the reference.
"""
from __future__ import annotations

import contextlib
import ctypes
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib

# kernels.py:24-29
SUPPORTED_POWERS = (1, 2, 3)
SUPPORTED_DTYPES = {
    "fp32": torch.float32,
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
}
# kernels.py:57
EPS = 1e-12
# Longest row the fused normalisation kernels take (the reference stops at
# 4096, kernels.py:236-240; the gfx950 kernels hold up to 8192 in registers).
MAX_ROW_COLS = 8192

_DTYPE_CODE = {torch.float32: _lib.SA_F32, torch.float16: _lib.SA_F16, torch.bfloat16: _lib.SA_BF16}


@dataclass(frozen=True)
class FamilyConfig:
    """squareplus(alpha * (x - theta))^power / sum — kernels.py:65-89."""

    alpha: float = 2.0
    theta: float = 0.5
    power: int = 2

    def __post_init__(self):
        if self.power not in SUPPORTED_POWERS:
            raise ValueError(f"power must be one of {SUPPORTED_POWERS}, got {self.power}")

    @property
    def cache_key(self):
        return (float(self.alpha), float(self.theta), int(self.power))

    @property
    def kernel_kwargs(self):
        return {"ALPHA": float(self.alpha), "THETA": float(self.theta), "POWER": int(self.power)}

    @property
    def label(self):
        return f"squareplus({self.alpha:g} * (x - {self.theta:g}))^{self.power} / sum"


@dataclass(frozen=True)
class RowwiseBenchmarkResult:
    """kernels.py:92-97."""

    shape: tuple
    torch_softmax_us: float
    triton_softmax_us: float
    family_us: float


@dataclass(frozen=True)
class CausalBenchmarkResult:
    """kernels.py:100-114."""

    dtype: torch.dtype
    batch: int
    heads: int
    seq_len: int
    torch_softmax_us: float
    triton_softmax_us: float
    family_us: float
    softmax_err: float
    family_err: float
    softmax_sums_ok: bool
    family_sums_ok: bool
    softmax_meta: dict
    family_meta: dict


DEFAULT_FAMILY = FamilyConfig()
BENCH_ALPHA = DEFAULT_FAMILY.alpha
BENCH_THETA = DEFAULT_FAMILY.theta
BENCH_POWER = DEFAULT_FAMILY.power


# ---------------------------------------------------------------------------
# Validation (kernels.py:167-240), same messages and exception types.
# ---------------------------------------------------------------------------
def _resolve_family(alpha, theta, power, family):
    if family is None:
        return FamilyConfig(alpha=alpha, theta=theta, power=power)
    if (alpha, theta, power) != (DEFAULT_FAMILY.alpha, DEFAULT_FAMILY.theta, DEFAULT_FAMILY.power):
        raise ValueError("pass either family=... or alpha/theta/power overrides, not both")
    return family


def _validate_cuda_tensor(x, *, name):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not x.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if x.dtype not in SUPPORTED_DTYPES.values():
        raise ValueError(f"{name} dtype must be one of {tuple(SUPPORTED_DTYPES.values())}, got {x.dtype}")


def _check_same_device(ref_name, ref, **tensors):
    """Every tensor argument of a fused entry point must be a CUDA tensor on
    the device of ``ref`` (the kernels dereference them all as device
    pointers there).  Raised before any launch, with the wording of
    kernels.py:179-187; ``None`` entries (optional arguments) are skipped."""
    for name, t in ((ref_name, ref), *tensors.items()):
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if not t.is_cuda:
            raise ValueError(f"{name} must be a CUDA tensor")
        if t.device != ref.device:
            raise ValueError(f"{name} must live on the same CUDA device as {ref_name} ({ref.device}), "
                             f"got {t.device}")


def _prepare_rowwise_input(x):
    _validate_cuda_tensor(x, name="x")
    if x.ndim != 2:
        raise ValueError(f"row-wise kernels expect a 2D tensor, got shape {tuple(x.shape)}")
    return x if x.is_contiguous() else x.contiguous()


def _prepare_attention_input(x):
    _validate_cuda_tensor(x, name="x")
    if x.ndim < 2:
        raise ValueError("attention scores must have at least 2 dimensions")
    if x.shape[-1] != x.shape[-2]:
        raise ValueError("causal attention expects square score matrices on the last two dims")
    return x if x.is_contiguous() else x.contiguous()


def _prepare_output(out, reference):
    _validate_cuda_tensor(out, name="out")
    if out.shape != reference.shape:
        raise ValueError(f"out shape {tuple(out.shape)} must match input shape {tuple(reference.shape)}")
    if out.dtype != reference.dtype:
        raise ValueError(f"out dtype {out.dtype} must match input dtype {reference.dtype}")
    if out.device != reference.device:
        raise ValueError("out and input must live on the same CUDA device")
    if out.is_contiguous():
        return out, None
    return torch.empty_like(reference), out


def _finalize_output(kernel_out, user_out):
    if user_out is None:
        return kernel_out
    user_out.copy_(kernel_out)
    return user_out


def _check_row_length(n_cols):
    if n_cols > MAX_ROW_COLS:
        raise ValueError(f"n_cols={n_cols} is too large for this fused row kernel")


def _stream(t):
    """The current HIP stream of t's device as a raw handle (without building
    a torch Stream object on every launch)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


_NO_GUARD = contextlib.nullcontext()


def _device_of(t):
    """Context that makes t's device current for the launch: a no-op when it
    already is (the common case), else torch.cuda.device."""
    if t.device.index == torch._C._cuda_getDevice():
        return _NO_GUARD
    return torch.cuda.device(t.device)


def _is_winner_family(family):
    return family.cache_key == DEFAULT_FAMILY.cache_key


_LAUNCH_META_CACHE = {}


def _row_launch_meta(variant, kind, x2d, y2d, rerun, power=2):
    """Launch metadata of a row entry point — the keys of kernels.py:310-317
    and :423-427.  Everything but ``time_us`` describes the kernel the call
    just ran (``sa_*_launch_info``: variant, grid, registers, static LDS,
    resident blocks per CU); ``time_us`` is the median of a few re-runs of
    the same call, measured on the first request per shape and cached, as the
    reference's autotuner measures its candidates on first use."""
    n_rows, n_cols = x2d.shape
    # the variant names the mode (row-wise or causal): same launch, other time
    key = (variant, kind, power, x2d.dtype, n_rows, n_cols, x2d.stride(0), y2d.stride(0),
           x2d.data_ptr() % 16 == 0 and y2d.data_ptr() % 16 == 0, x2d.device.index)
    meta = _LAUNCH_META_CACHE.get(key)
    if meta is None:
        if n_rows == 0 or n_cols == 0:
            meta = {"block_size": 0, "num_warps": 0, "num_stages": 1, "num_programs": 0, "rows_per_program": 0,
                    "waves_per_row": 0, "kernel": None, "occupancy": None, "n_regs": None, "shared_mem": 0,
                    "time_us": None}
        else:
            lib = _lib.load()
            info = _lib.LaunchInfo()
            with _device_of(x2d):
                if kind == "norm":
                    st = lib.sa_norm_fwd_launch_info(x2d.data_ptr(), y2d.data_ptr(), n_rows, n_cols, x2d.stride(0),
                                                     y2d.stride(0), _DTYPE_CODE[x2d.dtype], int(power),
                                                     ctypes.byref(info))
                else:
                    st = lib.sa_softmax_fwd_launch_info(x2d.data_ptr(), y2d.data_ptr(), n_rows, n_cols,
                                                        x2d.stride(0), y2d.stride(0), _DTYPE_CODE[x2d.dtype],
                                                        ctypes.byref(info))
            _lib.check(st, f"sa_{kind}_fwd_launch_info")
            meta = {
                "block_size": info.row_pass_elems,
                "num_warps": info.block_threads // 64,
                "num_stages": 1,
                "num_programs": info.grid_x,
                "rows_per_program": info.rows_per_block,
                "waves_per_row": info.waves_per_row,
                "kernel": _lib.ROW_VARIANTS.get(info.variant, str(info.variant)),
                "occupancy": info.blocks_per_cu,
                "n_regs": info.n_vgprs,
                "shared_mem": info.shared_mem_bytes,
                "time_us": _median_cuda_us(rerun, warmup=2, iters=5),
            }
        _LAUNCH_META_CACHE[key] = meta
    return {"variant": variant, **meta}


# ---------------------------------------------------------------------------
# Row-wise and causal normalisation (forward and fused backward).
# ---------------------------------------------------------------------------
def _norm_fwd_2d(x2d, out2d, family, causal):
    n_rows, n_cols = x2d.shape
    _check_row_length(n_cols)
    lib = _lib.load()
    with _device_of(x2d):
        st = lib.sa_norm_fwd(
            x2d.data_ptr(), out2d.data_ptr(), n_rows, n_cols, x2d.stride(0), out2d.stride(0),
            _DTYPE_CODE[x2d.dtype], 1 if causal else 0, float(family.alpha), float(family.theta),
            int(family.power), _stream(x2d),
        )
    _lib.check(st, "sa_norm_fwd")


def _norm_bwd_2d(x2d, g2d, dx2d, family, causal):
    n_rows, n_cols = x2d.shape
    _check_row_length(n_cols)
    lib = _lib.load()
    with _device_of(x2d):
        st = lib.sa_norm_bwd(
            x2d.data_ptr(), g2d.data_ptr(), dx2d.data_ptr(), n_rows, n_cols, x2d.stride(0),
            g2d.stride(0), dx2d.stride(0), _DTYPE_CODE[x2d.dtype], _DTYPE_CODE[g2d.dtype],
            1 if causal else 0, float(family.alpha), float(family.theta), int(family.power), _stream(x2d),
        )
    _lib.check(st, "sa_norm_bwd")


def softplus_norm_triton(x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                         power=DEFAULT_FAMILY.power, *, family=None, return_meta=False):
    """Row-wise forward into a new tensor — kernels.py:985-1003."""
    family = _resolve_family(alpha, theta, power, family)
    x_row = _prepare_rowwise_input(x)
    out = torch.empty_like(x_row)
    _norm_fwd_2d(x_row, out, family, causal=False)
    if return_meta:
        return out, _row_launch_meta("softplus_norm", "norm", x_row, out,
                                     lambda: _norm_fwd_2d(x_row, out, family, causal=False), family.power)
    return out


def softplus_norm_triton_out(out, x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                             power=DEFAULT_FAMILY.power, *, family=None, return_meta=False):
    """Row-wise forward into ``out`` — kernels.py:1006-1031."""
    family = _resolve_family(alpha, theta, power, family)
    x_row = _prepare_rowwise_input(x)
    kernel_out, user_out = _prepare_output(out, x_row)
    _norm_fwd_2d(x_row, kernel_out, family, causal=False)
    result = _finalize_output(kernel_out, user_out)
    if return_meta:
        return result, _row_launch_meta("softplus_norm", "norm", x_row, kernel_out,
                                        lambda: _norm_fwd_2d(x_row, kernel_out, family, causal=False),
                                        family.power)
    return result


def sp2norm_triton(x, return_meta=False):
    """kernels.py:1034-1035."""
    return softplus_norm_triton(x, family=DEFAULT_FAMILY, return_meta=return_meta)


def softplus_norm_causal_triton_out(out, x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                                    power=DEFAULT_FAMILY.power, *, family=None, return_meta=False):
    """Causal forward into ``out`` — kernels.py:1274-1297.

    One kernel for every family and length: the reference's tiered launches
    and full-matrix ``zero_()`` (kernels.py:1042-1094) are subsumed by causal
    chunk skipping and in-kernel zero fill.
    """
    family = _resolve_family(alpha, theta, power, family)
    x_attn = _prepare_attention_input(x)
    kernel_out, user_out = _prepare_output(out, x_attn)
    seq_len = x_attn.shape[-1]
    x2d = x_attn.view(-1, seq_len)
    o2d = kernel_out.view(-1, seq_len)
    _norm_fwd_2d(x2d, o2d, family, causal=True)
    result = _finalize_output(kernel_out, user_out)
    if return_meta:
        variant = "squareplus_winner" if _is_winner_family(family) else "softplus_norm_causal"
        return result, _row_launch_meta(variant, "norm", x2d, o2d,
                                        lambda: _norm_fwd_2d(x2d, o2d, family, causal=True), family.power)
    return result


def softplus_norm_causal_triton(x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                                power=DEFAULT_FAMILY.power, *, family=None, return_meta=False):
    """Causal forward into a new tensor — kernels.py:1254-1271."""
    family = _resolve_family(alpha, theta, power, family)
    x_attn = _prepare_attention_input(x)
    out = torch.empty_like(x_attn)
    return softplus_norm_causal_triton_out(out, x_attn, family=family, return_meta=return_meta)


def _softplus_norm_causal_backward(x, grad_output, family):
    """Fused causal backward — replaces kernels.py:1197-1230 (dx has x's dtype).

    dy may be fp32 or x's dtype; the kernel reads it directly (no upcast pass).
    """
    _check_same_device("x", x, grad_output=grad_output)
    seq_len = x.shape[-1]
    x2d = x.reshape(-1, seq_len)
    g = grad_output
    if g.dtype not in (torch.float32, x.dtype):
        g = g.float()
    g2d = g.reshape(-1, seq_len)
    if not g2d.is_contiguous():
        g2d = g2d.contiguous()
    dx = torch.empty_like(x2d)
    _norm_bwd_2d(x2d, g2d, dx, family, causal=True)
    return dx.view_as(x)


def _softplus_norm_backward(x, grad_output, family):
    """Fused row-wise backward (the reference has only eager autograd, :1332-1346)."""
    _check_same_device("x", x, grad_output=grad_output)
    g = grad_output if grad_output.dtype in (torch.float32, x.dtype) else grad_output.float()
    g = g.contiguous()
    dx = torch.empty_like(x)
    _norm_bwd_2d(x, g, dx, family, causal=False)
    return dx


class _SoftplusNormCausalAutogradFn(torch.autograd.Function):
    """kernels.py:1373-1398."""

    @staticmethod
    def forward(ctx, x, alpha, theta, power):
        family = FamilyConfig(alpha=float(alpha), theta=float(theta), power=int(power))
        x_attn = _prepare_attention_input(x)
        out = torch.empty_like(x_attn)
        result = softplus_norm_causal_triton_out(out, x_attn, family=family)
        ctx.family = family
        ctx.save_for_backward(x_attn)
        return result

    @staticmethod
    def backward(ctx, grad_output):
        if not ctx.needs_input_grad[0]:
            return None, None, None, None
        (saved_x,) = ctx.saved_tensors
        grad_x = _softplus_norm_causal_backward(saved_x, grad_output.contiguous(), ctx.family)
        return grad_x, None, None, None


def softplus_norm_causal(x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                         power=DEFAULT_FAMILY.power, *, family=None, implementation="triton"):
    """kernels.py:1401-1420.  ``implementation="triton"`` selects the HIP kernels
    (the name is kept for drop-in compatibility); ``"eager"`` is the reference's
    eager formula in fp32, cast back to x's dtype."""
    family = _resolve_family(alpha, theta, power, family)
    if implementation == "triton":
        return _SoftplusNormCausalAutogradFn.apply(x, family.alpha, family.theta, family.power)
    if implementation == "eager":
        return softplus_norm_causal_eager(x.float(), family=family).to(x.dtype)
    raise ValueError("implementation must be 'triton' or 'eager'")


class SoftplusNormCausal(torch.nn.Module):
    """kernels.py:1423-1442."""

    def __init__(self, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta, power=DEFAULT_FAMILY.power,
                 *, family=None, implementation="triton"):
        super().__init__()
        self.family = _resolve_family(alpha, theta, power, family)
        self.implementation = implementation

    def forward(self, x):
        return softplus_norm_causal(x, family=self.family, implementation=self.implementation)


# ---------------------------------------------------------------------------
# Eager formulas (public API of the reference, kernels.py:1328-1370).  These
# are plain torch expressions on whatever device the input lives on; they are
# part of the API surface, not the measured path.
# ---------------------------------------------------------------------------
def _causal_mask(seq_len, device):
    return torch.triu(torch.ones(seq_len, seq_len, device=device, dtype=torch.bool), diagonal=1)


def _apply_family_activation_eager(arg):
    return 0.5 * (arg + torch.sqrt(arg * arg + 4.0))


def softplus_norm_eager(x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                        power=DEFAULT_FAMILY.power, *, family=None):
    family = _resolve_family(alpha, theta, power, family)
    y = _apply_family_activation_eager(family.alpha * (x - family.theta))
    if family.power == 2:
        y = y * y
    elif family.power == 3:
        y = y * y * y
    return y / (y.sum(dim=-1, keepdim=True) + EPS)


def softplus_norm_causal_eager(x, alpha=DEFAULT_FAMILY.alpha, theta=DEFAULT_FAMILY.theta,
                               power=DEFAULT_FAMILY.power, *, family=None):
    family = _resolve_family(alpha, theta, power, family)
    mask = _causal_mask(x.shape[-1], x.device)
    y = _apply_family_activation_eager(family.alpha * (x - family.theta))
    if family.power == 2:
        y = y * y
    elif family.power == 3:
        y = y * y * y
    y = y.masked_fill(mask, 0.0)
    return y / (y.sum(dim=-1, keepdim=True) + EPS)


# ---------------------------------------------------------------------------
# Softmax comparison baselines (kernels.py:1233-1325).
# ---------------------------------------------------------------------------
def _softmax_2d(x2d, out2d, causal):
    n_rows, n_cols = x2d.shape
    _check_row_length(n_cols)
    lib = _lib.load()
    with _device_of(x2d):
        st = lib.sa_softmax_fwd(x2d.data_ptr(), out2d.data_ptr(), n_rows, n_cols, x2d.stride(0), out2d.stride(0),
                                _DTYPE_CODE[x2d.dtype], 1 if causal else 0, _stream(x2d))
    _lib.check(st, "sa_softmax_fwd")


def softmax_triton(x, return_meta=False):
    """Row-wise softmax into a new tensor — kernels.py:1233-1235."""
    x_row = _prepare_rowwise_input(x)
    out = torch.empty_like(x_row)
    _softmax_2d(x_row, out, causal=False)
    if return_meta:
        return out, _row_launch_meta("softmax", "softmax", x_row, out, lambda: _softmax_2d(x_row, out, causal=False))
    return out


def softmax_triton_out(out, x, return_meta=False):
    """Row-wise softmax into ``out`` — kernels.py:1238-1251."""
    x_row = _prepare_rowwise_input(x)
    kernel_out, user_out = _prepare_output(out, x_row)
    _softmax_2d(x_row, kernel_out, causal=False)
    result = _finalize_output(kernel_out, user_out)
    if return_meta:
        return result, _row_launch_meta("softmax", "softmax", x_row, kernel_out,
                                        lambda: _softmax_2d(x_row, kernel_out, causal=False))
    return result


def softmax_causal_triton_out(out, x, return_meta=False):
    """Causal softmax over [..., L, L] into ``out`` (zeros above the
    diagonal) — kernels.py:1312-1325."""
    x_attn = _prepare_attention_input(x)
    kernel_out, user_out = _prepare_output(out, x_attn)
    seq_len = x_attn.shape[-1]
    x2d = x_attn.view(-1, seq_len)
    o2d = kernel_out.view(-1, seq_len)
    _softmax_2d(x2d, o2d, causal=True)
    result = _finalize_output(kernel_out, user_out)
    if return_meta:
        return result, _row_launch_meta("softmax_causal", "softmax", x2d, o2d,
                                        lambda: _softmax_2d(x2d, o2d, causal=True))
    return result


def softmax_causal_triton(x, return_meta=False):
    """Causal softmax into a new tensor — kernels.py:1300-1309."""
    x_attn = _prepare_attention_input(x)
    out = torch.empty_like(x_attn)
    return softmax_causal_triton_out(out, x_attn, return_meta=return_meta)


def softmax_causal_eager(x):
    mask = _causal_mask(x.shape[-1], x.device)
    return F.softmax(x.masked_fill(mask, float("-inf")), dim=-1)


def sp2norm_flash_attention_eager(q, k, v, *, scale=None, window_size=0):
    """Materialised attention — kernels.py:2053-2084."""
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if H_kv < H_q:
        n_groups = H_q // H_kv
        k = k.unsqueeze(2).expand(B, H_kv, n_groups, T, D).reshape(B, H_q, T, D)
        v = v.unsqueeze(2).expand(B, H_kv, n_groups, T, D).reshape(B, H_q, T, D)
    scores = torch.matmul(q.float(), k.float().transpose(-2, -1).contiguous()) * scale
    arg = 2.0 * scores - 1.0
    sp = 0.5 * (arg + torch.sqrt(arg * arg + 4.0))
    y = sp * sp
    y = y.masked_fill(_causal_mask(T, q.device), 0.0)
    if window_size > 0:
        positions = torch.arange(T, device=q.device)
        window_mask = (positions[:, None] - positions[None, :]) >= window_size
        y = y.masked_fill(window_mask.unsqueeze(0).unsqueeze(0), 0.0)
    attn = y / (y.sum(dim=-1, keepdim=True) + EPS)
    return torch.matmul(attn, v.float()).to(q.dtype)


# ---------------------------------------------------------------------------
# Fused attention (bf16 / fp16 / fp32 MFMA).
# ---------------------------------------------------------------------------
_FLASH_HEAD_DIMS = (32, 64, 128)


# Row strides above this are copied first (the kernels address K / V tiles
# with 32-bit offsets).
_MAX_ROW_STRIDE_BYTES = 1 << 24


def _flash_operand(t):
    """The kernels take any (b, h, t) strides that are multiples of 16 bytes
    with a unit stride along D, a 16-byte aligned base and rows at most
    16 MiB apart; anything else is copied to a contiguous tensor first."""
    a = 16 // t.element_size()
    ok = (t.stride(-1) == 1 and all(s % a == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0
          and t.stride(-2) * t.element_size() <= _MAX_ROW_STRIDE_BYTES)
    return t if ok else t.clone(memory_format=torch.contiguous_format)


# Head dims the fused-attention kernels are built for, per input dtype.
_FLASH_KERNEL_DIMS = {torch.bfloat16: (32, 64, 128, 256, 512), torch.float16: (32, 64, 128, 256, 512),
                      torch.float32: (32, 64, 128, 256, 512)}


def _kernel_head_dim(D, dtype=None):
    """The head dim the kernels are called with for a head dim D.  bf16 /
    fp16: D rounded up to a multiple of 8 (kernels built for 32, 64, 128,
    256 and 512), fp32 to a multiple of 4 (kernels built for the same head
    dims); those kernels take any such D up to their size, reading only
    its columns; fp8: the next of the head dims its kernels are built for.  Where it
    differs from D, inputs are zero-padded and outputs sliced: zero columns
    add nothing to q.k, and the padded columns of O, dQ, dK, dV are dropped.
    The reference computes at next_pow2(D) (kernels.py:1918) without masking
    the columns past D."""
    dims = _FLASH_KERNEL_DIMS.get(dtype, _FLASH_HEAD_DIMS)
    if D < 1 or D > dims[-1]:
        raise ValueError(f"fused attention supports head dims 1..{dims[-1]}, got {D}")
    if dtype in (torch.bfloat16, torch.float16):
        return -(-D // 8) * 8
    if dtype == torch.float32:
        return -(-D // 4) * 4
    return next(d for d in dims if d >= D)


def _pad_head_dim(t, Dk):
    return t if t.shape[-1] == Dk else F.pad(t, (0, Dk - t.shape[-1]))


def _check_flash_dtypes(q, k, v):
    """bf16 / fp16 run on the 16-bit MFMA kernels, fp32 on the fp32-MFMA ones
    (products exact in fp32, P and dS kept in fp32)."""
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"fused attention expects bf16, fp16 or fp32 q/k/v of one dtype, got "
                         f"{q.dtype}/{k.dtype}/{v.dtype}")


def _sp2norm_flash_fwd(q, k, v, scale, n_kv_groups=1, window_size=0, use_fast_sqrt=True):
    """(o, row_sums) of the fused forward — replaces kernels.py:1912-1931."""
    _check_same_device("q", q, k=k, v=v)
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    _check_flash_dtypes(q, k, v)
    if H_kv * n_kv_groups != H_q:
        raise ValueError("n_kv_groups must equal H_q // H_kv")
    Dk = _kernel_head_dim(D, q.dtype)
    if Dk != D:
        o, row_sums = _sp2norm_flash_fwd(_pad_head_dim(q, Dk), _pad_head_dim(k, Dk), _pad_head_dim(v, Dk), scale,
                                         n_kv_groups, window_size, use_fast_sqrt)
        return o[..., :D].contiguous(), row_sums
    q, k, v = _flash_operand(q), _flash_operand(k), _flash_operand(v)
    o = torch.empty_like(q)
    if o.stride(-1) != 1:
        o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    row_sums = torch.empty(B, H_q, T, device=q.device, dtype=torch.float32)
    lib = _lib.load()
    with _device_of(q):
        st = lib.sa_flash_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), row_sums.data_ptr(),
            B, H_q, H_kv, T, D, _lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(o),
            float(scale), int(window_size), 0 if use_fast_sqrt else 1, _DTYPE_CODE[q.dtype], _stream(q),
        )
    _lib.check(st, "sa_flash_fwd")
    return o, row_sums


def _sp2norm_flash_bwd(q, k, v, o, do, row_sums, scale, n_kv_groups=1, window_size=0, use_fast_sqrt=True):
    """(dq, dk, dv) of the fused attention — replaces kernels.py:1934-1989."""
    _check_same_device("q", q, k=k, v=v, o=o, do=do, row_sums=row_sums)
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    _check_flash_dtypes(q, k, v)
    Dk = _kernel_head_dim(D, q.dtype)
    if Dk != D:
        pad = [_pad_head_dim(t, Dk) for t in (q, k, v, o, do.to(q.dtype))]
        dq, dk, dv = _sp2norm_flash_bwd(*pad, row_sums, scale, n_kv_groups, window_size, use_fast_sqrt)
        return dq[..., :D].contiguous(), dk[..., :D].contiguous(), dv[..., :D].contiguous()
    q, k, v, o = _flash_operand(q), _flash_operand(k), _flash_operand(v), _flash_operand(o)
    do = _flash_operand(do.to(q.dtype))
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    delta = torch.empty(B, H_q, T, device=q.device, dtype=torch.float32)
    rs = row_sums.contiguous()
    lib = _lib.load()
    # fp32 partials of the dK/dV blocks split over their query tiles (short
    # grids with long causal rows), when the library splits them
    ws_bytes = int(lib.sa_flash_bwd_workspace_size(B, H_q, H_kv, T, D, int(window_size), _DTYPE_CODE[q.dtype]))
    ws = torch.empty(ws_bytes // 4, device=q.device, dtype=torch.float32) if ws_bytes > 0 else None
    with _device_of(q):
        st = lib.sa_flash_bwd_ws(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), rs.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), B, H_q, H_kv, T, D,
            _lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(o), _lib.strides(do),
            _lib.strides(dq), _lib.strides(dk), _lib.strides(dv), float(scale), int(window_size),
            0 if use_fast_sqrt else 1, _DTYPE_CODE[q.dtype], None if ws is None else ws.data_ptr(),
            max(ws_bytes, 0), _stream(q),
        )
    _lib.check(st, "sa_flash_bwd_ws")
    return dq, dk, dv


class _SP2NormFlashAttentionFn(torch.autograd.Function):
    """kernels.py:1992-2013."""

    @staticmethod
    def forward(ctx, q, k, v, scale, n_kv_groups, window_size, use_fast_sqrt):
        o, row_sums = _sp2norm_flash_fwd(q, k, v, scale, n_kv_groups, window_size, use_fast_sqrt=use_fast_sqrt)
        ctx.save_for_backward(q, k, v, o, row_sums)
        ctx.scale = scale
        ctx.n_kv_groups = n_kv_groups
        ctx.window_size = window_size
        ctx.use_fast_sqrt = use_fast_sqrt
        return o

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, o, row_sums = ctx.saved_tensors
        dq, dk, dv = _sp2norm_flash_bwd(q, k, v, o, grad_output, row_sums, ctx.scale, ctx.n_kv_groups,
                                        ctx.window_size, use_fast_sqrt=ctx.use_fast_sqrt)
        return dq, dk, dv, None, None, None, None


def sp2norm_flash_attention(q, k, v, *, scale=None, window_size=0, exact_math=False):
    """Fused causal squareplus attention with autograd, GQA and sliding
    windows — kernels.py:2016-2050."""
    assert q.ndim == 4 and k.ndim == 4 and v.ndim == 4
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    assert k.shape == (B, H_kv, T, D) and v.shape == (B, H_kv, T, D)
    assert H_q % H_kv == 0, f"H_q ({H_q}) must be divisible by H_kv ({H_kv})"
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    n_kv_groups = H_q // H_kv
    return _SP2NormFlashAttentionFn.apply(q, k, v, scale, n_kv_groups, window_size, not exact_math)


# ---------------------------------------------------------------------------
# RoPE-fused attention forwards.
# ---------------------------------------------------------------------------
def precompute_rope_cos_sin(dim, seq_len, base=10000.0, device="cuda", dtype=torch.float32):
    """cos / sin tables [seq_len, dim/2] of rotate-half RoPE — kernels.py:2093-2101."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, device=device).float() / dim))
    t = torch.arange(seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().to(dtype), freqs.sin().to(dtype)


def _rope_tables(cos, sin, T, D):
    """fp32 contiguous, 16-byte aligned tables for the kernel."""
    def fix(t):
        t = t.to(torch.float32)
        ok = t.is_contiguous() and t.data_ptr() % 16 == 0
        return t if ok else t.clone(memory_format=torch.contiguous_format)
    return fix(cos), fix(sin)


def _rope_rotate(x, cos, sin):
    """Rotate-half RoPE of a [B, H, T, D] 16-bit tensor into a new contiguous
    tensor (sa_rope_rotate)."""
    B, H, T, D = x.shape
    x = _flash_operand(x)
    out = torch.empty(B, H, T, D, device=x.device, dtype=x.dtype)
    lib = _lib.load()
    with _device_of(x):
        st = lib.sa_rope_rotate(x.data_ptr(), out.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, H, T, D,
                                _lib.strides(x), _DTYPE_CODE[x.dtype], _stream(x))
    _lib.check(st, "sa_rope_rotate")
    return out


def _sp2norm_rope_flash_fwd(q, k, v, cos, sin, scale, n_kv_groups=1, window_size=0, o=None):
    """(o, row_sums) of the RoPE forward; ``o`` may be a caller view (e.g. of a
    [B, T, Hq, D] buffer) with 16-byte aligned rows.  16-bit head dims 32,
    64 and 128 rotate Q in registers inside the fused kernel (K once into a
    workspace); fp32, and other head dims that are multiples of 16 (up to
    512), rotate Q and K by sa_rope_rotate
    and run the plain fused forward (whose kernels take those head dims
    unpadded, reading only their columns)."""
    _check_same_device("q", q, k=k, v=v, cos=cos, sin=sin, o=o)
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"RoPE attention expects bf16, fp16 or fp32 q/k/v of one dtype, got "
                         f"{q.dtype}/{k.dtype}/{v.dtype}")
    if D % 16 or not 16 <= D <= 512:  # rotate-half pairs 8-element chunks d, d + D/2
        raise ValueError(f"RoPE attention supports head dims that are multiples of 16 in 16..512, got {D}")
    cos, sin = _rope_tables(cos, sin, T, D)
    if D not in _FLASH_HEAD_DIMS or q.dtype == torch.float32:
        o_full, row_sums = _sp2norm_flash_fwd(_rope_rotate(q, cos, sin), _rope_rotate(k, cos, sin), v, scale,
                                              n_kv_groups, window_size)
        if o is None:
            return o_full, row_sums
        o.copy_(o_full)
        return o, row_sums
    q, k, v = _flash_operand(q), _flash_operand(k), _flash_operand(v)
    if o is None:
        o = torch.empty_like(q)
    row_sums = torch.empty(B, H_q, T, device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.sa_flash_rope_workspace_size(B, H_kv, T, D)), 16), dtype=torch.uint8,
                     device=q.device)
    with _device_of(q):
        st = lib.sa_flash_rope_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(), o.data_ptr(),
            row_sums.data_ptr(), ws.data_ptr(), ws.numel(), B, H_q, H_kv, T, D, _lib.strides(q), _lib.strides(k),
            _lib.strides(v), _lib.strides(o), float(scale), int(window_size), _DTYPE_CODE[q.dtype], _stream(q),
        )
    _lib.check(st, "sa_flash_rope_fwd")
    return o, row_sums


def sp2norm_rope_flash_attention(q, k, v, cos, sin, *, scale=None, window_size=0):
    """Fused rotate-half RoPE + squareplus attention forward — kernels.py:2373-2426.

    q, k are un-rotated; cos / sin are [T, D/2] tables
    (precompute_rope_cos_sin).  Q is rotated in registers, K once into a
    workspace; rotated values are rounded to the input type (the reference
    rounds them to bf16 for any input type)."""
    assert q.ndim == 4 and k.ndim == 4 and v.ndim == 4
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    assert H_q % H_kv == 0
    assert D % 2 == 0
    assert cos.shape == (T, D // 2) and sin.shape == (T, D // 2)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o, _ = _sp2norm_rope_flash_fwd(q, k, v, cos, sin, scale, H_q // H_kv, window_size)
    return o


def sp2norm_rope_flash_attention_proj(q, k, v, w_o, cos, sin, *, scale=None, window_size=0):
    """RoPE attention followed by the output projection, [B, T, D_model] —
    kernels.py:2429-2487.

    The attention writes O straight into [B, T, Hq, D] order; the projection
    is then one GEMM O[B*T, Hq*D] x W_o[Hq*D, D_model] with fp32
    accumulation over every head (deterministic), where the reference adds
    per-head bf16 products with atomics."""
    assert q.ndim == 4 and k.ndim == 4 and v.ndim == 4
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    assert H_q % H_kv == 0
    assert D % 2 == 0
    assert w_o.shape[0] == H_q and w_o.shape[1] == D
    _check_same_device("q", q, k=k, v=v, w_o=w_o, cos=cos, sin=sin)
    D_model = w_o.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o_bthd = torch.empty(B, T, H_q, D, device=q.device, dtype=q.dtype)
    _sp2norm_rope_flash_fwd(q, k, v, cos, sin, scale, H_q // H_kv, window_size, o=o_bthd.transpose(1, 2))
    w = w_o.to(q.dtype).reshape(H_q * D, D_model)
    if q.dtype == torch.float32:
        return torch.matmul(o_bthd.view(B * T, H_q * D), w).view(B, T, D_model)
    # W_o^T contiguous: the GEMM then takes its faster layout (F.linear form)
    w_t = _transpose16(w)
    return F.linear(o_bthd.view(B * T, H_q * D), w_t).view(B, T, D_model)


def _transpose16(x):
    """Contiguous transpose of a 2-D bf16/fp16 CUDA matrix by sa_transpose16."""
    assert x.ndim == 2 and x.dtype in (torch.bfloat16, torch.float16)
    _check_same_device("x", x)
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    rows, cols = x.shape
    out = torch.empty(cols, rows, device=x.device, dtype=x.dtype)
    if out.stride(0) % 8:  # rows not a multiple of 8: fall back to a torch copy of the view
        return x.t().contiguous()
    lib = _lib.load()
    with _device_of(x):
        st = lib.sa_transpose16(x.data_ptr(), out.data_ptr(), rows, cols, x.stride(0), out.stride(0), _stream(x))
    _lib.check(st, "sa_transpose16")
    return out


# ---------------------------------------------------------------------------
# fp8 fused attention.
# ---------------------------------------------------------------------------
FP8_MAX = 448.0


def _quantize_to_fp8_device(x):
    """(x8, scale) with the scale left on the device (no host sync)."""
    _check_same_device("x", x)
    if x.dtype not in _DTYPE_CODE:
        raise ValueError(f"cannot quantise dtype {x.dtype}")
    xc = x.detach().contiguous()
    x8 = torch.empty(xc.shape, dtype=torch.float8_e4m3fn, device=x.device)
    ws = torch.empty(2, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    with _device_of(x):
        st = lib.sa_fp8_quantize(xc.data_ptr(), x8.data_ptr(), xc.numel(), _DTYPE_CODE[xc.dtype],
                                 ws.data_ptr(), ws.data_ptr() + 4, _stream(xc))
    _lib.check(st, "sa_fp8_quantize")
    return x8, ws[1]


def _quantize_to_fp8(x):
    """kernels.py:2592-2601: returns (x_fp8, python float scale)."""
    x8, scale = _quantize_to_fp8_device(x)
    return x8, scale.item()


def _scale_tensor(s, device):
    if isinstance(s, torch.Tensor):
        return s.reshape(1).to(device=device, dtype=torch.float32)
    return torch.tensor([float(s)], dtype=torch.float32, device=device)


def _sp2norm_fp8_flash_fwd(q_fp8, k_fp8, v_fp8, q_scale, k_scale, v_scale, attn_scale, n_kv_groups=1,
                           window_size=0):
    """(o, row_sums) of the fp8 forward — replaces kernels.py:2604-2627.

    Scales may be Python floats or device scalars.  ``v_fp8`` may also be a
    bf16 tensor, in which case ``v_scale`` is ignored (PV on bf16 V).
    """
    _check_same_device("q_fp8", q_fp8, k_fp8=k_fp8, v_fp8=v_fp8)
    B, H_q, T, D = q_fp8.shape
    H_kv = k_fp8.shape[1]
    if q_fp8.dtype != torch.float8_e4m3fn or k_fp8.dtype != torch.float8_e4m3fn:
        raise ValueError("q and k must be float8_e4m3fn")
    if v_fp8.dtype not in (torch.float8_e4m3fn, torch.bfloat16):
        raise ValueError("v must be float8_e4m3fn or bfloat16")
    if D < 1 or D > 512:
        raise ValueError(f"fused attention supports head dims 1..512, got {D}")
    if D > 128:
        return _fp8_wide_fwd(q_fp8, k_fp8, v_fp8, q_scale, k_scale, v_scale, attn_scale, n_kv_groups, window_size)
    Dk = _kernel_head_dim(D)
    if Dk != D:
        # zero codes pad the head dim exactly (F.pad works on the bytes)
        pad8 = lambda t: _pad_head_dim(t.view(torch.uint8), Dk).view(t.dtype) if t.dtype == torch.float8_e4m3fn \
            else _pad_head_dim(t, Dk)
        o, row_sums = _sp2norm_fp8_flash_fwd(pad8(q_fp8), pad8(k_fp8), pad8(v_fp8), q_scale, k_scale, v_scale,
                                             attn_scale, n_kv_groups, window_size)
        return o[..., :D].contiguous(), row_sums
    v_code = _lib.SA_FP8_E4M3FN if v_fp8.dtype == torch.float8_e4m3fn else _lib.SA_BF16
    dev = q_fp8.device
    q8, k8, v8 = _flash_operand(q_fp8), _flash_operand(k_fp8), _flash_operand(v_fp8)
    o = torch.empty(B, H_q, T, D, device=dev, dtype=torch.bfloat16)
    row_sums = torch.empty(B, H_q, T, device=dev, dtype=torch.float32)
    qs, ks = _scale_tensor(q_scale, dev), _scale_tensor(k_scale, dev)
    vs = _scale_tensor(1.0 if v_scale is None else v_scale, dev)
    lib = _lib.load()
    with _device_of(q8):
        st = lib.sa_flash_fp8_fwd(
            q8.data_ptr(), k8.data_ptr(), v8.data_ptr(), o.data_ptr(), row_sums.data_ptr(), qs.data_ptr(),
            ks.data_ptr(), vs.data_ptr(), B, H_q, H_kv, T, D, _lib.strides(q8), _lib.strides(k8),
            _lib.strides(v8), _lib.strides(o), float(attn_scale), int(window_size), v_code, _stream(q8),
        )
    _lib.check(st, "sa_flash_fp8_fwd")
    return o, row_sums


def _fp8_wide_fwd(q8, k8, v8, q_scale, k_scale, v_scale, attn_scale, n_kv_groups, window_size):
    """fp8 attention at head dims 129..512: the e4m3fn codes are widened to
    bf16 (exact: every e4m3fn value is a bf16 value), the bf16 head-dim-256
    and -512 kernels run with the dequantisation folded into the score scale
    (q_s * k_s * attn_scale), and fp8 V is widened as v_s * V rounded to
    bf16, so the output is rounded once, at the kernel's store (the
    reference applies v_s to each fp32 P V product, kernels.py:2579;
    rounding V instead leaves per-key errors that average over the keys).
    Device scales are read on the host in one transfer (one
    synchronisation, where the reference's entry point makes three)."""
    scale_v = v8.dtype == torch.float8_e4m3fn and v_scale is not None
    given = [q_scale, k_scale] + ([v_scale] if scale_v else [])
    on_dev = [t.reshape(-1)[:1].float() for t in given if isinstance(t, torch.Tensor)]
    read = iter(torch.cat(on_dev).tolist() if on_dev else [])
    vals = [next(read) if isinstance(t, torch.Tensor) else float(t) for t in given]
    s_eff = float(attn_scale) * vals[0] * vals[1]
    vb = (v8.float() * vals[2]).to(torch.bfloat16) if scale_v else v8.to(torch.bfloat16)
    return _sp2norm_flash_fwd(q8.to(torch.bfloat16), k8.to(torch.bfloat16), vb, s_eff, n_kv_groups, window_size)


def sp2norm_fp8_flash_attention(q, k, v, *, scale=None, window_size=0, quantize_v=True):
    """fp8 fused causal attention — kernels.py:2630-2673.

    Q, K (and V unless ``quantize_v=False``) are quantised per tensor on the
    device; QK^T runs on fp8 MFMA, PV on bf16 MFMA.  ``quantize_v`` (default
    True, as in the reference entry point) is an addition: False keeps V in
    bf16.  Returns bf16; no autograd graph (as in the reference).
    """
    assert q.ndim == 4 and k.ndim == 4 and v.ndim == 4
    B, H_q, T, D = q.shape
    H_kv = k.shape[1]
    assert k.shape == (B, H_kv, T, D) and v.shape == (B, H_kv, T, D)
    assert H_q % H_kv == 0, f"H_q ({H_q}) must be divisible by H_kv ({H_kv})"
    _check_same_device("q", q, k=k, v=v)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    n_kv_groups = H_q // H_kv
    q8, q_s = _quantize_to_fp8_device(q)
    k8, k_s = _quantize_to_fp8_device(k)
    if quantize_v:
        v8, v_s = _quantize_to_fp8_device(v)
    else:
        v8, v_s = v.detach().to(torch.bfloat16), None
    o, _row_sums = _sp2norm_fp8_flash_fwd(q8, k8, v8, q_s, k_s, v_s, scale, n_kv_groups, window_size)
    return o


# ---------------------------------------------------------------------------
# Paged decode.
# ---------------------------------------------------------------------------
def _check_paging_args(B, D, k_cache, v_cache, block_table, context_lens):
    """The kernels read B block-table rows and B context lengths, and cache
    rows of D elements: reject shorter arrays here rather than read past them
    on the device (the reference does not check these)."""
    if k_cache.ndim != 4 or v_cache.shape != k_cache.shape or k_cache.shape[3] != D:
        raise ValueError(f"k/v caches must both be [n_pages, H_kv, block_size, {D}], got "
                         f"{tuple(k_cache.shape)} / {tuple(v_cache.shape)}")
    if block_table.ndim != 2 or block_table.shape[0] < B:
        raise ValueError(f"block_table must be [B={B}, max_pages], got {tuple(block_table.shape)}")
    if context_lens.numel() < B:
        raise ValueError(f"context_lens must hold B={B} lengths, got {context_lens.numel()}")
    for t in (block_table, context_lens):
        if t.dtype.is_floating_point or t.dtype.is_complex or t.device != k_cache.device:
            raise ValueError("block_table and context_lens must be integer tensors on the caches' device")


_PAGED_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_PAGED_CACHE_DTYPES = _PAGED_DTYPES + (torch.float8_e4m3fn,)
_CACHE_CODE = {**_DTYPE_CODE, torch.float8_e4m3fn: _lib.SA_FP8_E4M3FN}


def _paged_dtype_code(q_dtype, k_dtype, v_dtype):
    """The C ABI's dtype argument for a decode over these tensors.  The
    reference upcasts q, K and V to fp32 whatever they are
    (kernels.py:2716-2717, :2746, :2765): here q may be fp32, bf16, fp16 or
    e4m3fn and the caches fp32, bf16, fp16 or e4m3fn (unscaled values, as
    the reference reads them) of one dtype; a q whose dtype differs from the
    caches' runs as fp32 (an exact conversion), except a bf16 q over e4m3fn
    caches, which the kernels take as it is."""
    if (q_dtype not in _PAGED_CACHE_DTYPES or k_dtype not in _PAGED_CACHE_DTYPES or v_dtype != k_dtype):
        raise ValueError("paged decode expects fp32, bf16, fp16 or e4m3fn q and fp32, bf16, fp16 or e4m3fn caches "
                         f"of one dtype, got q {q_dtype}, k_cache {k_dtype}, v_cache {v_dtype}")
    if q_dtype == k_dtype and q_dtype in _PAGED_DTYPES:
        return _DTYPE_CODE[q_dtype]
    if q_dtype == torch.bfloat16 and k_dtype == torch.float8_e4m3fn:
        return _lib.paged_dtypes(_lib.SA_BF16, _lib.SA_FP8_E4M3FN)  # bf16 q as it is
    return _lib.paged_dtypes(_lib.SA_F32, _CACHE_CODE[k_dtype])


def sp2norm_paged_attention(q, k_cache, v_cache, block_table, context_lens, *, scale=None, block_size=16):
    """Paged single-token decode — kernels.py:2776-2829 (output bf16 [B, Hq, D])."""
    assert q.ndim == 4 and q.shape[2] == 1, "Decode: q must be [B, H, 1, D]"
    B, H_q, _, D = q.shape
    H_kv = k_cache.shape[1]
    assert H_q % H_kv == 0
    assert k_cache.shape[2] == block_size and v_cache.shape[2] == block_size
    if block_size < 1 or block_size & (block_size - 1):
        # the reference rounds BLOCK_SIZE up to a power of two and then
        # addresses the pages wrongly (kernels.py:2815, :2737-2743)
        raise ValueError(f"block_size must be a power of two, got {block_size}")
    if D % 8 or not 8 <= D <= 1024:
        # 16-byte cache rows; the reference takes any D through next_pow2 (kernels.py:2814)
        raise ValueError(f"paged decode supports head dims that are multiples of 8 in 8..1024, got {D}")
    if D > 512 and (k_cache.dtype == torch.float32 or (k_cache.dtype == torch.float16 and q.dtype != torch.float16)):
        # those caches are read as bf16 hi + lo tiles, twice the LDS of the 16-bit ones
        raise ValueError(f"paged decode over {k_cache.dtype} caches with a {q.dtype} q supports head dims up to 512, "
                         f"got {D}")
    max_blocks_per_seq = block_table.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    _check_same_device("q", q, k_cache=k_cache, v_cache=v_cache, block_table=block_table,
                       context_lens=context_lens)
    code = _paged_dtype_code(q.dtype, k_cache.dtype, v_cache.dtype)
    if (code & 0xFF) == _lib.SA_F32 and q.dtype != torch.float32:
        q = q.float()  # exact; fp32 q runs over fp32, bf16, fp16 or e4m3fn caches
    if k_cache.dtype == torch.float8_e4m3fn and D % 16:
        raise ValueError(f"paged decode over e4m3fn caches needs a head dim that is a multiple of 16, got {D}")
    _check_paging_args(B, D, k_cache, v_cache, block_table, context_lens)
    q = _flash_operand(q)
    k_cache = _flash_operand(k_cache)
    v_cache = _flash_operand(v_cache)
    block_table = block_table.to(torch.int32)
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    context_lens = context_lens.to(torch.int32).contiguous()
    out = torch.empty(B, H_q, D, device=q.device, dtype=torch.bfloat16)
    lib = _lib.load()
    ws_bytes = lib.sa_paged_decode_workspace_size(B, H_q, D, max_blocks_per_seq, block_size)
    ws = torch.empty(max(1, (ws_bytes + 3) // 4), dtype=torch.float32, device=q.device)
    with _device_of(q):
        st = lib.sa_paged_decode(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), B, H_q, H_kv, D, block_size, max_blocks_per_seq, k_cache.shape[0],
            _lib.strides(q),
            _lib.strides(k_cache), _lib.strides(v_cache), _lib.strides(out), block_table.stride(0),
            float(scale), code, ws.data_ptr(), ws.numel() * 4, _stream(q),
        )
    _lib.check(st, "sa_paged_decode")
    return out


def sp2norm_paged_kv_append(k_cache, v_cache, k_new, v_new, block_table, context_lens, *, block_size=16):
    """Write ``n_new`` new tokens per sequence into the paged caches, at
    positions ``context_lens[b] .. context_lens[b] + n_new - 1`` through the
    block table; returns ``context_lens + n_new`` (a new int32 tensor).

    k_new, v_new: [B, Hkv, n_new, D]; caches [n_pages, Hkv, block_size, D].
    No counterpart in the reference, which builds its caches with Python
    loops (tests/test_paged_attention.py:10-73)."""
    assert k_new.ndim == 4 and v_new.shape == k_new.shape
    B, H_kv, n_new, D = k_new.shape
    assert k_cache.shape[1] == H_kv and k_cache.shape[3] == D and v_cache.shape == k_cache.shape
    assert k_cache.shape[2] == block_size
    _check_same_device("k_cache", k_cache, v_cache=v_cache, k_new=k_new, v_new=v_new, block_table=block_table,
                       context_lens=context_lens)
    if k_cache.dtype not in _PAGED_CACHE_DTYPES or v_cache.dtype != k_cache.dtype:
        raise ValueError("paged caches must be fp32, bf16, fp16 or e4m3fn of one dtype")
    _check_paging_args(B, D, k_cache, v_cache, block_table, context_lens)
    per = 16 // k_cache.element_size()
    for t in (k_cache, v_cache):
        if t.stride(-1) != 1 or any(s % per for s in t.stride()[:-1]) or t.data_ptr() % 16 or D % per:
            raise ValueError("paged caches need 16-byte aligned rows with unit stride along D")
    k_new = _flash_operand(k_new.to(k_cache.dtype))
    v_new = _flash_operand(v_new.to(k_cache.dtype))
    if v_new.stride() != k_new.stride():  # one stride set serves both
        k_new = k_new.clone(memory_format=torch.contiguous_format)
        v_new = v_new.clone(memory_format=torch.contiguous_format)
    block_table = block_table.to(torch.int32)
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    context_lens = context_lens.to(torch.int32).contiguous()
    lib = _lib.load()
    with _device_of(k_cache):
        st = lib.sa_paged_kv_append(
            k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), B, H_kv, n_new, D, block_size, block_table.shape[1], k_cache.shape[0],
            _lib.strides(k_new), _lib.strides(k_cache), _lib.strides(v_cache), block_table.stride(0),
            _CACHE_CODE[k_cache.dtype], _stream(k_cache),
        )
    _lib.check(st, "sa_paged_kv_append")
    return context_lens + n_new


# ---------------------------------------------------------------------------
# Timing helpers (kernels.py:322-336, :2832-2838): one event pair per
# iteration on the current stream, median in microseconds.
# ---------------------------------------------------------------------------
def _median_cuda_us(fn, warmup=300, iters=1000):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) * 1000.0 for s, e in zip(starts, ends))
    return times[len(times) // 2]


def bench(fn, x=None, warmup=300, iters=1000):
    callback = (lambda: fn(x)) if x is not None else fn
    return _median_cuda_us(callback, warmup=warmup, iters=iters)


def bench_out(fn, out, x, warmup=300, iters=1000):
    return _median_cuda_us(lambda: fn(out, x), warmup=warmup, iters=iters)


# ---------------------------------------------------------------------------
# Benchmark harness entry points, also reachable from this module as in the
# reference (console script ``smooth_attn.kernels:main``, pyproject.toml:37);
# the implementation lives in smooth_attn.cli.
# ---------------------------------------------------------------------------
def benchmark_rowwise_suite(family, shapes=None, warmup=50, iters=200):
    """kernels.py:2841-2867."""
    from . import cli
    return cli.benchmark_rowwise_suite(family, shapes=shapes, warmup=warmup, iters=iters)


def benchmark_causal_suite(family, dtypes, lengths, batch=2, heads=8, warmup=50, iters=200):
    """kernels.py:2870-2932."""
    from . import cli
    return cli.benchmark_causal_suite(family, dtypes, lengths, batch=batch, heads=heads, warmup=warmup, iters=iters)


def validate_causal_backward(family, dtypes, seq_len=128, batch=2, heads=4):
    """kernels.py:2935-2967."""
    from . import cli
    return cli.validate_causal_backward(family, dtypes, seq_len=seq_len, batch=batch, heads=heads)


def main(argv=None):
    """kernels.py:3078-3128."""
    from . import cli
    return cli.main(argv)
