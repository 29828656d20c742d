"""Head dims below the 16-bit fused-attention kernels' built sizes (GPU).

bf16 / fp16 head dims that are multiples of 8 in 8..512 run on the kernels
built for 32, 64, 128, 256 and 512, which read only the first D columns of every
row and store only those (the reference computes at D_HEAD = next_pow2(D)
and masks no column, kernels.py:1918 and :1572-1581, so for other head dims
its loads run past each row).  Here every input is a
view of a wider tensor whose columns past D hold NaN, so a read of any of
them would turn the results into NaN, and every output is a view of a wider
buffer holding a sentinel, which a store past D would change.  The calls go
through the C ABI with those views' strides.

fp32 head dims that are multiples of 4 run the same way on the fp32 kernels.

Bar as the other attention tests: O within 1e-2 (fp32: 1e-5) of max|oracle|
(float64 oracle), row sums within 1e-5, dQ / dK / dV within 1e-2 (fp32:
1e-5) of max(max|oracle|, 1e-2).
"""
import math

import pytest
import torch

from oracle import eager
from smooth_attn import _lib, kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"
SENTINEL = 7.0


def rel_err(got, ref, floor=1e-30):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / max(float(ref.abs().max()), floor))


def nan_padded(x, extra):
    """x (CPU) as the first D columns of a device tensor whose other columns are NaN."""
    wide = torch.full((*x.shape[:-1], x.shape[-1] + extra), float("nan"), dtype=x.dtype)
    wide[..., :x.shape[-1]] = x
    return wide.to(DEV)[..., :x.shape[-1]]


def sentinel_view(shape, dtype, extra):
    wide = torch.full((*shape[:-1], shape[-1] + extra), SENTINEL, dtype=dtype, device=DEV)
    return wide, wide[..., :shape[-1]]


def fwd(q, k, v, o, rs, scale, window, exact):
    B, Hq, T, D = q.shape
    st = _lib.load().sa_flash_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), rs.data_ptr(), B, Hq, k.shape[1], T, D,
        _lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(o), scale, window, int(exact),
        kernels._DTYPE_CODE[q.dtype], kernels._stream(q))
    _lib.check(st, "sa_flash_fwd")


def bwd(q, k, v, o, do, rs, dq, dk, dv, scale, window, exact):
    B, Hq, T, D = q.shape
    delta = torch.empty(B, Hq, T, dtype=torch.float32, device=DEV)
    st = _lib.load().sa_flash_bwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), rs.data_ptr(), dq.data_ptr(),
        dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), B, Hq, k.shape[1], T, D, _lib.strides(q), _lib.strides(k),
        _lib.strides(v), _lib.strides(o), _lib.strides(do), _lib.strides(dq), _lib.strides(dk), _lib.strides(dv),
        scale, window, int(exact), kernels._DTYPE_CODE[q.dtype], kernels._stream(q))
    _lib.check(st, "sa_flash_bwd")


def run_case(D, dtype, T, window=0, exact=False, extra=24, seed=0):
    B, Hq, Hkv = 1, 4, 2
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    do = torch.randn(B, Hq, T, D, generator=g).to(dtype)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod = (nan_padded(t, extra) for t in (q, k, v, do))
    what = f"D={D} {dtype} T={T} window={window} exact={exact}"

    o_wide, o = sentinel_view(q.shape, dtype, extra)
    rs = torch.empty(B, Hq, T, dtype=torch.float32, device=DEV)
    fwd(qd, kd, vd, o, rs, scale, window, exact)
    torch.cuda.synchronize()
    ref, ref_rs = eager.flash_attention_eager(q.double(), k.double(), v.double(), window_size=window,
                                              return_row_sums=True)
    assert bool((o_wide[..., D:] == SENTINEL).all()), what + ": store past D"
    assert bool(torch.isfinite(o).all()), what + ": O read past D"
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_err(o, ref) <= tol, what
    assert rel_err(rs, ref_rs) <= 1e-5, what

    grads = [sentinel_view(t.shape, dtype, extra) for t in (q, k, v)]
    od = nan_padded(o.cpu(), extra)
    bwd(qd, kd, vd, od, dod, rs, grads[0][1], grads[1][1], grads[2][1], scale, window, exact)
    torch.cuda.synchronize()
    refs = eager.flash_attention_bwd(q.double(), k.double(), v.double(), o.cpu().double(), do.double(),
                                     window_size=window)
    for name, (wide, got), want in zip(("dq", "dk", "dv"), grads, refs):
        assert bool((wide[..., D:] == SENTINEL).all()), f"{what}: {name} store past D"
        assert bool(torch.isfinite(got).all()), f"{what}: {name} read past D"
        err = rel_err(got, want, floor=1e-2)
        assert err <= tol, f"{what}: {name} rel err {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [8, 24, 40, 56, 72, 96, 120])
def test_head_dims_below_128(D, dtype):
    run_case(D, dtype, T=150, seed=D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [136, 168, 200, 248])
def test_head_dims_above_128(D, dtype):
    run_case(D, dtype, T=150, seed=D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [264, 400, 504, 512])
def test_head_dims_above_256(D, dtype):
    # the head-dim-512 kernels (4-wave blocks of 64 rows, 32-row tiles)
    run_case(D, dtype, T=150, seed=D)


def test_head_dim_512_several_blocks():
    # more query / key blocks than one (64 rows each), heaviest first
    run_case(512, torch.bfloat16, T=333, seed=5)


@pytest.mark.parametrize("D", [40, 96, 200, 320, 512])
def test_head_dims_window_and_exact(D):
    run_case(D, torch.bfloat16, T=300, window=70, seed=D + 1)
    run_case(D, torch.bfloat16, T=130, exact=True, extra=8, seed=D + 2)


@pytest.mark.parametrize("D", [4, 20, 36, 48, 100, 132, 200, 252, 260, 400, 508])
def test_fp32_head_dims(D):
    run_case(D, torch.float32, T=150, seed=D + 7)
    run_case(D, torch.float32, T=130, window=33, exact=True, extra=4, seed=D + 8)


@pytest.mark.parametrize("D", [32, 64, 128, 256, 512])
def test_built_head_dims_in_wider_rows(D):
    # D equal to a built size, rows of a wider tensor: nothing read or written past D
    run_case(D, torch.bfloat16, T=200, extra=8, seed=D + 3)
    run_case(D, torch.float32, T=100, extra=4, seed=D + 4)


def test_built_head_dim_512_in_wider_rows():
    run_case(512, torch.float16, T=200, extra=8, seed=515)


def test_public_api_takes_multiples_of_8_without_copies():
    # the autograd entry point runs bf16 D = 96 on the kernels directly: the
    # outputs are the kernels' own tensors (no slicing of a padded result)
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 4, 100, 96, generator=g).to(torch.bfloat16).to(DEV).requires_grad_() for _ in range(3))
    o = kernels.sp2norm_flash_attention(q, k, v)
    assert o.shape == (1, 4, 100, 96) and o.stride() == (4 * 100 * 96, 100 * 96, 96, 1)
    ref = eager.flash_attention_eager(q.detach().cpu().double(), k.detach().cpu().double(),
                                      v.detach().cpu().double())
    assert rel_err(o, ref) <= 1e-2
    o.float().square().sum().backward()
    for t in (q, k, v):
        assert t.grad.shape == t.shape and bool(torch.isfinite(t.grad).all())
