"""The attention backward with dK / dV key blocks split over their query
tiles (sa_flash_bwd_ws), GPU, on the kernels for head dims up to 128 and
for head dims 136..512.

Causally, key block j of the dK/dV kernel sees the query tiles from j on, so
the first blocks hold the most work; where B x Hkv is small the library
splits every block's (head, query tile) iterations n_split ways, writes fp32
partials to the workspace and sums them in one more kernel.  Checked here:
- against the float64 oracle (oracle.eager.flash_attention_bwd on
  GQA-expanded K/V, dK / dV summed over each group) at the 16-bit bar, 1e-2
  of max(max|oracle|, 1e-2), with windows, exact square roots, head dims
  below the kernel's (inputs NaN past D, outputs holding a sentinel there)
  and splits holding no iteration;
- against the unsplit path (sa_flash_bwd) on the same inputs: dQ identical
  (the same kernel), dK / dV within two bf16 steps of max|dK|, max|dV| (the
  partial sums differ from one running sum only in fp32 rounding before the
  final rounding to the 16-bit type), for every split count the workspace
  size allows, and at config-like long-context sizes the oracle is too slow
  for;
- that the same call twice gives identical results (the sum runs in a fixed
  order).
"""
import ctypes
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
    wide = torch.full((*x.shape[:-1], x.shape[-1] + extra), float("nan"), dtype=x.dtype)
    wide[..., :x.shape[-1]] = x
    return wide.to(DEV)[..., :x.shape[-1]]


def sentinel_view(shape, dtype, extra):
    wide = torch.full((*shape[:-1], shape[-1] + extra), SENTINEL, dtype=dtype, device=DEV)
    return wide, wide[..., :shape[-1]]


def ws_size(q, k, window):
    B, Hq, T, D = q.shape
    return int(_lib.load().sa_flash_bwd_workspace_size(B, Hq, k.shape[1], T, D, window, kernels._DTYPE_CODE[q.dtype]))


def bwd(q, k, v, o, do, rs, grads, scale, window, exact, ws_bytes):
    """One C-ABI backward into the (dq, dk, dv) views grads; ws_bytes None: sa_flash_bwd."""
    B, Hq, T, D = q.shape
    dq, dk, dv = grads
    delta = torch.empty(B, Hq, T, dtype=torch.float32, device=DEV)
    lib = _lib.load()
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), rs.data_ptr(), dq.data_ptr(),
            dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), B, Hq, k.shape[1], T, D, _lib.strides(q),
            _lib.strides(k), _lib.strides(v), _lib.strides(o), _lib.strides(do), _lib.strides(dq), _lib.strides(dk),
            _lib.strides(dv), scale, window, int(exact), kernels._DTYPE_CODE[q.dtype])
    if ws_bytes is None:
        st = lib.sa_flash_bwd(*args, kernels._stream(q))
    else:
        ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=DEV)
        st = lib.sa_flash_bwd_ws(*args, ctypes.c_void_p(ws.data_ptr()), ws_bytes, kernels._stream(q))
    _lib.check(st, "sa_flash_bwd_ws")
    torch.cuda.synchronize()


def inputs(B, Hq, Hkv, T, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    do = torch.randn(B, Hq, T, D, generator=g).to(dtype)
    return q, k, v, do


def forward(qd, kd, vd, scale, G, window):
    o, rs = kernels._sp2norm_flash_fwd(qd, kd, vd, scale, G, window)
    return o, rs


@pytest.mark.parametrize("B,Hq,Hkv,T,D,window,exact,dtype", [
    (1, 4, 2, 333, 40, 0, False, torch.bfloat16),
    (1, 4, 2, 333, 40, 70, False, torch.bfloat16),
    (2, 2, 1, 300, 64, 0, True, torch.float16),
    (1, 8, 2, 520, 128, 0, False, torch.bfloat16),
    (1, 3, 1, 257, 96, 33, False, torch.float16),
    (1, 2, 1, 1, 32, 0, False, torch.bfloat16),
    # the head-dim-256 and -512 kernels (dK and dV kernels one after the other)
    (1, 4, 2, 333, 200, 0, False, torch.bfloat16),
    (1, 4, 1, 300, 256, 64, False, torch.float16),
    (1, 2, 1, 260, 400, 0, True, torch.bfloat16),
    (1, 2, 2, 200, 512, 0, False, torch.bfloat16),
    (1, 2, 1, 1, 256, 0, False, torch.bfloat16),
])
def test_split_matches_oracle(B, Hq, Hkv, T, D, window, exact, dtype):
    q, k, v, do = inputs(B, Hq, Hkv, T, D, dtype, seed=T + D)
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    n = ws_size(q, k, window)
    assert n > 0, "these sizes split"
    extra = 8
    qd, kd, vd, dod = (nan_padded(t, extra) for t in (q, k, v, do))
    o, rs = forward(q.to(DEV), k.to(DEV), v.to(DEV), scale, G, window)
    od = nan_padded(o.cpu(), extra)
    grads = [sentinel_view(t.shape, dtype, extra) for t in (q, k, v)]
    bwd(qd, kd, vd, od, dod, rs, [g[1] for g in grads], scale, window, exact, n)
    ke = k.double().repeat_interleave(G, dim=1)
    ve = v.double().repeat_interleave(G, dim=1)
    rq, rk, rv = eager.flash_attention_bwd(q.double(), ke, ve, o.cpu().double(), do.double(), scale=scale,
                                           window_size=window)
    rk = rk.reshape(B, Hkv, G, T, D).sum(2)
    rv = rv.reshape(B, Hkv, G, T, D).sum(2)
    # every query sees a single key only at T = 1: there dQ and dK are rounding noise
    gscale = max(float(rv.abs().max()), 1e-2) if T == 1 else 1e-2
    what = f"B={B} Hq={Hq} Hkv={Hkv} T={T} D={D} window={window} exact={exact} {dtype} ws={n}"
    for name, (wide, got), want, floor in zip(("dq", "dk", "dv"), grads, (rq, rk, rv), (gscale, gscale, 1e-2)):
        assert bool((wide[..., D:] == SENTINEL).all()), f"{what}: {name} store past D"
        assert bool(torch.isfinite(got).all()), f"{what}: {name} read past D"
        err = rel_err(got, want, floor)
        assert err <= 1e-2, f"{what}: {name} rel err {err:.3e}"


def split_unit(B, Hkv, T, D):
    """Workspace bytes per split: fp32 partials of dK and dV at the kernel's
    head dim (32, 64, 128), or one buffer the dK and dV kernels of head dim
    256 / 512 take in turn."""
    kd = next(d for d in (32, 64, 128, 256, 512) if D <= d)
    return (2 if kd <= 128 else 1) * B * Hkv * T * kd * 4


def close_to_unsplit(got, ref):
    """max |got - ref| within two bf16 steps of max|ref|."""
    scale = float(ref.float().abs().max())
    return float((got.float() - ref.float()).abs().max()) <= 2 * 2.0 ** -7 * max(scale, 1e-30)


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [(1, 8, 2, 700, 128), (1, 4, 1, 1000, 64), (2, 4, 2, 640, 32),
                                         (1, 8, 2, 1000, 256), (1, 4, 1, 900, 448), (2, 2, 1, 640, 512)])
def test_every_split_count_matches_unsplit(B, Hq, Hkv, T, D):
    dtype = torch.bfloat16
    q, k, v, do = (t.to(DEV) for t in inputs(B, Hq, Hkv, T, D, dtype, seed=B * T))
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    o, rs = forward(q, k, v, scale, G, 0)
    base = [torch.empty_like(t) for t in (q, k, v)]
    bwd(q, k, v, o, do, rs, base, scale, 0, False, None)
    n = ws_size(q, k, 0)
    unit = split_unit(B, Hkv, T, D)
    assert n > 0 and n % unit == 0
    splits = n // unit
    seen = 0
    while splits >= 1:
        got = [torch.empty_like(t) for t in (q, k, v)]
        bwd(q, k, v, o, do, rs, got, scale, 0, False, splits * unit if splits > 1 else 0)
        assert torch.equal(got[0], base[0]), splits
        assert close_to_unsplit(got[1], base[1]) and close_to_unsplit(got[2], base[2]), splits
        splits //= 2
        seen += 1
    assert seen >= 2


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [(1, 32, 8, 8192, 128), (1, 8, 1, 32768, 128), (1, 16, 2, 16384, 256),
                                         (1, 8, 1, 16384, 512)])
def test_long_context_split_matches_unsplit(B, Hq, Hkv, T, D):
    # config-like long rows over few KV heads (the split's case)
    dtype = torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(T)
    q = torch.randn(B, Hq, T, D, generator=g, device=DEV).to(dtype)
    k = torch.randn(B, Hkv, T, D, generator=g, device=DEV).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g, device=DEV).to(dtype)
    do = torch.randn(B, Hq, T, D, generator=g, device=DEV).to(dtype)
    scale = 1.0 / math.sqrt(D)
    o, rs = forward(q, k, v, scale, Hq // Hkv, 0)
    n = ws_size(q, k, 0)
    assert n > 0
    base = [torch.empty_like(t) for t in (q, k, v)]
    bwd(q, k, v, o, do, rs, base, scale, 0, False, None)
    got = [torch.empty_like(t) for t in (q, k, v)]
    bwd(q, k, v, o, do, rs, got, scale, 0, False, n)
    assert torch.equal(got[0], base[0])
    assert close_to_unsplit(got[1], base[1]) and close_to_unsplit(got[2], base[2])
    again = [torch.empty_like(t) for t in (q, k, v)]
    bwd(q, k, v, o, do, rs, again, scale, 0, False, n)
    assert all(torch.equal(a, b) for a, b in zip(again, got))
    # the public entry point takes the split path
    dq, dk, dv = kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, scale, Hq // Hkv)
    assert torch.equal(dk, got[1]) and torch.equal(dv, got[2])
