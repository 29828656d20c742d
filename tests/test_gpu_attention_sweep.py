"""Randomised parity sweep of the fused attention (forward and backward)
against the float64 oracle, over combinations the fixed cases do not
enumerate: dtype (bf16, fp16, fp32), head dims 8..256 (run on the next
kernel up with the columns past D masked, and the D = 256 kernels), head
dims 260..512 (the D = 512 kernels), GQA
group sizes, windows, query counts around the 32/64/128/256-row tile edges,
and scales (GPU).

Bars, as in the per-path tests: O within 1e-2 (16-bit) or 1e-5 (fp32) of
max|oracle|, row sums within 1e-5, and each gradient within the same bar of
max(max|oracle|, 1e-2).  Where every query sees a single key (T = 1 or
window 1) the exact dQ and dK vanish and the kernels return fp32 rounding
noise of dP - delta, so there dQ and dK are judged against the gradients'
natural scale max|dV| instead.  Backward oracle:
oracle.eager.flash_attention_bwd on GQA-expanded K/V, fed the HIP forward's
O, with dK and dV summed over each group.
"""
import math
import random

import pytest
import torch

from oracle import eager
from smooth_attn import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(got, ref, floor):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / max(float(ref.abs().max()), floor))


def _case(rng, seed, wide=False):
    dt = rng.choice([torch.bfloat16, torch.float16, torch.float32])
    D = rng.choice([260, 264, 328, 400, 448, 512] if wide else [8, 24, 32, 40, 64, 96, 128, 136, 200, 256])
    if D % 8 and dt != torch.float32:
        D += 4  # 16-bit head dims are multiples of 8 here
    hkv = rng.choice([1, 2, 3])
    G = rng.choice([1, 2, 4])
    T = rng.choice([1, 2, 31, 33, 63, 65, 127, 129, 255, 257, 300])
    W = rng.choice([0, 0, 0, 1, 5, 33, 100])
    B = rng.choice([1, 2])
    sc = rng.choice([1 / math.sqrt(D), 0.05, 0.3])
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, hkv * G, T, D, generator=g).to(dt)
    k = torch.randn(B, hkv, T, D, generator=g).to(dt)
    v = torch.randn(B, hkv, T, D, generator=g).to(dt)
    do = torch.randn(B, hkv * G, T, D, generator=g).to(dt)
    return dt, G, W, sc, q, k, v, do


@pytest.mark.parametrize("sweep_seed,n,wide", [(11, 40, False), (12, 40, False), (13, 16, True), (14, 16, True)])
def test_random_attention_cases(sweep_seed, n, wide):
    rng = random.Random(sweep_seed)
    for i in range(n):
        dt, G, W, sc, q, k, v, do = _case(rng, 1000 * sweep_seed + i, wide)
        B, hq, T, D = q.shape
        hkv = k.shape[1]
        what = f"case {i}: {dt} B={B} hq={hq} hkv={hkv} T={T} D={D} window={W} scale={sc:.3g}"
        o, rs = kernels._sp2norm_flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), sc, G, W)
        dq, dk, dv = kernels._sp2norm_flash_bwd(q.to(DEV), k.to(DEV), v.to(DEV), o, do.to(DEV), rs, sc, G, W)
        ke = k.double().repeat_interleave(G, dim=1)
        ve = v.double().repeat_interleave(G, dim=1)
        ref, ref_rs = eager.flash_attention_eager(q.double(), ke, ve, scale=sc, window_size=W, return_row_sums=True)
        rq, rk, rv = eager.flash_attention_bwd(q.double(), ke, ve, o.cpu().double(), do.double(), scale=sc,
                                               window_size=W)
        rk = rk.reshape(B, hkv, G, T, D).sum(2)
        rv = rv.reshape(B, hkv, G, T, D).sum(2)
        tol = 1e-5 if dt == torch.float32 else 1e-2
        single_key = T == 1 or W == 1
        gscale = max(float(rv.abs().max()), 1e-2) if single_key else 1e-2
        assert _rel(o, ref, 1e-30) <= tol, what
        assert _rel(rs, ref_rs, 1e-30) <= 1e-5, what
        assert _rel(dv, rv, 1e-2) <= tol, what
        assert _rel(dq, rq, gscale) <= tol, what
        assert _rel(dk, rk, gscale) <= tol, what
