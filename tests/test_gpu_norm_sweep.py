"""Randomised parity sweep of the normalisation kernels (row-wise and causal,
forward and fused backward) against the float64 oracle (GPU): random
families (alpha, theta, p = 1..3), dtypes (bf16, fp16, fp32; dy in the input
dtype or fp32), row lengths that take the element, one-wave and split-row
kernels (1 .. 2048, including non-multiples of the 16-byte vector), and
row-padded (strided) views.

Bars as in the per-path tests: 1e-2 (16-bit) or 1e-5 (fp32) of max|oracle|,
causal zeros exact.  The backward's denominator is floored at 1e-3 max|dy|,
the gradients' natural scale: a row of one element (L = 1) has an exactly
vanishing gradient, where the float64 oracle returns about 1e-12 and the
kernels fp32 rounding noise.
"""
import random

import pytest
import torch

import smooth_attn
from oracle import eager
from smooth_attn import FamilyConfig, kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.bfloat16: 1e-2, torch.float16: 1e-2, torch.float32: 1e-5}


def _rel(got, ref, floor=1e-30):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=floor))


@pytest.mark.parametrize("sweep_seed", [21, 22])
def test_random_norm_cases(sweep_seed):
    rng = random.Random(sweep_seed)
    for i in range(30):
        dt = rng.choice([torch.bfloat16, torch.float16, torch.float32])
        gdt = dt if rng.random() < 0.7 else torch.float32
        fam = FamilyConfig(alpha=rng.choice([2.0, 1.5, 0.75, 3.0]), theta=rng.choice([0.5, 0.25, -0.5, 0.0]),
                           power=rng.choice([1, 2, 3]))
        causal = rng.random() < 0.5
        L = rng.choice([1, 3, 8, 63, 64, 65, 255, 511, 512, 513, 1000, 1024, 1500, 2048])
        shape = (rng.choice([1, 2]), 1, L, L) if causal else (rng.choice([1, 2, 5, 17]), L)
        strided = rng.random() < 0.3
        g = torch.Generator().manual_seed(1000 * sweep_seed + i)
        x = (torch.randn(shape, generator=g) * rng.choice([0.5, 1.0, 3.0])).to(dt)
        dy = torch.randn(shape, generator=g).to(gdt)
        what = f"case {i}: {dt} dy {gdt} family {fam.label} causal={causal} shape={shape} strided={strided}"
        xd = x.to(DEV)
        if strided:  # rows padded by 8 elements
            buf = torch.zeros(shape[:-1] + (L + 8,), dtype=dt, device=DEV)
            buf[..., :L] = xd
            xd = buf[..., :L]
        if causal:
            y = smooth_attn.softplus_norm_causal(xd, family=fam)
            ref = eager.softplus_norm_causal_eager(x.double(), fam.alpha, fam.theta, fam.power)
            dx = kernels._softplus_norm_causal_backward(xd, dy.to(DEV), fam)
        else:
            y = smooth_attn.softplus_norm_triton(xd, family=fam)
            ref = eager.softplus_norm_eager(x.double(), fam.alpha, fam.theta, fam.power)
            dx = kernels._softplus_norm_backward(xd, dy.to(DEV), fam)
        dref = eager.softplus_norm_backward(x.double(), dy.double(), fam.alpha, fam.theta, fam.power, causal=causal)
        assert _rel(y, ref) <= TOL[dt], what
        assert _rel(dx, dref, 1e-3 * float(dy.double().abs().max())) <= TOL[dt], what
        if causal:
            up = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
            assert bool((y.cpu()[..., up] == 0).all()) and bool((dx.cpu()[..., up] == 0).all()), what
