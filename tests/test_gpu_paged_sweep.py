"""Randomised parity sweep of the paged decode against the float64 oracle
(GPU): random batch sizes, per-sequence context lengths (zero and page-edge
lengths included), page sizes (powers of two), head dims (multiples of 8 up
to 1024; 512 over fp32 caches and under an fp32 q over fp16 caches), GQA
groups, cache dtypes (fp32, bf16, fp16) with q of the caches' dtype or fp32,
and shuffled block tables.

Bar as in test_gpu_paged.py: bf16 output within 1e-2 of max|oracle|;
sequences with an empty context return exact zeros.
"""
import random

import pytest
import torch

import smooth_attn
from oracle import eager, paging

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


@pytest.mark.parametrize("sweep_seed", [31, 32])
def test_random_paged_cases(sweep_seed):
    rng = random.Random(sweep_seed)
    for i in range(25):
        B = rng.choice([1, 2, 3, 7])
        hkv = rng.choice([1, 2, 4])
        hq = hkv * rng.choice([1, 2, 4, 8])
        D = rng.choice([8, 16, 40, 64, 72, 128, 200, 256, 320, 512, 576, 1024])
        P = rng.choice([1, 4, 8, 16, 32, 64, 128])
        dt = rng.choice([torch.bfloat16, torch.float16] if D > 512 else [torch.bfloat16, torch.float16, torch.float32])
        qdt = rng.choice([dt] if D > 512 and dt == torch.float16 else [dt, torch.float32])
        lens = [rng.choice([0, 1, P - 1 if P > 1 else 1, P, P + 1, 100, 257, 1000, 2048]) for _ in range(B)]
        T = max(max(lens), 1)
        g = torch.Generator().manual_seed(1000 * sweep_seed + i)
        q = torch.randn(B, hq, 1, D, generator=g).to(qdt)
        k = torch.randn(B, hkv, T, D, generator=g).to(dt)
        v = torch.randn(B, hkv, T, D, generator=g).to(dt)
        kc, vc, table, lens_t = paging.build_paged_cache(k, v, page_size=P, shuffle=True, generator=g,
                                                         context_lens=lens)
        what = f"case {i}: B={B} hq={hq} hkv={hkv} D={D} page={P} q {qdt} caches {dt} lens={lens}"
        out = smooth_attn.sp2norm_paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), lens_t.to(DEV),
                                                  block_size=P)
        ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens_t)
        live = [b for b in range(B) if lens[b] > 0]
        if live:
            assert _rel(out[live], ref[live]) <= 1e-2, what
        for b in range(B):
            if lens[b] == 0:
                assert bool((out[b] == 0).all()), what
