"""Writes the golden fixtures of tests/golden/*.npz from the CPU oracle.

The reference commits no golden vectors (its tests draw unseeded CUDA inputs
and compare against its eager functions at run time), so these fixtures are
this repository's own: small seeded inputs, exactly representable in bf16
(stored as float32), and the oracle's float64 outputs.  The oracle itself is
pinned by tests/test_oracle.py (brute-force loops, closed forms, invariants,
finite differences); tests/test_golden.py checks that it still reproduces
these files, and the GPU tests compare the HIP path against them.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import eager, paging  # noqa: E402

OUT = Path(__file__).resolve().parent

FAMILIES = [(2.0, 0.5, 2), (1.5, 0.25, 3), (0.75, -0.5, 1)]


def bf16_exact(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).float()


def f64(t):
    return t.detach().double().numpy()


def norm_fixtures():
    out = {}
    x = bf16_exact((2, 2, 24, 24), 101)
    dy = bf16_exact((2, 2, 24, 24), 102)
    xr = bf16_exact((9, 40), 103, scale=2.0)
    dyr = bf16_exact((9, 40), 104)
    out.update(x_causal=x.numpy(), dy_causal=dy.numpy(), x_rowwise=xr.numpy(), dy_rowwise=dyr.numpy(),
               families=np.array(FAMILIES, dtype=np.float64))
    for i, (a, t, p) in enumerate(FAMILIES):
        out[f"y_causal_{i}"] = f64(eager.softplus_norm_causal_eager(x.double(), a, t, p))
        out[f"dx_causal_{i}"] = f64(eager.softplus_norm_backward(x.double(), dy.double(), a, t, p, causal=True))
        out[f"y_rowwise_{i}"] = f64(eager.softplus_norm_eager(xr.double(), a, t, p))
        out[f"dx_rowwise_{i}"] = f64(eager.softplus_norm_backward(xr.double(), dyr.double(), a, t, p, causal=False))
    return out


def attention_fixtures():
    q = bf16_exact((1, 4, 37, 32), 201)
    k = bf16_exact((1, 2, 37, 32), 202)
    v = bf16_exact((1, 2, 37, 32), 203)
    do = bf16_exact((1, 4, 37, 32), 204)
    out = dict(q=q.numpy(), k=k.numpy(), v=v.numpy(), do=do.numpy(), windows=np.array([0, 5], dtype=np.int64))
    for w in (0, 5):
        o, rs = eager.flash_attention_eager(q.double(), k.double(), v.double(), window_size=w, return_row_sums=True)
        dq, dk, dv = eager.flash_attention_bwd(q.double(), k.double(), v.double(), o, do.double(), window_size=w)
        out.update({f"o_w{w}": f64(o), f"rs_w{w}": f64(rs), f"dq_w{w}": f64(dq), f"dk_w{w}": f64(dk),
                    f"dv_w{w}": f64(dv)})
    return out


def fp8_fixtures():
    g = torch.Generator().manual_seed(301)
    x = (torch.randn(1000, generator=g) * torch.exp(torch.randn(1000, generator=g) * 2)).to(torch.bfloat16).float()
    x8, s = eager.quantize_to_fp8(x)
    q = bf16_exact((1, 4, 40, 32), 302)
    k = bf16_exact((1, 2, 40, 32), 303)
    v = bf16_exact((1, 2, 40, 32), 304)
    q8, qs = eager.quantize_to_fp8(q)
    k8, ks = eager.quantize_to_fp8(k)
    attn_scale = 1.0 / math.sqrt(32)
    o = eager.fp8_flash_attention_eager(q8, k8, v, qs, ks, 1.0, attn_scale)
    return dict(x=x.numpy(), x_codes=x8.view(torch.uint8).numpy(), x_scale=np.float32(s.item()),
                q=q.numpy(), k=k.numpy(), v=v.numpy(), q_codes=q8.view(torch.uint8).numpy(),
                k_codes=k8.view(torch.uint8).numpy(), q_scale=np.float32(qs.item()), k_scale=np.float32(ks.item()),
                attn_scale=np.float64(attn_scale), o=f64(o))


def paged_fixtures():
    B, Hq, Hkv, D, P, T = 3, 4, 2, 32, 8, 30
    lens = [5, 17, 30]
    k = bf16_exact((B, Hkv, T, D), 401)
    v = bf16_exact((B, Hkv, T, D), 402)
    q = bf16_exact((B, Hq, 1, D), 403)
    kc, vc, table, ctx = paging.build_paged_cache(k, v, P, shuffle=True, generator=torch.Generator().manual_seed(404),
                                                  context_lens=lens)
    o = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, ctx)
    # append 4 tokens per sequence: the last sequence (30 + 4 > 32 slots) drops its overflow
    kn = bf16_exact((B, Hkv, 4, D), 405)
    vn = bf16_exact((B, Hkv, 4, D), 406)
    kc2, vc2 = paging.append_kv(kc, vc, kn, vn, table, ctx)
    return dict(q=q.numpy(), k_cache=kc.numpy(), v_cache=vc.numpy(), block_table=table.numpy(),
                context_lens=ctx.numpy(), page_size=np.int64(P), o=f64(o), k_new=kn.numpy(), v_new=vn.numpy(),
                k_cache_appended=kc2.numpy(), v_cache_appended=vc2.numpy())


def rope_fixtures():
    q = bf16_exact((1, 4, 37, 32), 501)
    k = bf16_exact((1, 2, 37, 32), 502)
    v = bf16_exact((1, 2, 37, 32), 503)
    cos, sin = eager.rope_cos_sin(32, 37)
    o = eager.rope_flash_attention_eager(q, k, v, cos, sin)
    return dict(q=q.numpy(), k=k.numpy(), v=v.numpy(), cos=cos.numpy(), sin=sin.numpy(), o=f64(o))


def softmax_fixtures():
    x = bf16_exact((6, 45), 601, scale=3.0)
    xc = bf16_exact((2, 1, 12, 12), 602, scale=3.0)
    return dict(x_rowwise=x.numpy(), y_rowwise=f64(eager.softmax_eager(x.double())),
                x_causal=xc.numpy(), y_causal=f64(eager.softmax_causal_eager(xc.double())))


FIXTURES = {
    "norm": norm_fixtures,
    "attention": attention_fixtures,
    "fp8": fp8_fixtures,
    "paged": paged_fixtures,
    "rope": rope_fixtures,
    "softmax": softmax_fixtures,
}


def main():
    for name, fn in FIXTURES.items():
        arrays = fn()
        np.savez_compressed(OUT / f"{name}.npz", **arrays)
        print(f"wrote {name}.npz ({sum(a.nbytes for a in map(np.asarray, arrays.values()))} bytes raw)")


if __name__ == "__main__":
    main()
