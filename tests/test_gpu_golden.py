"""HIP path vs the committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the float64 oracle).  Tolerances as in the
other GPU tests: max|HIP - golden| / max|golden| <= 1e-2 for 16-bit outputs
attention gradients included, <= 1e-5 for fp32 outputs and row sums;
fp8 codes and the paged-KV append bit-exact."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import smooth_attn
from smooth_attn import FamilyConfig, kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz") as f:
        return {k: f[k] for k in f.files}


def t(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = torch.as_tensor(ref).double()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 1e-2), (torch.float32, 1e-5)])
@pytest.mark.parametrize("fam", [0, 1, 2])
def test_norm_golden(dtype, tol, fam):
    g = load("norm")
    a, th, p = g["families"][fam]
    family = FamilyConfig(alpha=float(a), theta=float(th), power=int(p))
    x, dy = t(g["x_causal"], dtype), t(g["dy_causal"], dtype)
    y = smooth_attn.softplus_norm_causal_triton(x, family=family)
    assert rel_err(y, g[f"y_causal_{fam}"]) <= tol
    assert bool((y.cpu()[..., torch.triu(torch.ones(24, 24, dtype=torch.bool), 1)] == 0).all())
    dx = kernels._softplus_norm_causal_backward(x, dy, family)
    assert rel_err(dx, g[f"dx_causal_{fam}"]) <= tol
    xr, dyr = t(g["x_rowwise"], dtype), t(g["dy_rowwise"], dtype)
    yr = smooth_attn.softplus_norm_triton(xr, family=family)
    assert rel_err(yr, g[f"y_rowwise_{fam}"]) <= tol
    dxr = kernels._softplus_norm_backward(xr, dyr, family)
    assert rel_err(dxr, g[f"dx_rowwise_{fam}"]) <= tol


@pytest.mark.parametrize("window", [0, 5])
def test_attention_golden(window):
    g = load("attention")
    q, k, v, do = (t(g[n]) for n in ("q", "k", "v", "do"))
    sc = 1.0 / math.sqrt(32)
    o, rs = kernels._sp2norm_flash_fwd(q, k, v, sc, 2, window)
    assert rel_err(o, g[f"o_w{window}"]) <= 1e-2
    assert rel_err(rs, g[f"rs_w{window}"]) <= 1e-5
    dq, dk, dv = kernels._sp2norm_flash_bwd(q, k, v, o, do, rs, sc, 2, window)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert rel_err(got, g[f"{name}_w{window}"]) <= 1e-2, name


def test_fp8_golden():
    g = load("fp8")
    x8, s = kernels._quantize_to_fp8_device(t(g["x"]))
    assert np.array_equal(x8.view(torch.uint8).cpu().numpy(), g["x_codes"])
    assert float(s) == float(g["x_scale"])
    q8, qs = kernels._quantize_to_fp8_device(t(g["q"]))
    k8, ks = kernels._quantize_to_fp8_device(t(g["k"]))
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), g["q_codes"])
    assert np.array_equal(k8.view(torch.uint8).cpu().numpy(), g["k_codes"])
    assert float(qs) == float(g["q_scale"]) and float(ks) == float(g["k_scale"])
    o, _ = kernels._sp2norm_fp8_flash_fwd(q8, k8, t(g["v"]), qs, ks, None, float(g["attn_scale"]), 2)
    assert rel_err(o, g["o"]) <= 1e-2


def test_paged_golden():
    g = load("paged")
    P = int(g["page_size"])
    kc, vc = t(g["k_cache"]), t(g["v_cache"])
    table = torch.from_numpy(g["block_table"]).to(DEV)
    ctx = torch.from_numpy(g["context_lens"]).to(DEV)
    o = smooth_attn.sp2norm_paged_attention(t(g["q"]), kc, vc, table, ctx, block_size=P)
    assert rel_err(o.reshape(g["o"].shape), g["o"]) <= 1e-2
    new_ctx = smooth_attn.sp2norm_paged_kv_append(kc, vc, t(g["k_new"]), t(g["v_new"]), table, ctx, block_size=P)
    assert new_ctx.cpu().tolist() == [int(c) + 4 for c in g["context_lens"]]
    # bit-exact, including the rows the last sequence drops past its table
    assert torch.equal(kc.float().cpu(), torch.from_numpy(g["k_cache_appended"]))
    assert torch.equal(vc.float().cpu(), torch.from_numpy(g["v_cache_appended"]))


def test_rope_golden():
    g = load("rope")
    cos = torch.from_numpy(g["cos"]).to(DEV)
    sin = torch.from_numpy(g["sin"]).to(DEV)
    o = smooth_attn.sp2norm_rope_flash_attention(t(g["q"]), t(g["k"]), t(g["v"]), cos, sin)
    assert rel_err(o, g["o"]) <= 1e-2


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 1e-2), (torch.float32, 1e-5)])
def test_softmax_golden(dtype, tol):
    g = load("softmax")
    y = smooth_attn.softmax_triton(t(g["x_rowwise"], dtype))
    assert rel_err(y, g["y_rowwise"]) <= tol
    yc = smooth_attn.softmax_causal_triton(t(g["x_causal"], dtype))
    assert rel_err(yc, g["y_causal"]) <= tol
