"""Parity of the RoPE-fused attention forwards (HIP) with the CPU oracle (GPU).

Oracle: the reference test's own construction (tests/test_rope_proj.py:46-146)
restated in oracle.eager — rotate q, k in fp32, round to the input type,
eager attention (and the per-head projection sum) in float64.  Tolerances:
max|HIP - oracle| / max|oracle| <= 1e-2 for the attention output and the
projected output (O is rounded to 16 bits before the projection, as in the
reference); fp32 row sums <= 1e-5; plus the reference tests' absolute
bounds (max error < 0.05 attention, < 0.1 projection).
"""
import math

import pytest
import torch

import smooth_attn
from oracle import eager
from smooth_attn import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


def inputs(B, Hq, Hkv, T, D, dtype, seed, layout="bhtd"):
    g = _g(seed)
    if layout == "bthd":
        q, k, v = (torch.randn(B, T, H, D, generator=g).to(dtype).transpose(1, 2) for H in (Hq, Hkv, Hkv))
    else:
        q, k, v = (torch.randn(B, H, T, D, generator=g).to(dtype) for H in (Hq, Hkv, Hkv))
    return q, k, v


def check_rope(q, k, v, window=0, tol=1e-2):
    T, D = q.shape[2], q.shape[3]
    cos, sin = smooth_attn.precompute_rope_cos_sin(D, T, device=DEV)
    out = smooth_attn.sp2norm_rope_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), cos, sin, window_size=window)
    ref = eager.rope_flash_attention_eager(q.double(), k.double(), v.double(), cos.cpu(), sin.cpu(),
                                           window_size=window, round_to=q.dtype)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert not out.isnan().any()
    assert rel_err(out, ref) <= tol
    assert float((out.float().cpu() - ref.float()).abs().max()) < 0.05  # tests/test_rope_proj.py:69
    return out


@pytest.mark.parametrize("B,H,T,D", [(1, 4, 64, 32), (2, 4, 128, 32), (2, 8, 256, 64), (1, 2, 200, 128),
                                     (1, 2, 1, 64), (1, 2, 100, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_forward_matches_oracle(B, H, T, D, dtype):
    # tests/test_rope_proj.py:46-70 shapes, plus D=128, ragged T and T=1
    check_rope(*inputs(B, H, H, T, D, dtype, seed=T + D + B))


def test_rope_forward_gqa():
    # tests/test_rope_proj.py:73-95
    check_rope(*inputs(2, 8, 2, 128, 32, torch.bfloat16, seed=21))


@pytest.mark.parametrize("window", [1, 64])
def test_rope_forward_window(window):
    # tests/test_rope_proj.py:98-114
    check_rope(*inputs(2, 4, 4, 128, 32, torch.bfloat16, seed=22 + window), window=window)


def test_rope_forward_noncontiguous_and_row_sums():
    q, k, v = inputs(1, 4, 2, 96, 64, torch.bfloat16, seed=23, layout="bthd")
    assert not q.is_contiguous()
    D, T = 64, 96
    cos, sin = smooth_attn.precompute_rope_cos_sin(D, T, device=DEV)
    o, rs = kernels._sp2norm_rope_flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cos, sin, 1 / math.sqrt(D), 2)
    qr = eager.apply_rope(q.double(), cos.cpu().double(), sin.cpu().double()).to(torch.bfloat16).double()
    kr = eager.apply_rope(k.double(), cos.cpu().double(), sin.cpu().double()).to(torch.bfloat16).double()
    ref, ref_rs = eager.flash_attention_eager(qr, kr, v.double(), return_row_sums=True)
    assert rel_err(o, ref) <= 1e-2
    assert rel_err(rs, ref_rs) <= 1e-5


def test_rope_identity_tables_equal_plain_forward():
    # cos = 1, sin = 0 rotates nothing: the RoPE path must give the plain forward's output
    q, k, v = (t.to(DEV) for t in inputs(1, 4, 4, 160, 128, torch.bfloat16, seed=24))
    cos = torch.ones(160, 64, device=DEV)
    sin = torch.zeros(160, 64, device=DEV)
    o_rope, rs_rope = kernels._sp2norm_rope_flash_fwd(q, k, v, cos, sin, 1 / math.sqrt(128))
    o, rs = kernels._sp2norm_flash_fwd(q, k, v, 1 / math.sqrt(128))
    assert rel_err(o_rope, o) <= 4e-3
    assert rel_err(rs_rope, rs) <= 1e-6


@pytest.mark.parametrize("B,H,Hkv,T,D,M,window", [(2, 4, 4, 64, 32, 128, 0), (1, 8, 2, 130, 64, 96, 32),
                                                  (1, 4, 4, 256, 128, 512, 0)])
def test_rope_proj_matches_oracle(B, H, Hkv, T, D, M, window):
    # tests/test_rope_proj.py:117-146 (first case), GQA / window / D=128 cases
    q, k, v = inputs(B, H, Hkv, T, D, torch.bfloat16, seed=25 + M)
    w_o = (torch.randn(H, D, M, generator=_g(26)) * 0.02).to(torch.bfloat16)
    cos, sin = smooth_attn.precompute_rope_cos_sin(D, T, device=DEV)
    out = smooth_attn.sp2norm_rope_flash_attention_proj(q.to(DEV), k.to(DEV), v.to(DEV), w_o.to(DEV), cos, sin,
                                                        window_size=window)
    ref = eager.rope_proj_eager(q.double(), k.double(), v.double(), w_o.double(), cos.cpu(), sin.cpu(),
                                window_size=window)
    assert out.shape == (B, T, M) and out.dtype == torch.bfloat16
    assert not out.isnan().any()
    assert rel_err(out, ref) <= 1e-2
    assert float((out.float().cpu() - ref.float()).abs().max()) < 0.1  # tests/test_rope_proj.py:143
    # deterministic: the projection is one fp32-accumulating GEMM, no atomics
    out2 = smooth_attn.sp2norm_rope_flash_attention_proj(q.to(DEV), k.to(DEV), v.to(DEV), w_o.to(DEV), cos, sin,
                                                         window_size=window)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (64, 128), (72, 200), (8, 8), (1000, 16), (136, 4104)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_transpose16_bit_exact(rows, cols, dtype):
    # the projection's weight transpose: full 64x64 tiles and ragged edges
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype).to(DEV)
    y = kernels._transpose16(x)
    assert y.shape == (cols, rows) and y.is_contiguous()
    assert torch.equal(y.cpu(), x.cpu().t())
    # a strided source (a column slice of a wider matrix)
    wide = torch.randn(rows, cols + 16, generator=g).to(dtype).to(DEV)
    ys = kernels._transpose16(wide[:, 8:8 + cols])
    assert torch.equal(ys.cpu(), wide[:, 8:8 + cols].cpu().t())


@pytest.mark.parametrize("D", [16, 48, 80, 96, 160, 256, 384, 512])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_other_head_dims(D, dtype):
    # head dims other than 32 / 64 / 128: Q and K rotated by sa_rope_rotate,
    # then the plain fused forward (next kernel up, columns past D masked)
    check_rope(*inputs(2, 4, 2, 150, D, dtype, seed=D), window=0)
    check_rope(*inputs(1, 4, 4, 200, D, dtype, seed=D + 1, layout="bthd"), window=50)


def test_rope_rotate_matches_oracle():
    # sa_rope_rotate against the oracle's rotation, both in fp32 and rounded
    # to bf16 once: the kernel may fuse a product into an FMA, so a value can
    # round to the neighbouring bf16 number, never further
    for D in (16, 64, 256):
        x = torch.randn(2, 3, 70, D, generator=_g(D)).to(torch.bfloat16)
        cos, sin = smooth_attn.precompute_rope_cos_sin(D, 70, device=DEV)
        got = kernels._rope_rotate(x.to(DEV), cos, sin).cpu().float()
        want = eager.apply_rope(x.float(), cos.cpu(), sin.cpu())
        ulp = torch.ldexp(torch.ones_like(want), torch.frexp(want.abs().clamp(min=1e-30))[1] - 8)
        assert bool(((got - want).abs() <= ulp).all()), D
        assert float((got == want.to(torch.bfloat16).float()).float().mean()) > 0.99, D


def test_rope_proj_head_dim_256():
    B, H, Hkv, T, D, M = 1, 4, 2, 96, 256, 384
    q, k, v = inputs(B, H, Hkv, T, D, torch.bfloat16, seed=77)
    w_o = (torch.randn(H, D, M, generator=_g(78)) * 0.02).to(torch.bfloat16)
    cos, sin = smooth_attn.precompute_rope_cos_sin(D, T, device=DEV)
    out = smooth_attn.sp2norm_rope_flash_attention_proj(q.to(DEV), k.to(DEV), v.to(DEV), w_o.to(DEV), cos, sin)
    ref = eager.rope_proj_eager(q.double(), k.double(), v.double(), w_o.double(), cos.cpu(), sin.cpu())
    assert out.shape == (B, T, M)
    assert rel_err(out, ref) <= 1e-2


@pytest.mark.parametrize("D", [32, 128, 256, 384])
def test_rope_fp32(D):
    # fp32 q/k/v: rotation in fp32 (sa_rope_rotate), then the fp32-MFMA
    # attention; fp32 output held to 1e-5 against the float64 oracle
    q, k, v = inputs(1, 4, 2, 130, D, torch.float32, seed=D + 5)
    T = q.shape[2]
    cos, sin = smooth_attn.precompute_rope_cos_sin(D, T, device=DEV)
    out = smooth_attn.sp2norm_rope_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), cos, sin, window_size=60)
    ref = eager.rope_flash_attention_eager(q.double(), k.double(), v.double(), cos.cpu(), sin.cpu(),
                                           window_size=60, round_to=None)
    assert out.dtype == torch.float32 and out.shape == q.shape
    assert rel_err(out, ref) <= 1e-5
    w_o = torch.randn(4, D, 96, generator=_g(D)) * 0.05
    proj = smooth_attn.sp2norm_rope_flash_attention_proj(q.to(DEV), k.to(DEV), v.to(DEV), w_o.to(DEV), cos, sin)
    ref_p = eager.rope_proj_eager(q.double(), k.double(), v.double(), w_o.double(), cos.cpu(), sin.cpu(),
                                  round_to=None)
    assert proj.dtype == torch.float32 and rel_err(proj, ref_p) <= 1e-5
