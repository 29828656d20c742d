"""Parity of the fused attention forward (HIP, MFMA) with the CPU oracle (GPU).

Tolerances: bf16/fp16 outputs max|HIP - oracle| / max|oracle| <= 1e-2 against
the float64 oracle on the same seeded inputs; fp32 row sums <= 1e-5.  The
reference's own forward tolerances (tests/test_training_api.py:81-237: atol
2e-2, rtol 5e-2 vs eager) are checked too.
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


def qkv(B, Hq, Hkv, T, D, dtype, seed, layout="bhtd"):
    g = _g(seed)
    if layout == "bthd":  # [B,T,H,D].transpose(1,2): non-contiguous, as in the reference test
        q = torch.randn(B, T, Hq, D, generator=g).to(dtype).transpose(1, 2)
        k = torch.randn(B, T, Hkv, D, generator=g).to(dtype).transpose(1, 2)
        v = torch.randn(B, T, Hkv, D, generator=g).to(dtype).transpose(1, 2)
    else:
        q = torch.randn(B, Hq, T, D, generator=g).to(dtype)
        k = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
        v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    return q, k, v


def check_forward(q, k, v, window=0, exact=False, tol=1e-2):
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D)
    o, rs = kernels._sp2norm_flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), scale, q.shape[1] // k.shape[1], window,
                                       use_fast_sqrt=not exact)
    ref, ref_rs = eager.flash_attention_eager(q.double(), k.double(), v.double(), window_size=window,
                                              return_row_sums=True)
    assert o.dtype == q.dtype and o.shape == q.shape
    assert bool(torch.isfinite(o).all())
    assert rel_err(o, ref) <= tol
    assert rel_err(rs, ref_rs) <= 1e-5
    return o, ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("T", [1, 17, 64, 100, 128, 200, 512])
def test_forward_matches_oracle(dtype, D, T):
    check_forward(*qkv(2, 3, 3, T, D, dtype, seed=T * 7 + D))


@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 4), (4, 1)])
@pytest.mark.parametrize("window", [0, 1, 32, 64, 300])
def test_forward_gqa_window(hq, hkv, window):
    check_forward(*qkv(1, hq, hkv, 256, 64, torch.bfloat16, seed=hq * 10 + hkv + window), window=window)


@pytest.mark.parametrize("scale", [0.02, 0.3, 1.7, 2.0 ** -21, -0.05])
def test_forward_scales_d128(scale):
    # D = 128 bf16 computes the weights scaled by 1/scale^2 (start value
    # -1/(2 scale) on the score accumulators) for 2^-20 <= scale <= 2^20 and
    # the plain form otherwise (the last two); outputs and row sums must match
    # the oracle either way
    q, k, v = qkv(2, 4, 2, 200, 128, torch.bfloat16, seed=int(abs(scale) * 1000) + 11)
    o, rs = kernels._sp2norm_flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), scale, 2, 0)
    ref, ref_rs = eager.flash_attention_eager(q.double(), k.double(), v.double(), scale=scale,
                                              return_row_sums=True)
    assert bool(torch.isfinite(o).all())
    assert rel_err(o, ref) <= 1e-2
    assert rel_err(rs, ref_rs) <= 1e-5


def test_forward_exact_math():
    check_forward(*qkv(2, 4, 4, 256, 32, torch.bfloat16, seed=5), exact=True)


def test_forward_noncontiguous_gqa_window():
    # tests/test_training_api.py:110-125 with a seed
    q, k, v = qkv(2, 8, 2, 128, 32, torch.bfloat16, seed=6, layout="bthd")
    assert not q.is_contiguous()
    o = smooth_attn.sp2norm_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), window_size=32)
    ref = eager.flash_attention_eager(q.double(), k.double(), v.double(), window_size=32)
    assert rel_err(o, ref) <= 1e-2
    torch.testing.assert_close(o.float().cpu(), ref.float(), atol=2e-2, rtol=5e-2)


@pytest.mark.parametrize("seq_len", [64, 128, 256, 512])
def test_public_api_matches_reference_test(seq_len):
    # tests/test_training_api.py:81-93 with a seed
    q, k, v = qkv(2, 4, 4, seq_len, 32, torch.bfloat16, seed=seq_len)
    out = smooth_attn.sp2norm_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    ref = smooth_attn.sp2norm_flash_attention_eager(q.to(DEV), k.to(DEV), v.to(DEV))
    assert not out.isnan().any()
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=5e-2)


def test_strided_output_rows_and_offsets():
    # q/k/v slices of a wider buffer (t stride 3*H*D) keep the kernel path without copies
    B, H, T, D = 1, 4, 96, 64
    buf = torch.randn(B, T, 3, H, D, generator=_g(8)).to(torch.bfloat16).to(DEV)
    q, k, v = (buf[:, :, i].transpose(1, 2) for i in range(3))
    assert q.stride(2) == 3 * H * D
    o, _ = kernels._sp2norm_flash_fwd(q, k, v, 1 / 8.0)
    ref = eager.flash_attention_eager(q.cpu().double(), k.cpu().double(), v.cpu().double())
    assert rel_err(o, ref) <= 1e-2


def test_identical_values_and_single_key_rows():
    B, H, T, D = 1, 2, 130, 128
    q, k, v = qkv(B, H, H, T, D, torch.bfloat16, seed=9)
    vc = v[:, :, :1].expand(B, H, T, D).contiguous()
    o, _ = kernels._sp2norm_flash_fwd(q.to(DEV), k.to(DEV), vc.to(DEV), 1 / math.sqrt(D))
    assert rel_err(o, vc) <= 1e-2  # identical V rows -> O = V
    o1, _ = kernels._sp2norm_flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), 1 / math.sqrt(D), window_size=1)
    assert rel_err(o1, v) <= 4e-3  # window 1 -> O_i = V_i


def test_full_size_config3_sampled():
    """config 3 at full size [4,32,4096,128] bf16: whole-output
    properties, oracle parity on two sampled heads."""
    B, H, T, D = 4, 32, 4096, 128
    gen = torch.Generator(device=DEV).manual_seed(3)
    q = torch.randn(B, H, T, D, generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, H, T, D, generator=gen, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, H, T, D, generator=gen, device=DEV).to(torch.bfloat16)
    o, rs = kernels._sp2norm_flash_fwd(q, k, v, 1 / math.sqrt(D))
    assert bool(torch.isfinite(o).all()) and bool((rs > 0).all())
    for b, h in [(0, 0), (3, 31)]:
        ref, ref_rs = eager.flash_attention_eager(q[b:b + 1, h:h + 1].cpu().double(), k[b:b + 1, h:h + 1].cpu().double(),
                                                  v[b:b + 1, h:h + 1].cpu().double(), return_row_sums=True)
        assert rel_err(o[b:b + 1, h:h + 1], ref) <= 1e-2
        assert rel_err(rs[b:b + 1, h:h + 1], ref_rs) <= 1e-5


@pytest.mark.parametrize("D", [8, 16, 48, 96])
@pytest.mark.parametrize("T", [1, 100, 300])
def test_forward_head_dims_below_128(D, T):
    # any head dim up to 128 (the reference takes powers of two through
    # next_pow2, kernels.py:1918): multiples of 8 run on the 32 / 64 / 128
    # kernels with the columns past D masked
    q, k, v = qkv(1, 4, 2, T, D, torch.bfloat16, seed=D + T)
    o, _ = check_forward(q, k, v)
    assert o.is_contiguous() and o.shape == (1, 4, T, D)
    out = smooth_attn.sp2norm_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert torch.equal(out, o)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 17, 100, 128, 300])
def test_forward_head_dim_256(dtype, T):
    # D = 256 runs its own kernels (one wave per SIMD, O accumulators in AGPRs)
    q, k, v = qkv(2, 4, 2, T, 256, dtype, seed=T + 256)
    check_forward(q, k, v)
    check_forward(q, k, v, window=45)


@pytest.mark.parametrize("D", [160, 200])
def test_forward_head_dims_above_128(D):
    # head dims 129..255 run on the D = 256 kernels with the columns past D masked
    q, k, v = qkv(1, 4, 4, 150, D, torch.bfloat16, seed=D)
    o, _ = check_forward(q, k, v, exact=True)
    assert o.is_contiguous() and o.shape == (1, 4, 150, D)


def test_forward_head_dim_256_layouts():
    q, k, v = qkv(2, 8, 2, 257, 256, torch.bfloat16, seed=7, layout="bthd")
    check_forward(q, k, v)
    out = smooth_attn.sp2norm_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    o, _ = kernels._sp2norm_flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), 1 / 16, 4)
    assert torch.equal(out, o)
