"""Pins of the CPU oracle (oracle/eager.py) — CPU only.

The reference ships no golden vectors or fixtures for this path (its tests
draw unseeded CUDA randn and compare against eager at run time), so the
oracle is pinned by what the mathematics fixes: float64 scalar loops
(oracle/brute.py), closed-form identities, invariants, central finite
differences, torch autograd, and the e4m3fn format definition.  Each pin is
chosen so that a dropped term, wrong sign/index or transposed operand in the
oracle fails it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import brute, eager, paging

DTYPE = torch.float64


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
# squareplus and the family
# ---------------------------------------------------------------------------
def test_squareplus_identities():
    a = torch.linspace(-30, 30, 601, dtype=DTYPE)
    sp = eager.squareplus(a)
    spn = eager.squareplus(-a)
    assert float(eager.squareplus(torch.zeros((), dtype=DTYPE))) == 1.0
    torch.testing.assert_close(sp * spn, torch.ones_like(a), rtol=1e-12, atol=0)
    torch.testing.assert_close(sp - spn, a, rtol=0, atol=1e-10)
    # sp is the positive root of z^2 - a z - 1 = 0
    torch.testing.assert_close(sp * sp - a * sp - 1.0, torch.zeros_like(a), rtol=0, atol=1e-9)
    assert bool((sp > 0).all())


@pytest.mark.parametrize("alpha,theta,power", [(2.0, 0.5, 2), (1.5, 0.25, 3), (0.7, -1.0, 1)])
def test_family_weights_vs_brute(alpha, theta, power):
    x = torch.randn(5, 7, generator=_g(1), dtype=DTYPE)
    got = eager.family_weights(x, alpha, theta, power).numpy()
    ref = brute.family_weights(x.numpy(), alpha, theta, power)
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=0)


def test_family_rejects_bad_power():
    with pytest.raises(ValueError):
        eager.family_weights(torch.zeros(2), 2.0, 0.5, 4)


# ---------------------------------------------------------------------------
# Normalisation forward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("alpha,theta,power", [(2.0, 0.5, 2), (1.5, 0.25, 3), (1.0, 0.0, 1)])
def test_rowwise_vs_brute(alpha, theta, power):
    x = torch.randn(4, 9, generator=_g(2), dtype=DTYPE)
    got = eager.softplus_norm_eager(x, alpha, theta, power).numpy()
    np.testing.assert_allclose(got, brute.norm_rowwise(x.numpy(), alpha, theta, power), rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("alpha,theta,power", [(2.0, 0.5, 2), (1.5, 0.25, 3), (1.0, 0.0, 1)])
def test_causal_vs_brute(alpha, theta, power):
    x = torch.randn(2, 3, 6, 6, generator=_g(3), dtype=DTYPE)
    got = eager.softplus_norm_causal_eager(x, alpha, theta, power).numpy()
    np.testing.assert_allclose(got, brute.norm_causal(x.numpy(), alpha, theta, power), rtol=1e-12, atol=1e-15)


def test_causal_invariants():
    L = 33
    x = torch.randn(2, L, L, generator=_g(4), dtype=DTYPE)
    y = eager.softplus_norm_causal_eager(x)
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((y[:, upper] == 0).all()), "strict upper triangle must be exactly zero"
    # rows sum to S / (S + 1e-12)
    torch.testing.assert_close(y.sum(-1), torch.ones(2, L, dtype=DTYPE), rtol=0, atol=1e-10)
    # row 0 is e0
    torch.testing.assert_close(y[:, 0, 0], torch.ones(2, dtype=DTYPE), rtol=0, atol=1e-10)
    # a constant matrix gives 1/(i+1) on the visible prefix
    c = eager.softplus_norm_causal_eager(torch.full((L, L), 0.3, dtype=DTYPE))
    expect = torch.tril(torch.ones(L, L, dtype=DTYPE)) / torch.arange(1, L + 1, dtype=DTYPE)[:, None]
    torch.testing.assert_close(c, expect, rtol=1e-10, atol=1e-15)
    # a constant row-wise row gives 1/L
    r = eager.softplus_norm_eager(torch.full((3, L), -0.7, dtype=DTYPE))
    torch.testing.assert_close(r, torch.full((3, L), 1.0 / L, dtype=DTYPE), rtol=1e-12, atol=0)


def test_cpu_path_casts_back():
    x = torch.randn(1, 2, 8, 8, generator=_g(5)).to(torch.bfloat16)
    y = eager.softplus_norm_causal_cpu_path(x)
    assert y.dtype == torch.bfloat16
    torch.testing.assert_close(y.float(), eager.softplus_norm_causal_eager(x.float()), atol=4e-3, rtol=1e-2)


# ---------------------------------------------------------------------------
# Normalisation backward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("alpha,theta,power", [(2.0, 0.5, 2), (1.5, 0.25, 3), (0.8, -0.3, 1)])
def test_backward_vs_autograd(causal, alpha, theta, power):
    x = torch.randn(2, 7, 7, generator=_g(6), dtype=DTYPE)
    dy = torch.randn(2, 7, 7, generator=_g(7), dtype=DTYPE)
    xr = x.clone().requires_grad_(True)
    f = eager.softplus_norm_causal_eager if causal else eager.softplus_norm_eager
    (f(xr, alpha, theta, power) * dy).sum().backward()
    got = eager.softplus_norm_backward(x, dy, alpha, theta, power, causal=causal)
    torch.testing.assert_close(got, xr.grad, rtol=1e-10, atol=1e-13)


@pytest.mark.parametrize("causal", [True, False])
def test_backward_vs_finite_differences(causal):
    x = torch.randn(1, 5, 5, generator=_g(8), dtype=DTYPE)
    dy = torch.randn(1, 5, 5, generator=_g(9), dtype=DTYPE)
    f = brute.norm_causal if causal else brute.norm_rowwise
    fd = brute.fd_grad(lambda z: f(z), x.numpy(), dy.numpy())
    got = eager.softplus_norm_backward(x, dy, causal=causal).numpy()
    np.testing.assert_allclose(got, fd, rtol=1e-5, atol=1e-8)


def test_backward_known_answers():
    L = 12
    x = torch.randn(3, L, L, generator=_g(10), dtype=DTYPE)
    # dy constant along each row: dx = dydx/S * g * (1 - sum P) ~ 0
    dy = torch.randn(3, L, 1, generator=_g(11), dtype=DTYPE).expand(3, L, L)
    dx = eager.softplus_norm_backward(x, dy, causal=True)
    assert float(dx.abs().max()) < 1e-9
    # strictly upper triangle exactly zero, even with garbage dy there
    dy2 = torch.randn(3, L, L, generator=_g(12), dtype=DTYPE)
    dy2[:, torch.triu(torch.ones(L, L, dtype=torch.bool), 1)] = float("nan")
    dx2 = eager.softplus_norm_backward(x, dy2, causal=True)
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((dx2[:, upper] == 0).all())
    assert bool(torch.isfinite(dx2).all())


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("alpha,theta,power", [(2.0, 0.5, 2), (1.5, 0.25, 3), (0.75, -0.5, 1)])
def test_backward_row_invariant(causal, alpha, theta, power):
    # dx_j = alpha p y_j (dy_j - T) / sqrt(a_j^2 + 4) with T = sum_k dy_k y_k,
    # so sum_j dx_j sqrt(a_j^2 + 4) = alpha p T (1 - sum_j y_j) = O(eps) for
    # every row (the GPU tests check this over whole full-size outputs); a
    # dropped or mis-signed T term or a wrong activation derivative breaks it
    L = 40
    x = torch.randn(5, L, L, generator=_g(13), dtype=DTYPE)
    dy = torch.randn(5, L, L, generator=_g(14), dtype=DTYPE)
    dx = eager.softplus_norm_backward(x, dy, alpha, theta, power, causal=causal)
    a = alpha * (x - theta)
    inv = (dx * torch.sqrt(a * a + 4.0)).sum(-1)
    assert float(inv.abs().max()) < 1e-9  # alpha p |T| eps / S, S as small as 1e-2 here
    # and it is not vacuous: the terms themselves are O(1)
    assert float((dx * torch.sqrt(a * a + 4.0)).abs().sum(-1).min()) > (1e-3 if not causal else 0.0)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("hq,hkv,window", [(2, 2, 0), (4, 2, 0), (4, 1, 3), (2, 2, 1)])
def test_attention_vs_brute(hq, hkv, window):
    T, D = 6, 4
    q = torch.randn(1, hq, T, D, generator=_g(20), dtype=DTYPE)
    k = torch.randn(1, hkv, T, D, generator=_g(21), dtype=DTYPE)
    v = torch.randn(1, hkv, T, D, generator=_g(22), dtype=DTYPE)
    got = eager.flash_attention_eager(q, k, v, window_size=window).numpy()
    ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), window_size=window)
    np.testing.assert_allclose(got, ref, rtol=1e-11, atol=1e-13)


def test_attention_properties():
    B, H, T, D = 1, 2, 9, 8
    q = torch.randn(B, H, T, D, generator=_g(23), dtype=DTYPE)
    k = torch.randn(B, H, T, D, generator=_g(24), dtype=DTYPE)
    v = torch.randn(B, H, T, D, generator=_g(25), dtype=DTYPE)
    o = eager.flash_attention_eager(q, k, v)
    # query 0 sees only key 0
    torch.testing.assert_close(o[:, :, 0], v[:, :, 0], rtol=1e-10, atol=1e-10)
    # identical V rows -> O = V
    vc = v[:, :, :1].expand(B, H, T, D)
    torch.testing.assert_close(eager.flash_attention_eager(q, k, vc), vc, rtol=1e-10, atol=1e-10)
    # window >= T is full causal; window = 1 gives O_i = V_i
    torch.testing.assert_close(eager.flash_attention_eager(q, k, v, window_size=T), o, rtol=0, atol=0)
    torch.testing.assert_close(eager.flash_attention_eager(q, k, v, window_size=1), v, rtol=1e-10, atol=1e-10)
    # composition: attention == causal norm of scaled scores, times V
    s = (q @ k.transpose(-1, -2)) / math.sqrt(D)
    torch.testing.assert_close(o, eager.softplus_norm_causal_eager(s) @ v, rtol=1e-12, atol=1e-12)
    # row sums returned are sum y + eps
    _, rs = eager.flash_attention_eager(q, k, v, return_row_sums=True)
    a = 2 * s - 1
    y = torch.tril((0.5 * (a + torch.sqrt(a * a + 4))) ** 2)
    torch.testing.assert_close(rs, y.sum(-1) + eager.EPS, rtol=1e-12, atol=0)


def test_attention_gqa_is_repeat_interleave():
    q = torch.randn(2, 6, 7, 4, generator=_g(26), dtype=DTYPE)
    k = torch.randn(2, 2, 7, 4, generator=_g(27), dtype=DTYPE)
    v = torch.randn(2, 2, 7, 4, generator=_g(28), dtype=DTYPE)
    got = eager.flash_attention_eager(q, k, v, window_size=3)
    ref = eager.flash_attention_eager(q, k.repeat_interleave(3, 1), v.repeat_interleave(3, 1), window_size=3)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


def test_attention_grads_vs_finite_differences():
    q = torch.randn(1, 2, 4, 3, generator=_g(29), dtype=DTYPE)
    k = torch.randn(1, 1, 4, 3, generator=_g(30), dtype=DTYPE)
    v = torch.randn(1, 1, 4, 3, generator=_g(31), dtype=DTYPE)
    do = torch.randn(1, 2, 4, 3, generator=_g(32), dtype=DTYPE)
    dq, dk, dv = eager.flash_attention_grads(q, k, v, do, window_size=3)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    fd_q = brute.fd_grad(lambda z: brute.attention(z, kn, vn, window_size=3), qn, don)
    fd_k = brute.fd_grad(lambda z: brute.attention(qn, z, vn, window_size=3), kn, don)
    fd_v = brute.fd_grad(lambda z: brute.attention(qn, kn, z, window_size=3), vn, don)
    np.testing.assert_allclose(dq.numpy(), fd_q, rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(dk.numpy(), fd_k, rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(dv.numpy(), fd_v, rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("hq,hkv,window,T", [(2, 2, 0, 1), (2, 2, 0, 37), (4, 2, 5, 37), (6, 2, 1, 20),
                                             (3, 1, 64, 50)])
def test_backward_formula_vs_autograd(hq, hkv, window, T):
    # the reference's backward formula given the exact forward output equals
    # autograd of the eager attention
    q = torch.randn(2, hq, T, 8, generator=_g(40 + T), dtype=DTYPE)
    k = torch.randn(2, hkv, T, 8, generator=_g(41 + T), dtype=DTYPE)
    v = torch.randn(2, hkv, T, 8, generator=_g(42 + T), dtype=DTYPE)
    do = torch.randn(2, hq, T, 8, generator=_g(43 + T), dtype=DTYPE)
    o = eager.flash_attention_eager(q, k, v, window_size=window)
    got = eager.flash_attention_bwd(q, k, v, o, do, window_size=window)
    ref = eager.flash_attention_grads(q, k, v, do, window_size=window)
    for g_, r_ in zip(got, ref):
        torch.testing.assert_close(g_, r_, rtol=1e-10, atol=1e-12)


def test_backward_formula_single_key_rows():
    # one visible key per row (window 1): dQ = dK = 0 and dV = dO exactly when
    # o is exact; a perturbed o moves only dQ / dK, through delta
    q, k, v, do = (torch.randn(1, 2, 9, 4, generator=_g(50 + i), dtype=DTYPE) for i in range(4))
    o = eager.flash_attention_eager(q, k, v, window_size=1)
    dq, dk, dv = eager.flash_attention_bwd(q, k, v, o, do, window_size=1)
    # (nonzero only through EPS: dP - delta = dP * EPS / (y + EPS))
    assert float(dq.abs().max()) < 1e-9 and float(dk.abs().max()) < 1e-9
    torch.testing.assert_close(dv, do, rtol=1e-9, atol=1e-9)
    dq2, _, dv2 = eager.flash_attention_bwd(q, k, v, o * (1 + 2 ** -9), do, window_size=1)
    assert float(dq2.abs().max()) > 1e-6
    torch.testing.assert_close(dv2, dv, rtol=0, atol=0)


# ---------------------------------------------------------------------------
# fp8 quantiser
# ---------------------------------------------------------------------------
def test_e4m3fn_grid_definition():
    grid = brute.e4m3fn_grid()
    assert grid[-1, 1] == 448.0
    assert grid[1, 1] == 2.0 ** -9  # smallest subnormal
    assert grid[8, 1] == 2.0 ** -6  # smallest normal
    # torch's own decoding of every finite positive code agrees with the format definition
    codes = torch.arange(0, 0x7F, dtype=torch.uint8)
    decoded = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    np.testing.assert_array_equal(decoded, grid[:, 1])


def test_quantize_bits_vs_brute():
    x = torch.randn(257, generator=_g(40)) * 3.0
    x[0] = 0.0
    x[1] = -x.abs().max()  # exactly -amax -> -448
    x8, scale = eager.quantize_to_fp8(x)
    assert scale.dtype == torch.float32 and scale.dim() == 0
    assert float(scale) == float((x.abs().amax() / 448.0).clamp(min=1e-12))
    bits = x8.view(torch.uint8).numpy()
    xs = (x / scale).clamp(-448, 448).numpy()
    want = np.array([brute.e4m3fn_round(float(v)) for v in xs], dtype=np.uint8)
    np.testing.assert_array_equal(bits, want)
    assert int(bits[1]) == 0xFE  # -448
    # dequantisation error is at most half a unit in the last place (3 mantissa bits)
    err = (x8.float() * scale - x).abs()
    assert bool((err <= x.abs() * 2.0 ** -4 + float(scale) * 2.0 ** -10).all())


def test_quantize_zero_tensor_uses_floor_scale():
    x8, scale = eager.quantize_to_fp8(torch.zeros(16))
    assert float(scale) == pytest.approx(1e-12)
    assert bool((x8.view(torch.uint8) == 0).all())


def test_fp8_attention_is_dequantised_attention():
    q = torch.randn(1, 4, 8, 8, generator=_g(41))
    k = torch.randn(1, 2, 8, 8, generator=_g(42))
    v = torch.randn(1, 2, 8, 8, generator=_g(43))
    q8, qs = eager.quantize_to_fp8(q)
    k8, ks = eager.quantize_to_fp8(k)
    v8, vs = eager.quantize_to_fp8(v)
    got = eager.fp8_flash_attention_eager(q8, k8, v8, qs, ks, vs, 1 / math.sqrt(8), window_size=5)
    ref = brute.attention((q8.double() * float(qs)).numpy(), (k8.double() * float(ks)).numpy(),
                          (v8.double() * float(vs)).numpy(), window_size=5)
    np.testing.assert_allclose(got.numpy(), ref, rtol=2e-5, atol=2e-6)


# ---------------------------------------------------------------------------
# Paged decode
# ---------------------------------------------------------------------------
def test_paged_decode_is_last_causal_row():
    B, Hq, Hkv, T, D = 2, 4, 2, 37, 8
    q = torch.randn(B, Hq, 1, D, generator=_g(50), dtype=DTYPE)
    k = torch.randn(B, Hkv, T, D, generator=_g(51), dtype=DTYPE)
    v = torch.randn(B, Hkv, T, D, generator=_g(52), dtype=DTYPE)
    kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=8, shuffle=True, generator=_g(53))
    got = eager.paged_decode_eager(q, kc, vc, table, lens)
    # decode query = last query of a causal sequence
    qs = torch.zeros(B, Hq, T, D, dtype=DTYPE)
    qs[:, :, -1] = q[:, :, 0]
    ref = eager.flash_attention_eager(qs, k, v)[:, :, -1]
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


def test_paged_decode_layout_independence():
    B, Hq, Hkv, T, D = 3, 4, 4, 29, 8
    q = torch.randn(B, Hq, 1, D, generator=_g(54), dtype=DTYPE)
    k = torch.randn(B, Hkv, T, D, generator=_g(55), dtype=DTYPE)
    v = torch.randn(B, Hkv, T, D, generator=_g(56), dtype=DTYPE)
    outs = []
    for ps, sh in [(8, False), (8, True), (16, True), (32, False)]:
        kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=ps, shuffle=sh, generator=_g(57))
        outs.append(eager.paged_decode_eager(q, kc, vc, table, lens))
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], rtol=1e-12, atol=1e-12)
    # ctx = 1 gives V0; variable lengths equal per-sequence truncation
    kc, vc, table, _ = paging.build_paged_cache(k, v, page_size=8, context_lens=[1, 17, 29])
    o = eager.paged_decode_eager(q, kc, vc, table, torch.tensor([1, 17, 29], dtype=torch.int32))
    torch.testing.assert_close(o[0], v[0, :, 0].repeat_interleave(Hq // Hkv, 0), rtol=1e-10, atol=1e-10)
    kc2, vc2, table2, lens2 = paging.build_paged_cache(k[1:2, :, :17], v[1:2, :, :17], page_size=8)
    torch.testing.assert_close(o[1], eager.paged_decode_eager(q[1:2], kc2, vc2, table2, lens2)[0],
                               rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def test_rope_tables_closed_form():
    cos, sin = eager.rope_cos_sin(16, 40)
    t = np.arange(40)[:, None]
    ang = t * 10000.0 ** (-np.arange(0, 16, 2)[None, :] / 16.0)
    np.testing.assert_allclose(cos.numpy(), np.cos(ang), rtol=0, atol=2e-6)
    np.testing.assert_allclose(sin.numpy(), np.sin(ang), rtol=0, atol=2e-6)


def test_rope_vs_complex_rotation():
    x = torch.randn(2, 3, 9, 8, generator=_g(60), dtype=DTYPE)
    cos, sin = eager.rope_cos_sin(8, 9, dtype=DTYPE)
    got = eager.apply_rope(x, cos, sin).numpy()
    # the fp32 tables carry ~1e-7 relative error at these angles
    np.testing.assert_allclose(got, brute.rope(x.numpy()), rtol=0, atol=2e-6)


def test_rope_invariants():
    D, T = 16, 12
    cos, sin = eager.rope_cos_sin(D, T, dtype=DTYPE)
    x = torch.randn(1, 1, T, D, generator=_g(61), dtype=DTYPE)
    r = eager.apply_rope(x, cos, sin)
    torch.testing.assert_close(r[..., 0, :], x[..., 0, :], rtol=0, atol=0)  # position 0: identity
    pair = lambda z: z[..., : D // 2] ** 2 + z[..., D // 2:] ** 2
    # rotations keep pair norms (cos^2 + sin^2 = 1 to the fp32 tables' precision)
    torch.testing.assert_close(pair(r), pair(x), rtol=1e-6, atol=1e-9)
    # <R_m q, R_n k> depends only on m - n: put the same q / k at every position
    q = torch.randn(D, generator=_g(62), dtype=DTYPE).expand(1, 1, T, D)
    k = torch.randn(D, generator=_g(63), dtype=DTYPE).expand(1, 1, T, D)
    rq, rk = eager.apply_rope(q, cos, sin)[0, 0], eager.apply_rope(k, cos, sin)[0, 0]
    dots = rq @ rk.T
    for off in range(-3, 4):
        d = torch.diagonal(dots, offset=off)
        torch.testing.assert_close(d, d[:1].expand_as(d), rtol=1e-5, atol=1e-5)


def test_rope_proj_is_one_gemm():
    B, H, T, D, M = 2, 3, 10, 8, 5
    q, k, v = (torch.randn(B, H, T, D, generator=_g(64 + i), dtype=DTYPE) for i in range(3))
    w = torch.randn(H, D, M, generator=_g(67), dtype=DTYPE)
    cos, sin = eager.rope_cos_sin(D, T, dtype=DTYPE)
    got = eager.rope_proj_eager(q, k, v, w, cos, sin, round_to=None)
    o = eager.rope_flash_attention_eager(q, k, v, cos, sin, round_to=None)
    ref = o.transpose(1, 2).reshape(B, T, H * D) @ w.reshape(H * D, M)
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# Softmax baselines
# ---------------------------------------------------------------------------
def test_softmax_vs_brute_and_invariants():
    x = torch.randn(5, 13, generator=_g(70), dtype=DTYPE) * 4
    y = eager.softmax_eager(x)
    np.testing.assert_allclose(y.numpy(), brute.softmax(x.numpy()), rtol=1e-13, atol=0)
    torch.testing.assert_close(y.sum(-1), torch.ones(5, dtype=DTYPE), rtol=0, atol=1e-14)
    torch.testing.assert_close(eager.softmax_eager(x + 123.0), y, rtol=1e-12, atol=1e-15)


def test_softmax_causal_vs_brute_prefixes():
    L = 9
    x = torch.randn(2, L, L, generator=_g(71), dtype=DTYPE) * 3
    y = eager.softmax_causal_eager(x)
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((y[:, upper] == 0).all())
    torch.testing.assert_close(y[:, 0, 0], torch.ones(2, dtype=DTYPE), rtol=0, atol=0)
    for i in range(L):
        np.testing.assert_allclose(y[:, i, : i + 1].numpy(), brute.softmax(x[:, i, : i + 1].numpy()),
                                   rtol=1e-13, atol=0)


def test_append_kv_rebuilds_cache_and_composes():
    B, H, T, D, P = 2, 3, 37, 8, 8
    k = torch.randn(B, H, T, D, generator=_g(80), dtype=DTYPE)
    v = torch.randn(B, H, T, D, generator=_g(81), dtype=DTYPE)
    kc, vc, table, lens = paging.build_paged_cache(k, v, P, shuffle=True, generator=_g(82))
    empty_k, empty_v = torch.zeros_like(kc), torch.zeros_like(vc)
    zero = torch.zeros(B, dtype=torch.int32)
    k1, v1 = paging.append_kv(empty_k, empty_v, k, v, table, zero)
    torch.testing.assert_close(k1, kc, rtol=0, atol=0)
    torch.testing.assert_close(v1, vc, rtol=0, atol=0)
    # two appends (20 rows, then 17) equal one
    k2, v2 = paging.append_kv(empty_k, empty_v, k[:, :, :20], v[:, :, :20], table, zero)
    k2, v2 = paging.append_kv(k2, v2, k[:, :, 20:], v[:, :, 20:], table, zero + 20)
    torch.testing.assert_close(k2, kc, rtol=0, atol=0)
    torch.testing.assert_close(v2, vc, rtol=0, atol=0)
    # rows past the table (page index >= max_pages) are dropped, nothing else changes
    full = torch.full((B,), table.shape[1] * P, dtype=torch.int32)
    k3, _ = paging.append_kv(kc, vc, k[:, :, :4], v[:, :, :4], table, full)
    torch.testing.assert_close(k3, kc, rtol=0, atol=0)
    # table entries outside the cache are dropped too
    bad = table.clone()
    bad[:, 0] = -1
    k4, _ = paging.append_kv(empty_k, empty_v, k[:, :, :P], v[:, :, :P], bad, zero)
    assert float(k4.abs().max()) == 0.0
