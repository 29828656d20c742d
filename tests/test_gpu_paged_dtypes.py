"""Paged decode over fp32, e4m3fn and mixed-dtype q / caches (GPU).

The reference upcasts q, K and V to fp32 whatever their storage type and
computes scores, weights and the weighted sum in fp32 (kernels.py:2716-2717,
:2746, :2765), writing a bf16 output.  Here q may be fp32, bf16 or fp16 and
the caches fp32, bf16, fp16 or e4m3fn (K and V of one dtype, e4m3fn values
read unscaled as the reference reads them); a q whose dtype differs from the
caches', or an e4m3fn q, runs as fp32.  Pairs other than bf16 / bf16 and
fp16 / fp16 run every product as bf16 hi + lo splits (16 significant bits;
e4m3fn values widen to bf16 exactly) with fp32 weights split the same way.

Bars, against the float64 oracle (oracle.eager.paged_decode_eager) on the
same stored values:
- every pair: max|out - ref| / max|ref| <= 1e-2 (the bf16 output bar);
- the split pairs: the output equals bf16(ref) up to one bf16 step, and at
  least 97% of elements equal it exactly.  Rounding the products to plain
  bf16 (dropping the lo parts) leaves about 1e-3 relative error before the
  final rounding and fails the exact-match share (checked here by running
  the same comparison on the plain bf16 pair).
"""
import ctypes

import pytest
import torch

import smooth_attn
from oracle import eager, paging
from smooth_attn import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn]


def _g(seed):
    return torch.Generator().manual_seed(seed)


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


def bf16_match(out, ref):
    """(share of elements equal to bf16(ref), largest difference in bf16
    steps).  The step of an element is that of its own binade plus 2^-14 of
    max|ref|: outputs near zero come from sums of terms of the size of V, so
    their absolute error is set by that scale, not by their own."""
    out = out.detach().cpu().double()
    ref = ref.detach().cpu().double()
    rb = ref.float().to(torch.bfloat16).double()
    diff = (out - rb).abs()
    _, e = torch.frexp(rb)  # |rb| in [2^(e-1), 2^e): one bf16 step (8 significant bits) is 2^(e-8)
    step = torch.ldexp(torch.ones_like(rb), e - 8)
    # references within 1% of a step of a rounding midpoint may round either
    # way (fp16 values hold 11 bits: an eighth of them are exact midpoints)
    decided = (ref - rb).abs() < 0.49 * step
    share = float((diff == 0)[decided].double().mean())
    return share, float((diff / (step + 2.0 ** -14 * float(rb.abs().max()))).max())


def decode(q, kc, vc, table, lens, P):
    return smooth_attn.sp2norm_paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), lens.to(DEV),
                                               block_size=P)


def make(B, Hq, Hkv, T, D, P, qdt, cdt, seed):
    g = _g(seed)
    q = torch.randn(B, Hq, 1, D, generator=g).to(qdt)
    k = torch.randn(B, Hkv, T, D, generator=g).to(cdt)
    v = torch.randn(B, Hkv, T, D, generator=g).to(cdt)
    kc, vc, table, _ = paging.build_paged_cache(k, v, page_size=P, shuffle=True, generator=_g(seed + 1))
    lens = torch.tensor([T, 1, (T + 1) // 2][:B], dtype=torch.int32)
    return q, kc, vc, table, lens


@pytest.mark.parametrize("qdt", DTYPES)
@pytest.mark.parametrize("cdt", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 256, 40, 512, 1024])
def test_paged_dtype_pairs(qdt, cdt, D):
    q, kc, vc, table, lens = make(3, 8, 2, 333, D, 16, qdt, cdt, seed=D + 7)
    if cdt == torch.float8_e4m3fn and D % 16:
        with pytest.raises(ValueError, match="multiple of 16"):  # 16-byte rows of 1-byte elements
            decode(q, kc, vc, table, lens, 16)
        return
    if D > 512 and (cdt == torch.float32 or (cdt == torch.float16 and qdt != torch.float16)):
        with pytest.raises(ValueError, match="up to 512"):  # caches read as bf16 hi + lo tiles
            decode(q, kc, vc, table, lens, 16)
        return
    out = decode(q, kc, vc, table, lens, 16)
    assert out.dtype == torch.bfloat16 and out.shape == (3, 8, D)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2
    if not (qdt == cdt and qdt in (torch.bfloat16, torch.float16)):
        share, steps = bf16_match(out, ref)
        assert steps <= 1.0 + 1e-6, (qdt, cdt, D, steps)
        assert share >= 0.97, (qdt, cdt, D, share)


def test_plain_bf16_rounding_fails_the_exact_match_bar():
    # the discriminating power of bf16_match: the 16-bit pair (products and
    # weights rounded to bf16) falls well short of 97% exact matches
    q, kc, vc, table, lens = make(3, 8, 2, 333, 128, 16, torch.bfloat16, torch.bfloat16, seed=11)
    out = decode(q, kc, vc, table, lens, 16)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    share, _ = bf16_match(out, ref)
    assert share < 0.9  # about 0.67 for these rows (an fp64 emulation of both paths gives 0.57-0.86 per row)


@pytest.mark.parametrize("P", [1, 4, 64])
def test_paged_fp32_page_sizes(P):
    # pages smaller than a load instruction's tokens take per-lane page ids
    q, kc, vc, table, lens = make(3, 4, 4, 200, 128, P, torch.float32, torch.float32, seed=P)
    out = decode(q, kc, vc, table, lens, P)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    share, steps = bf16_match(out, ref)
    assert steps <= 1.0 + 1e-6 and share >= 0.97


def test_paged_fp32_config5_layout():
    """config 5's layout (Hq 32 / Hkv 8, D 128, page 16, seeded permutation
    of all pages, ctx ~ U[512, 16384]) with fp32 caches and q, 16 sequences;
    three sampled against the oracle, all finite."""
    g = _g(55)
    B, Hq, Hkv, D, P = 16, 32, 8, 128, 16
    lens = torch.randint(512, 16385, (B,), generator=g)
    table, n_pages = paging.random_paged_layout(lens.tolist(), P, generator=g)
    kc = torch.randn(n_pages, Hkv, P, D, generator=g)
    vc = torch.randn(n_pages, Hkv, P, D, generator=g)
    q = torch.randn(B, Hq, 1, D, generator=g)
    out = decode(q, kc, vc, table, lens.to(torch.int32), P)
    assert bool(torch.isfinite(out).all())
    sel = [0, 7, 15]
    ref = eager.paged_decode_eager(q[sel].double(), kc.double(), vc.double(), table[sel], lens[sel])
    assert rel_err(out[sel], ref) <= 1e-2
    share, steps = bf16_match(out[sel], ref)
    assert steps <= 1.0 + 1e-6 and share >= 0.97


def test_paged_fp32_q_over_bf16_cache_through_the_c_abi():
    # SA_PAGED_DTYPES(SA_F32, SA_BF16) through the C ABI equals the Python
    # entry point (which converts a bf16 q to fp32 for fp32 caches itself)
    B, Hq, Hkv, D, P = 2, 8, 2, 64, 16
    q, kc, vc, table, lens = make(B, Hq, Hkv, 100, D, P, torch.float32, torch.bfloat16, seed=3)
    qd, kd, vd, td, ld = (t.to(DEV) for t in (q, kc, vc, table, lens))
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    lib = _lib.load()
    ws_bytes = lib.sa_paged_decode_workspace_size(B, Hq, D, table.shape[1], P)
    ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=DEV)
    st = lib.sa_paged_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), td.data_ptr(),
                             ld.data_ptr(), B, Hq, Hkv, D, P, table.shape[1], kc.shape[0], _lib.strides(qd),
                             _lib.strides(kd), _lib.strides(vd), _lib.strides(out), td.stride(0), D ** -0.5,
                             _lib.paged_dtypes(_lib.SA_F32, _lib.SA_BF16), ctypes.c_void_p(ws.data_ptr()),
                             ws.numel() * 4, torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "sa_paged_decode")
    ref = decode(q, kc, vc, table, lens, P)
    assert torch.equal(out, ref)


def test_paged_mismatched_cache_dtypes_are_refused():
    q, kc, vc, table, lens = make(1, 4, 2, 40, 32, 16, torch.float32, torch.float32, seed=9)
    with pytest.raises(ValueError, match="one dtype"):
        decode(q, kc, vc.to(torch.bfloat16), table, lens, 16)


def test_paged_fp8_cache_c_abi_and_append():
    # e4m3fn caches filled by the paged-KV writer (a byte copy) and decoded
    # through SA_PAGED_DTYPES(SA_F32, SA_FP8_E4M3FN): equal to the Python
    # entry point over the same caches, and to the oracle's bf16 rounding
    B, Hq, Hkv, D, P, T = 2, 8, 2, 64, 16, 90
    g = _g(41)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.float8_e4m3fn)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.float8_e4m3fn)
    q = torch.randn(B, Hq, 1, D, generator=g)
    full_k, full_v, table, lens = paging.build_paged_cache(k, v, P, shuffle=True, generator=_g(42))
    kd = torch.zeros_like(full_k).to(DEV)
    vd = torch.zeros_like(full_v).to(DEV)
    ctx = torch.zeros(B, dtype=torch.int32, device=DEV)
    ctx = smooth_attn.sp2norm_paged_kv_append(kd, vd, k.to(DEV), v.to(DEV), table.to(DEV), ctx, block_size=P)
    assert torch.equal(kd.cpu().view(torch.uint8), full_k.view(torch.uint8))
    assert torch.equal(vd.cpu().view(torch.uint8), full_v.view(torch.uint8))
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    lib = _lib.load()
    qd, td = q.to(DEV), table.to(DEV)
    ws = torch.empty(lib.sa_paged_decode_workspace_size(B, Hq, D, table.shape[1], P) // 4 + 1, device=DEV)
    st = lib.sa_paged_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), td.data_ptr(),
                             ctx.data_ptr(), B, Hq, Hkv, D, P, table.shape[1], full_k.shape[0], _lib.strides(qd),
                             _lib.strides(kd), _lib.strides(vd), _lib.strides(out), td.stride(0), D ** -0.5,
                             _lib.paged_dtypes(_lib.SA_F32, _lib.SA_FP8_E4M3FN), ctypes.c_void_p(ws.data_ptr()),
                             ws.numel() * 4, torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "sa_paged_decode")
    assert torch.equal(out, smooth_attn.sp2norm_paged_attention(qd, kd, vd, td, ctx, block_size=P))
    ref = eager.paged_decode_eager(q.double(), full_k.double(), full_v.double(), table, lens)
    share, steps = bf16_match(out, ref)
    assert steps <= 1.0 + 1e-6 and share >= 0.97


@pytest.mark.parametrize("qdt", [torch.float32, torch.bfloat16])
def test_e4m3fn_codes_widen_exactly(qdt):
    # every finite e4m3fn code (subnormals and both zeros included) as a V
    # element of a one-token context: the output is V itself (weight / row
    # sum = 1 up to the 2^-16 of the hi + lo split, far below the distance
    # of a 4-bit value from a bf16 rounding midpoint), so it must equal the
    # code widened to bf16 (values compared: the accumulation turns -0 into
    # +0); K is zero, so every score is 0
    B, Hq, Hkv, D, P = 2, 2, 2, 64, 16
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # the two NaN codes
    v = codes.view(torch.float8_e4m3fn).reshape(B, Hkv, 1, D)
    k = torch.zeros(B, Hkv, 1, D, dtype=torch.uint8).view(torch.float8_e4m3fn)
    kc, vc, table, _ = paging.build_paged_cache(k, v, page_size=P)
    q = torch.randn(B, Hq, 1, D, generator=_g(3)).to(qdt)
    lens = torch.ones(B, dtype=torch.int32)
    out = decode(q, kc, vc, table, lens, P)
    want = v.reshape(B, Hkv, D).to(torch.bfloat16)
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("D", [64, 128, 1024])
def test_bf16_q_over_e4m3fn_equals_fp32_q(D):
    # a bf16 q over e4m3fn caches runs as it is (no lo part); widened to fp32
    # it splits into the same hi and a zero lo, so the two decodes agree bit
    # for bit
    q, kc, vc, table, lens = make(3, 8, 2, 333, D, 16, torch.bfloat16, torch.float8_e4m3fn, seed=D + 3)
    out = decode(q, kc, vc, table, lens, 16)
    B, Hq, _, _ = q.shape
    qd, kd, vd, td, ld = (t.to(DEV) for t in (q.float(), kc, vc, table, lens))
    lib = _lib.load()
    ref = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(lib.sa_paged_decode_workspace_size(B, Hq, D, td.shape[1], 16) // 4 + 1, device=DEV)
    st = lib.sa_paged_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ref.data_ptr(), td.data_ptr(),
                             ld.data_ptr(), B, Hq, kd.shape[1], D, 16, td.shape[1], kd.shape[0], _lib.strides(qd),
                             _lib.strides(kd), _lib.strides(vd), _lib.strides(ref), td.stride(0), D ** -0.5,
                             _lib.paged_dtypes(_lib.SA_F32, _lib.SA_FP8_E4M3FN), ctypes.c_void_p(ws.data_ptr()),
                             ws.numel() * 4, torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "sa_paged_decode")
    assert torch.equal(out, ref)
