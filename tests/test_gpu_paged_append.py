"""Paged-KV cache writer (HIP) against the CPU oracle (GPU).

Bit-exact: the writer only moves bytes (fp32, bf16 or fp16 rows), so the device caches must
equal oracle.paging.append_kv on the same inputs exactly; decode after a
sequence of appends must equal decode of the cache built in one piece.
"""
import pytest
import torch

import smooth_attn
from oracle import paging

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


CASES = [(dt, P, D, n) for dt in (torch.bfloat16, torch.float16, torch.float32)
         for P, D, n in ((16, 128, 1), (16, 64, 7), (8, 32, 33), (32, 128, 5))]
CASES += [(torch.float32, 4, 12, 9), (torch.bfloat16, 4, 24, 9)]  # 16-byte rows: fp32 D % 4, 16-bit D % 8
CASES += [(torch.float8_e4m3fn, 16, 64, 7), (torch.float8_e4m3fn, 8, 32, 33)]  # e4m3fn: D % 16


@pytest.mark.parametrize("dtype,P,D,n_new", CASES)
def test_append_matches_oracle(dtype, P, D, n_new):
    B, H, T = 3, 2, 70
    k = torch.randn(B, H, T, D, generator=_g(P + D)).to(dtype)
    v = torch.randn(B, H, T, D, generator=_g(P + D + 1)).to(dtype)
    kc, vc, table, _ = paging.build_paged_cache(k, v, P, shuffle=True, generator=_g(5))
    ctx = torch.tensor([0, 17, 70 - n_new], dtype=torch.int32)
    kn = torch.randn(B, H, n_new, D, generator=_g(6)).to(dtype)
    vn = torch.randn(B, H, n_new, D, generator=_g(7)).to(dtype)
    ref_k, ref_v = paging.append_kv(kc, vc, kn, vn, table, ctx)
    kd, vd = kc.to(DEV), vc.to(DEV)
    new_ctx = smooth_attn.sp2norm_paged_kv_append(kd, vd, kn.to(DEV), vn.to(DEV), table.to(DEV), ctx.to(DEV),
                                                  block_size=P)
    assert torch.equal(kd.cpu().view(torch.uint8), ref_k.view(torch.uint8))
    assert torch.equal(vd.cpu().view(torch.uint8), ref_v.view(torch.uint8))
    assert torch.equal(new_ctx.cpu(), ctx + n_new)


def test_append_skips_rows_outside_table_and_cache():
    B, H, P, D = 2, 2, 16, 64
    k = torch.randn(B, H, 32, D, generator=_g(8)).bfloat16()
    kc, vc, table, _ = paging.build_paged_cache(k, k, P, generator=_g(9))
    bad = table.clone()
    bad[1, 1] = 10_000  # outside the cache
    ctx = torch.tensor([30, 20], dtype=torch.int32)  # seq 0 runs past its 2 pages
    kn = torch.randn(B, H, 8, D, generator=_g(10)).bfloat16()
    ref_k, ref_v = paging.append_kv(kc, vc, kn, kn, bad, ctx)
    kd, vd = kc.to(DEV), vc.to(DEV)
    smooth_attn.sp2norm_paged_kv_append(kd, vd, kn.to(DEV), kn.to(DEV), bad.to(DEV), ctx.to(DEV), block_size=P)
    assert torch.equal(kd.cpu(), ref_k) and torch.equal(vd.cpu(), ref_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_after_appends_equals_prebuilt_cache(dtype):
    # prefill 50 tokens, then 3 single-token decode steps, against a cache built at once
    B, Hq, Hkv, P, D, T = 2, 8, 2, 16, 128, 53
    k = torch.randn(B, Hkv, T, D, generator=_g(11)).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=_g(12)).to(dtype)
    q = torch.randn(B, Hq, 1, D, generator=_g(13)).to(dtype)
    full_k, full_v, table, lens = paging.build_paged_cache(k, v, P, shuffle=True, generator=_g(14))
    kd = torch.zeros_like(full_k).to(DEV)
    vd = torch.zeros_like(full_v).to(DEV)
    tab = table.to(DEV)
    ctx = torch.zeros(B, dtype=torch.int32, device=DEV)
    ctx = smooth_attn.sp2norm_paged_kv_append(kd, vd, k[:, :, :50].to(DEV), v[:, :, :50].to(DEV), tab, ctx)
    for t in range(50, T):
        ctx = smooth_attn.sp2norm_paged_kv_append(kd, vd, k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), tab, ctx)
    assert torch.equal(kd.cpu(), full_k) and torch.equal(vd.cpu(), full_v)
    assert torch.equal(ctx.cpu(), lens)
    o1 = smooth_attn.sp2norm_paged_attention(q.to(DEV), kd, vd, tab, ctx)
    o2 = smooth_attn.sp2norm_paged_attention(q.to(DEV), full_k.to(DEV), full_v.to(DEV), tab, lens.to(DEV))
    assert torch.equal(o1, o2)
