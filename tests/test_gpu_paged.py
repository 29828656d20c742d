"""Paged decode on the GPU against the CPU oracle (oracle.eager.paged_decode_eager,
pinned in test_oracle.py against the last row of causal attention).

Tolerance: bf16 output max|HIP - oracle| / max|oracle| <= 1e-2 against the
float64 oracle on the same seeded inputs; the reference's own bounds
(tests/test_paged_attention.py: max error < 0.05; test_paged_long_context.py:
< 0.1 up to 8K, finite at 16K-32K) are checked as well.
"""
import math

import pytest
import torch

import smooth_attn
from oracle import eager, paging

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


def run(q, kc, vc, table, lens, page_size, dtype=torch.bfloat16):
    out = smooth_attn.sp2norm_paged_attention(q.to(dtype).to(DEV), kc.to(dtype).to(DEV), vc.to(dtype).to(DEV),
                                              table.to(DEV), lens.to(DEV), block_size=page_size)
    assert out.dtype == torch.bfloat16 and out.shape == (q.shape[0], q.shape[1], q.shape[3])
    return out


def case(B, Hq, Hkv, T, D, seed, dtype=torch.bfloat16):
    g = _g(seed)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("B,H,T,D,BS", [(1, 4, 64, 32, 16), (2, 4, 128, 32, 16), (2, 8, 256, 64, 16),
                                        (1, 4, 48, 32, 16), (3, 4, 1000, 128, 16), (2, 4, 1, 64, 8)])
@pytest.mark.parametrize("shuffle", [False, True])
def test_paged_matches_oracle(B, H, T, D, BS, shuffle):
    q, k, v = case(B, H, H, T, D, seed=T + D + B)
    kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=BS, shuffle=shuffle, generator=_g(1))
    out = run(q, kc, vc, table, lens, BS)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2
    assert float((out.double().cpu() - ref).abs().max()) < 0.05


@pytest.mark.parametrize("hq,hkv", [(8, 2), (32, 8), (4, 1), (32, 1)])
def test_paged_gqa(hq, hkv):
    q, k, v = case(2, hq, hkv, 300, 128, seed=hq + hkv)
    kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=16, shuffle=True, generator=_g(2))
    out = run(q, kc, vc, table, lens, 16)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2


def test_paged_variable_context_lengths():
    # tests/test_paged_attention.py:175-221 with a seed, plus zero and split-crossing lengths
    lens = [32, 64, 48, 128, 0, 513, 1, 1024]
    T = max(lens)
    q, k, v = case(len(lens), 4, 4, T, 64, seed=3)
    kc, vc, table, lens_t = paging.build_paged_cache(k, v, page_size=16, shuffle=True, generator=_g(4),
                                                     context_lens=lens)
    out = run(q, kc, vc, table, lens_t, 16)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens_t)
    assert rel_err(out, ref) <= 1e-2
    assert bool((out[4] == 0).all())  # empty context -> 0 / eps = 0 (reference: o_acc / 1e-12)


@pytest.mark.parametrize("D,BS,hq,hkv", [(64, 16, 4, 1), (128, 8, 8, 2)])
def test_paged_many_skewed_sequences(D, BS, hq, hkv):
    # 300 sequences (more than one 256-wide plan chunk and 64-lane search
    # chunk), lengths skewed with empty ones: waves' tile ranges cross many
    # sequence and head boundaries.
    g = _g(D + BS)
    B = 300
    lens = torch.randint(0, 700, (B,), generator=g)
    lens[::7] = 0
    lens[5] = 4000
    lens[-1] = 1
    table, n_pages = paging.random_paged_layout(lens.tolist(), BS, generator=g)
    kc = torch.randn(n_pages, hkv, BS, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_pages, hkv, BS, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, hq, 1, D, generator=g).to(torch.bfloat16)
    out = run(q, kc, vc, table, lens.to(torch.int32), BS)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens.to(torch.int32))
    assert bool(torch.isfinite(out).all())
    assert rel_err(out, ref) <= 1e-2
    empty = (lens == 0).nonzero().flatten()
    assert bool((out[empty] == 0).all())


@pytest.mark.parametrize("D,BS", [(128, 16), (128, 64), (64, 8), (32, 8), (32, 32), (128, 1), (64, 2), (32, 4),
                                  (128, 128), (64, 256)])
def test_paged_ignores_cache_past_context(D, BS):
    # Cache slots past each sequence's length (the tail of its last page,
    # and whole pages past it) hold NaN: the output must not see them.
    lens = [1, 15, 16, 17, 100, 511, 513, 700]
    T = max(lens)
    q, k, v = case(len(lens), 8, 2, T, D, seed=D + BS)
    kc, vc, table, lens_t = paging.build_paged_cache(k, v, page_size=BS, shuffle=True, generator=_g(7),
                                                     context_lens=lens)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens_t)
    kg, vg = kc.clone(), vc.clone()
    for b, n in enumerate(lens):
        for blk in range(table.shape[1]):
            valid = max(0, min(BS, n - blk * BS))
            phys = int(table[b, blk])
            kg[phys, :, valid:] = float("nan")
            vg[phys, :, valid:] = float("nan")
    out = run(q, kg, vg, table, lens_t, BS)
    assert bool(torch.isfinite(out).all())
    assert rel_err(out, ref) <= 1e-2


@pytest.mark.parametrize("BS", [1, 2, 4, 8, 16, 32, 64, 128, 256, 1024])
def test_paged_block_sizes_agree(BS):
    # every power-of-two page size (the reference's BLOCK_SIZE = next_pow2,
    # kernels.py:2815): pages smaller than a load instruction's tokens take
    # per-lane page lookups, larger ones hold whole 32-token tiles
    q, k, v = case(2, 4, 4, 128, 32, seed=5)
    kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=BS, shuffle=True, generator=_g(BS))
    out = run(q, kc, vc, table, lens, BS)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2


def test_paged_fp16():
    q, k, v = case(2, 8, 2, 200, 64, seed=6, dtype=torch.float16)
    kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=16, shuffle=True, generator=_g(6))
    out = run(q, kc, vc, table, lens, 16, dtype=torch.float16)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2


def test_paged_long_context():
    # tests/test_paged_long_context.py:83-161: 8K parity, 32K finite
    for T, hq, hkv, D in [(8192, 8, 2, 64), (32768, 32, 8, 128)]:
        q, k, v = case(1, hq, hkv, T, D, seed=T)
        kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=16, shuffle=True, generator=_g(T))
        out = run(q, kc, vc, table, lens, 16)
        assert bool(torch.isfinite(out).all())
        ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
        assert rel_err(out, ref) <= 1e-2
        assert float((out.double().cpu() - ref).abs().max()) < 0.1


def test_paged_config5():
    """config 5: 64 sequences, ctx ~ U[512, 16384], Hq 32 / Hkv 8,
    D 128, page 16, block table a seeded permutation of all pages."""
    g = _g(5)
    B, Hq, Hkv, D, P = 64, 32, 8, 128, 16
    lens = torch.randint(512, 16385, (B,), generator=g)
    table, n_pages = paging.random_paged_layout(lens.tolist(), P, generator=g)
    kc = torch.randn(n_pages, Hkv, P, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_pages, Hkv, P, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    out = run(q, kc, vc, table, lens.to(torch.int32), P)
    sel = [0, 17, 63]
    ref = eager.paged_decode_eager(q[sel].double(), kc.double(), vc.double(), table[sel], lens[sel])
    assert rel_err(out[sel], ref) <= 1e-2
    assert bool(torch.isfinite(out).all())


def test_index_tensors_on_another_device_are_refused():
    # a host block table or context array would be dereferenced by the
    # kernel as a device pointer: the entry points refuse it before launching
    B, Hq, Hkv, P, D = 2, 4, 2, 16, 64
    q = torch.randn(B, Hq, 1, D, generator=_g(31)).bfloat16().to(DEV)
    kc = torch.zeros(4, Hkv, P, D, dtype=torch.bfloat16, device=DEV)
    table = torch.arange(2 * B, dtype=torch.int32).view(B, 2)
    lens = torch.full((B,), 20, dtype=torch.int32)
    for tab, ctx in ((table, lens.to(DEV)), (table.to(DEV), lens)):
        with pytest.raises(ValueError):
            smooth_attn.sp2norm_paged_attention(q, kc, kc, tab, ctx, block_size=P)
        with pytest.raises(ValueError):
            smooth_attn.sp2norm_paged_kv_append(kc, kc, kc[:B, :, :1], kc[:B, :, :1], tab, ctx, block_size=P)
    out = smooth_attn.sp2norm_paged_attention(q, kc, kc, table.to(DEV), lens.to(DEV), block_size=P)
    assert out.shape == (B, Hq, D) and bool((out == 0).all())  # zero V rows


@pytest.mark.parametrize("D", [8, 16, 24, 48, 80, 96, 136, 160, 200, 256, 264, 384, 512, 520, 576, 768, 1024])
@pytest.mark.parametrize("BS", [1, 16, 64])
def test_paged_head_dims(D, BS):
    # any head dim that is a multiple of 8 up to 1024 (the reference takes
    # any D through next_pow2, kernels.py:2815): kernels for 32 / 64 / 128 /
    # 256, 512 (two waves per block, each owning half the columns) and 1024
    # (four waves), smaller head dims load only their own columns
    q, k, v = case(3, 8, 2, 333, D, seed=D + BS)
    kc, vc, table, lens = paging.build_paged_cache(k, v, page_size=BS, shuffle=True, generator=_g(D))
    lens = torch.tensor([333, 1, 170], dtype=torch.int32)
    out = run(q, kc, vc, table, lens, BS)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert out.shape == (3, 8, D)
    assert rel_err(out, ref) <= 1e-2


def test_paged_head_dim_256_config5_like():
    # 64 sequences of up to 2K tokens at D = 256, GQA 16 / 4
    g = _g(256)
    B, Hq, Hkv, D, BS = 16, 16, 4, 256, 16
    lens = torch.randint(1, 2049, (B,), generator=g, dtype=torch.int32)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, int(lens.max()), D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, int(lens.max()), D, generator=g).to(torch.bfloat16)
    kc, vc, table, _ = paging.build_paged_cache(k, v, page_size=BS, shuffle=True, generator=_g(3))
    out = run(q, kc, vc, table, lens, BS)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2


def test_paged_head_dim_576_serving_layout():
    # head dim 576 (a latent-attention width) on the head-dim-1024 kernels:
    # 8 sequences of up to 2000 tokens, 16 query heads on one KV head, page
    # 64, shuffled table, bf16 caches and fp32 q over e4m3fn caches
    g = _g(576)
    B, Hq, Hkv, D, BS = 8, 16, 1, 576, 64
    lens = torch.randint(1, 2001, (B,), generator=g, dtype=torch.int32)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, int(lens.max()), D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, int(lens.max()), D, generator=g).to(torch.bfloat16)
    kc, vc, table, _ = paging.build_paged_cache(k, v, page_size=BS, shuffle=True, generator=_g(9))
    out = run(q, kc, vc, table, lens, BS)
    ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
    assert rel_err(out, ref) <= 1e-2
    k8, v8 = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
    out8 = smooth_attn.sp2norm_paged_attention(q.float().to(DEV), k8.to(DEV), v8.to(DEV), table.to(DEV),
                                               lens.to(DEV), block_size=BS)
    ref8 = eager.paged_decode_eager(q.double(), k8.double(), v8.double(), table, lens)
    assert rel_err(out8, ref8) <= 1e-2


def test_paged_head_dim_512_config5_like():
    # head dim 512 on a serving-style layout: 12 sequences of up to 3000
    # tokens, GQA 16 / 4, page 16, shuffled table; both cache dtypes
    g = _g(512)
    B, Hq, Hkv, D, BS = 12, 16, 4, 512, 16
    lens = torch.randint(1, 3001, (B,), generator=g, dtype=torch.int32)
    for dt in (torch.bfloat16, torch.float16):
        q = torch.randn(B, Hq, 1, D, generator=g).to(dt)
        k = torch.randn(B, Hkv, int(lens.max()), D, generator=g).to(dt)
        v = torch.randn(B, Hkv, int(lens.max()), D, generator=g).to(dt)
        kc, vc, table, _ = paging.build_paged_cache(k, v, page_size=BS, shuffle=True, generator=_g(7))
        out = run(q, kc, vc, table, lens, BS, dtype=dt)
        ref = eager.paged_decode_eager(q.double(), kc.double(), vc.double(), table, lens)
        assert rel_err(out, ref) <= 1e-2
