"""The allocation-free paged decode, sa_paged_decode_noalloc, on the GPU
through the C ABI, against the workspace entry point sa_paged_decode
(through sp2norm_paged_attention) on the same inputs, and against the CPU
oracle.

Bar: where both entry points use the same split (their partials fit the
64 MiB scratch) they run the same kernels on the same plan, so the outputs
must be bit-identical; where the scratch forces a coarser split the
partials are summed in another grouping, so the bf16 outputs are held to
the path's 1e-2 bar (max|a - b| / max|b|) against each other and against
the float64 oracle.  Calls follow each other on one device, the second one
smaller, so the second reads a scratch array still holding the first one's
plan and partials.
"""
import math

import pytest
import torch

import smooth_attn
from oracle import eager
from oracle.paging import random_paged_layout
from smooth_attn import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


def call_noalloc(out, q, kc, vc, table, lens, page_size, stream=None):
    """sa_paged_decode_noalloc into ``out`` on ``stream`` (default: the current one)."""
    B, Hq, _, D = q.shape
    dtype = {torch.bfloat16: _lib.SA_BF16, torch.float16: _lib.SA_F16}[q.dtype]
    raw = torch._C._cuda_getCurrentRawStream(q.device.index) if stream is None else stream.cuda_stream
    st = _lib.load().sa_paged_decode_noalloc(
        q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), table.data_ptr(), lens.data_ptr(), B, Hq,
        kc.shape[1], D, page_size, table.shape[1], kc.shape[0], _lib.strides(q), _lib.strides(kc),
        _lib.strides(vc), _lib.strides(out), table.stride(0), 1.0 / math.sqrt(D), dtype, raw)
    _lib.check(st, "sa_paged_decode_noalloc")
    return out


def decode_noalloc(q, kc, vc, table, lens, page_size):
    """sp2norm_paged_attention's arguments, through sa_paged_decode_noalloc."""
    B, Hq, _, D = q.shape
    out = torch.empty(B, Hq, D, device=q.device, dtype=torch.bfloat16)
    return call_noalloc(out, q, kc, vc, table, lens, page_size)


def make_case(B, Hq, Hkv, D, P, max_ctx, seed, dtype=torch.bfloat16, table_pages=None):
    """Seeded contexts in [1, max_ctx], a shuffled serving-style block table
    (optionally wider than the contexts need) and random caches."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_ctx + 1, (B,), generator=g)
    table, n_pages = random_paged_layout(lens, P, generator=g)
    if table_pages is not None and table_pages > table.shape[1]:
        table = torch.cat([table, torch.zeros(B, table_pages - table.shape[1], dtype=torch.int32)], 1)
    kc = torch.randn(n_pages, Hkv, P, D, generator=g).to(dtype)
    vc = torch.randn(n_pages, Hkv, P, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dtype)
    cpu = (q, kc, vc, table, lens.to(torch.int32))
    return cpu, tuple(t.to(DEV) for t in cpu)


def workspace_bytes(B, Hq, D, max_pages, P):
    return _lib.load().sa_paged_decode_workspace_size(B, Hq, D, max_pages, P)


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: 16 sequences of up to 3000 tokens, Hq 32 / Hkv 8, D 128
    cpu, dev = make_case(16, 32, 8, 128, 16, 3000, seed=1)
    assert workspace_bytes(16, 32, 128, dev[3].shape[1], 16) <= _lib.PAGED_NOALLOC_SCRATCH_BYTES
    got = decode_noalloc(*dev, 16)
    want = smooth_attn.sp2norm_paged_attention(*dev, block_size=16)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert rel_err(got, eager.paged_decode_eager(*(t.double() if t.is_floating_point() else t for t in cpu))) <= 1e-2
    # second call, smaller: 3 sequences of up to 200 tokens, fp16, Hq 8 / Hkv 2,
    # D 64, page 8; the scratch still holds the first call's plan and partials
    cpu, dev = make_case(3, 8, 2, 64, 8, 200, seed=2, dtype=torch.float16)
    got = decode_noalloc(*dev, 8)
    want = smooth_attn.sp2norm_paged_attention(*dev, block_size=8)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert rel_err(got, eager.paged_decode_eager(*(t.double() if t.is_floating_point() else t for t in cpu))) <= 1e-2


def test_noalloc_coarsens_the_split_when_the_partials_do_not_fit():
    # 64 sequences x 64 query heads with a 1024-page (16K-token) table: the
    # workspace entry point's partials take about 70 MB, over the 64 MiB
    # scratch, so the allocation-free call runs a coarser split.  Contexts
    # stay short (at most 700 tokens) to keep the oracle quick.
    B, Hq, Hkv, D, P = 64, 64, 8, 128, 16
    cpu, dev = make_case(B, Hq, Hkv, D, P, 700, seed=3, table_pages=1024)
    assert workspace_bytes(B, Hq, D, 1024, P) > _lib.PAGED_NOALLOC_SCRATCH_BYTES
    got = decode_noalloc(*dev, P)
    want = smooth_attn.sp2norm_paged_attention(*dev, block_size=P)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(got.float()).all())
    assert rel_err(got, want) <= 1e-2
    ref = eager.paged_decode_eager(*(t.double() if t.is_floating_point() else t for t in cpu))
    assert rel_err(got, ref) <= 1e-2
    # and a smaller call right after it, back on the uncoarsened split
    cpu, dev = make_case(5, 32, 8, 128, 16, 1000, seed=4)
    got = decode_noalloc(*dev, 16)
    torch.cuda.synchronize()
    assert torch.equal(got, smooth_attn.sp2norm_paged_attention(*dev, block_size=16))


@pytest.mark.parametrize("P,D,dtype", [(1, 64, torch.float16), (128, 32, torch.bfloat16), (4, 128, torch.bfloat16),
                                     (16, 576, torch.float16), (16, 1024, torch.bfloat16)])
def test_noalloc_page_sizes_and_head_dims(P, D, dtype):
    # the allocation-free call on the page sizes and head dims the workspace
    # entry point takes, against it (same split: bit-identical) and the oracle
    cpu, dev = make_case(6, 16, 4, D, P, 900, seed=10 + P, dtype=dtype)
    got = decode_noalloc(*dev, P)
    want = smooth_attn.sp2norm_paged_attention(*dev, block_size=P)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ref = eager.paged_decode_eager(*(t.double() if t.is_floating_point() else t for t in cpu))
    assert rel_err(got, ref) <= 1e-2


def test_noalloc_replays_under_graph_capture_and_allocates_nothing():
    # after one eager call (the first call on a device looks up the scratch
    # address and sizes the launch on the host), the call allocates no
    # device memory and can be captured in a HIP graph: every replay equals
    # the eager output bit for bit, also when other allocation-free calls on
    # other inputs (which overwrite the shared scratch) run between replays
    cpu, dev = make_case(8, 32, 8, 128, 16, 2000, seed=21)
    want = decode_noalloc(*dev, 16)
    other = make_case(3, 8, 2, 128, 16, 500, seed=22)[1]
    out_other = torch.empty(3, 8, 128, device=DEV, dtype=torch.bfloat16)
    call_noalloc(out_other, *other, 16)
    out = torch.zeros_like(want)
    torch.cuda.synchronize()
    before_torch = torch.cuda.memory_allocated()
    before_free = torch.cuda.mem_get_info()[0]
    call_noalloc(out, *dev, 16)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == before_free
    assert torch.cuda.memory_allocated() == before_torch
    assert torch.equal(out, want)

    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=stream):
        call_noalloc(out, *dev, 16, stream=stream)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        call_noalloc(out_other, *other, 16)  # eager work on the shared scratch between replays
        torch.cuda.synchronize()
