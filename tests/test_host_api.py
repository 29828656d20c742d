"""Host-side behaviour of the drop-in API — CPU only, no kernel launches.

Mirrors the reference's CPU-runnable tests (tests/test_family_config.py:4-19)
and the validation errors it raises before any launch (kernels.py:71-73,
150-240, 1420, 2032-2036, 2795-2799).
"""
import inspect

import pytest
import torch

import smooth_attn
from smooth_attn import FamilyConfig, kernels

REFERENCE_EXPORTS = [
    "BENCH_ALPHA", "BENCH_POWER", "BENCH_THETA", "DEFAULT_FAMILY", "CausalBenchmarkResult", "FamilyConfig",
    "RowwiseBenchmarkResult", "SoftplusNormCausal", "bench", "bench_out", "benchmark_causal_suite",
    "benchmark_rowwise_suite", "main", "softmax_causal_eager", "softmax_causal_triton",
    "softmax_causal_triton_out", "softmax_triton", "softmax_triton_out", "softplus_norm_causal",
    "softplus_norm_causal_eager", "softplus_norm_causal_triton", "softplus_norm_causal_triton_out",
    "softplus_norm_eager", "softplus_norm_triton", "softplus_norm_triton_out", "sp2norm_flash_attention",
    "sp2norm_flash_attention_eager", "sp2norm_fp8_flash_attention", "sp2norm_rope_flash_attention",
    "sp2norm_rope_flash_attention_proj", "sp2norm_paged_attention", "precompute_rope_cos_sin", "sp2norm_triton",
]


# Exports added here with no reference counterpart (the paged-KV writer).
EXTRA_EXPORTS = ["sp2norm_paged_kv_append"]


def test_export_list_matches_reference():
    assert sorted(smooth_attn.__all__) == sorted(REFERENCE_EXPORTS + EXTRA_EXPORTS)
    for name in REFERENCE_EXPORTS + EXTRA_EXPORTS:
        assert hasattr(smooth_attn, name), name


def test_family_config_rejects_bad_power():
    with pytest.raises(ValueError):
        FamilyConfig(power=4)


def test_family_config_rejects_removed_activation_kwarg():
    with pytest.raises(TypeError):
        FamilyConfig(activation="softplus")


def test_family_config_properties():
    f = FamilyConfig(alpha=1.5, theta=0.25, power=3)
    assert f.cache_key == (1.5, 0.25, 3)
    assert f.kernel_kwargs == {"ALPHA": 1.5, "THETA": 0.25, "POWER": 3}
    assert f.label == "squareplus(1.5 * (x - 0.25))^3 / sum"
    assert smooth_attn.DEFAULT_FAMILY == FamilyConfig()
    assert (smooth_attn.BENCH_ALPHA, smooth_attn.BENCH_THETA, smooth_attn.BENCH_POWER) == (2.0, 0.5, 2)


def test_family_and_overrides_conflict():
    with pytest.raises(ValueError, match="not both"):
        kernels._resolve_family(1.0, 0.5, 2, FamilyConfig())
    assert kernels._resolve_family(2.0, 0.5, 2, FamilyConfig(power=3)).power == 3


def test_signatures_match_reference():
    sig = inspect.signature(smooth_attn.softplus_norm_causal_triton_out)
    assert list(sig.parameters) == ["out", "x", "alpha", "theta", "power", "family", "return_meta"]
    sig = inspect.signature(smooth_attn.sp2norm_flash_attention)
    assert list(sig.parameters) == ["q", "k", "v", "scale", "window_size", "exact_math"]
    sig = inspect.signature(smooth_attn.sp2norm_paged_attention)
    assert list(sig.parameters) == ["q", "k_cache", "v_cache", "block_table", "context_lens", "scale",
                                    "block_size"]
    sig = inspect.signature(smooth_attn.SoftplusNormCausal.__init__)
    assert list(sig.parameters) == ["self", "alpha", "theta", "power", "family", "implementation"]


def test_rejects_non_tensor_and_cpu_tensor():
    with pytest.raises(TypeError):
        smooth_attn.softplus_norm_triton([1.0, 2.0])
    with pytest.raises(ValueError, match="CUDA tensor"):
        smooth_attn.softplus_norm_triton(torch.zeros(4, 4))
    with pytest.raises(ValueError, match="CUDA tensor"):
        smooth_attn.softplus_norm_causal_triton(torch.zeros(1, 4, 4))


def test_implementation_switch():
    x = torch.randn(1, 2, 8, 8).to(torch.bfloat16)
    y = smooth_attn.softplus_norm_causal(x, implementation="eager")
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
    with pytest.raises(ValueError, match="implementation"):
        smooth_attn.softplus_norm_causal(x, implementation="cuda")


def test_eager_functions_run_on_cpu():
    x = torch.randn(2, 6, 6)
    torch.testing.assert_close(smooth_attn.softplus_norm_causal_eager(x).sum(-1), torch.ones(2, 6), atol=1e-5,
                               rtol=0)
    q = torch.randn(1, 2, 5, 4)
    o = smooth_attn.sp2norm_flash_attention_eager(q, q, q)
    assert o.shape == q.shape
    s = smooth_attn.softmax_causal_eager(x)
    torch.testing.assert_close(s.sum(-1), torch.ones(2, 6))


def test_flash_asserts_shapes():
    q = torch.zeros(1, 4, 8, 16)
    with pytest.raises(AssertionError):
        smooth_attn.sp2norm_flash_attention(q, torch.zeros(1, 3, 8, 16), torch.zeros(1, 3, 8, 16))
    with pytest.raises(AssertionError):
        smooth_attn.sp2norm_flash_attention(q[0], q[0], q[0])
    with pytest.raises(AssertionError):
        smooth_attn.sp2norm_paged_attention(torch.zeros(1, 4, 2, 16), torch.zeros(2, 4, 16, 16),
                                            torch.zeros(2, 4, 16, 16), torch.zeros(1, 2, dtype=torch.int32),
                                            torch.zeros(1, dtype=torch.int32))


def test_cli_parsing_matches_reference_defaults():
    # kernels.py:3061-3075 options and defaults; :150-164 list parsing
    from smooth_attn import cli
    a = cli.parse_args([])
    assert (a.mode, a.dtypes, a.lengths, a.batch, a.heads, a.warmup, a.iters) == \
        ("causal", "bf16", "128,256,512,1024", 2, 8, 50, 200)
    assert (a.alpha, a.theta, a.power, a.quick, a.check_backward) == (2.0, 0.5, 2, False, False)
    a = cli.parse_args(["--mode", "all", "--dtypes", "fp32,bf16", "--quick", "--check-backward"])
    assert a.mode == "all" and a.quick and a.check_backward
    assert cli._parse_dtype_list(" FP32, bf16 ,fp16") == [torch.float32, torch.bfloat16, torch.float16]
    assert cli._parse_int_list("128, 256,") == [128, 256]
    with pytest.raises(ValueError):
        cli._parse_dtype_list("fp64")
    with pytest.raises(ValueError):
        cli._parse_int_list(" , ")
    assert cli._dtype_label(torch.bfloat16) == "bf16" and cli._dtype_label(torch.int8) == "int8"
    assert len(cli.DEFAULT_ROWWISE_SHAPES) == 24
    with pytest.raises(SystemExit):
        cli.parse_args(["--mode", "bogus"])


def test_softmax_entry_points_validate_before_launch():
    import smooth_attn
    with pytest.raises(TypeError):
        smooth_attn.softmax_triton([1.0, 2.0])
    with pytest.raises(ValueError):
        smooth_attn.softmax_triton(torch.zeros(2, 2))  # not a device tensor
    with pytest.raises(ValueError):
        smooth_attn.softmax_causal_triton(torch.zeros(2, 3))


def test_paged_entry_points_reject_short_tables_before_launch():
    # the kernels read B block-table rows, B context lengths and D-wide cache
    # rows: shorter arrays are refused on the host, before any device call
    B, Hq, Hkv, P, D = 3, 4, 2, 16, 32
    q = torch.zeros(B, Hq, 1, D, dtype=torch.bfloat16)
    kc = torch.zeros(6, Hkv, P, D, dtype=torch.bfloat16)
    table = torch.zeros(B, 2, dtype=torch.int32)
    lens = torch.full((B,), 5, dtype=torch.int32)
    bad = [
        (kc, table[:2], lens),                         # block table shorter than B
        (kc, table, lens[:2]),                         # fewer context lengths than B
        (kc[..., :16].contiguous(), table, lens),      # cache rows narrower than D
        (kc, table.float(), lens),                     # floating-point block table
    ]
    messages = ["block_table must be", "context_lens must hold", "caches must both be", "integer tensors"]
    for (cache, tab, ctx), msg in zip(bad, messages):
        with pytest.raises(ValueError, match=msg):
            kernels._check_paging_args(B, D, cache, cache, tab, ctx)
        # the public entry points refuse these host tensors before any launch
        with pytest.raises(ValueError):
            smooth_attn.sp2norm_paged_attention(q, cache, cache, tab, ctx, block_size=P)
    new = torch.zeros(B, Hkv, 1, D, dtype=torch.bfloat16)
    for cache, tab, ctx in bad[:2] + bad[3:]:
        with pytest.raises(ValueError):
            smooth_attn.sp2norm_paged_kv_append(cache, cache, new, new, tab, ctx, block_size=P)


class _OnDevice(torch.Tensor):
    """A host tensor that reports itself as living on a given CUDA device:
    enough for the host-side device checks, which never dereference it."""

    @staticmethod
    def make(t, index):
        out = torch.Tensor._make_subclass(_OnDevice, t)
        out._index = index
        return out

    @property
    def is_cuda(self):
        return True

    @property
    def device(self):
        return torch.device("cuda", getattr(self, "_index", 0))  # views of a cuda:0 tensor


@pytest.fixture
def no_library(monkeypatch):
    """Any attempt to reach the HIP library fails the test: the device checks
    must fire before it is loaded."""
    from smooth_attn import _lib

    def fail():
        raise AssertionError("the HIP library was reached before the device check")

    monkeypatch.setattr(_lib, "load", fail)


def _fused_calls(mk, alt):
    """(label, call) for every fused entry point, built from the tensor maker
    ``mk(shape, dtype)`` (the reference device) with ``alt`` applied to the
    argument under test."""
    B, Hq, Hkv, T, D, P = 1, 4, 2, 16, 32, 16
    bf = torch.bfloat16
    q = mk((B, Hq, T, D), bf)
    k, v = mk((B, Hkv, T, D), bf), mk((B, Hkv, T, D), bf)
    o, do = mk((B, Hq, T, D), bf), mk((B, Hq, T, D), bf)
    rs = mk((B, Hq, T), torch.float32)
    cos, sin = mk((T, D // 2), torch.float32), mk((T, D // 2), torch.float32)
    w_o = mk((Hq, D, 64), bf)
    q8, k8 = mk((B, Hq, T, D), torch.float8_e4m3fn), mk((B, Hkv, T, D), torch.float8_e4m3fn)
    qd = mk((B, Hq, 1, D), bf)
    kc, vc = mk((4, Hkv, P, D), bf), mk((4, Hkv, P, D), bf)
    tab, lens = mk((B, 4), torch.int32), mk((B,), torch.int32)
    kn = mk((B, Hkv, 2, D), bf)
    x, g = mk((2, 8, 8), bf), mk((2, 8, 8), bf)
    fam = FamilyConfig()
    return [
        ("flash k", lambda: kernels._sp2norm_flash_fwd(q, alt(k), v, 0.1, 2)),
        ("flash v", lambda: kernels._sp2norm_flash_fwd(q, k, alt(v), 0.1, 2)),
        ("public flash", lambda: smooth_attn.sp2norm_flash_attention(q, alt(k), v)),
        ("flash bwd do", lambda: kernels._sp2norm_flash_bwd(q, k, v, o, alt(do), rs, 0.1, 2)),
        ("flash bwd row_sums", lambda: kernels._sp2norm_flash_bwd(q, k, v, o, do, alt(rs), 0.1, 2)),
        ("flash bwd o", lambda: kernels._sp2norm_flash_bwd(q, k, v, alt(o), do, rs, 0.1, 2)),
        ("rope cos", lambda: smooth_attn.sp2norm_rope_flash_attention(q, k, v, alt(cos), sin)),
        ("rope sin", lambda: smooth_attn.sp2norm_rope_flash_attention(q, k, v, cos, alt(sin))),
        ("rope v", lambda: smooth_attn.sp2norm_rope_flash_attention(q, k, alt(v), cos, sin)),
        ("rope proj w_o", lambda: smooth_attn.sp2norm_rope_flash_attention_proj(q, k, v, alt(w_o), cos, sin)),
        ("fp8 k8", lambda: kernels._sp2norm_fp8_flash_fwd(q8, alt(k8), v, 1.0, 1.0, None, 0.1, 2)),
        ("fp8 v", lambda: kernels._sp2norm_fp8_flash_fwd(q8, k8, alt(v), 1.0, 1.0, None, 0.1, 2)),
        ("fp8 public v", lambda: smooth_attn.sp2norm_fp8_flash_attention(q, k, alt(v))),
        ("paged k_cache", lambda: smooth_attn.sp2norm_paged_attention(qd, alt(kc), vc, tab, lens)),
        ("paged v_cache", lambda: smooth_attn.sp2norm_paged_attention(qd, kc, alt(vc), tab, lens)),
        ("paged table", lambda: smooth_attn.sp2norm_paged_attention(qd, kc, vc, alt(tab), lens)),
        ("paged lens", lambda: smooth_attn.sp2norm_paged_attention(qd, kc, vc, tab, alt(lens))),
        ("append k_new", lambda: smooth_attn.sp2norm_paged_kv_append(kc, vc, alt(kn), kn, tab, lens)),
        ("append table", lambda: smooth_attn.sp2norm_paged_kv_append(kc, vc, kn, kn, alt(tab), lens)),
        ("norm bwd dy", lambda: kernels._softplus_norm_causal_backward(x, alt(g), fam)),
        ("rowwise bwd dy", lambda: kernels._softplus_norm_backward(x[0], alt(g[0]), fam)),
    ]


@pytest.mark.parametrize("case", range(21))
def test_fused_entry_points_refuse_host_tensors(case, no_library):
    # one argument left on the host while the rest claim cuda:0
    mk = lambda shape, dtype: _OnDevice.make(torch.zeros(shape, dtype=dtype), 0)
    label, call = _fused_calls(mk, lambda t: t.as_subclass(torch.Tensor))[case]
    with pytest.raises(ValueError, match="must be a CUDA tensor"):
        call()


@pytest.mark.parametrize("case", range(21))
def test_fused_entry_points_refuse_mixed_devices(case, no_library):
    # one argument on cuda:1 while the rest are on cuda:0
    mk = lambda shape, dtype: _OnDevice.make(torch.zeros(shape, dtype=dtype), 0)
    label, call = _fused_calls(mk, lambda t: _OnDevice.make(t.as_subclass(torch.Tensor), 1))[case]
    with pytest.raises(ValueError, match="same CUDA device"):
        call()


@pytest.mark.parametrize("case", range(21))
def test_fused_entry_points_refuse_meta_tensors(case, no_library):
    mk = lambda shape, dtype: torch.empty(shape, dtype=dtype, device="meta")
    label, call = _fused_calls(mk, lambda t: t)[case]
    with pytest.raises(ValueError, match="must be a CUDA tensor"):
        call()


def test_head_dims_and_page_sizes_checked_before_launch(no_library):
    # fused attention, fp8 included: head dims up to 512 (16-bit: rounded
    # up to a multiple of 8, fp32 of 4; fp8:
    # zero-padded to a built size, or widened to bf16 above 128); larger head
    # dims, fp64 and mixed dtypes are refused with a clear error; paged
    # decode: power-of-two page sizes only
    mk = lambda shape, dtype: _OnDevice.make(torch.zeros(shape, dtype=dtype), 0)
    for D, dts, lim in ((513, (torch.float32, torch.bfloat16, torch.float16), 512),
                        (1024, (torch.float32, torch.bfloat16, torch.float16), 512)):
        for dt in dts:
            q = mk((1, 2, 8, D), dt)
            with pytest.raises(ValueError, match=f"head dims 1..{lim}"):
                kernels._sp2norm_flash_fwd(q, q, q, 0.1)
            with pytest.raises(ValueError, match=f"head dims 1..{lim}"):
                kernels._sp2norm_flash_bwd(q, q, q, q, q, mk((1, 2, 8), torch.float32), 0.1)
    q8 = mk((1, 2, 8, 520), torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="head dims 1..512"):
        kernels._sp2norm_fp8_flash_fwd(q8, q8, q8, 1.0, 1.0, 1.0, 0.1)
    dims = (1, 16, 32, 33, 64, 96, 128, 129, 200, 256)
    # 16-bit: multiples of 8 run as they are (columns past D masked in the kernels)
    assert [kernels._kernel_head_dim(d, torch.bfloat16) for d in dims] == [8, 16, 32, 40, 64, 96, 128, 136, 200, 256]
    assert [kernels._kernel_head_dim(d, torch.bfloat16) for d in (257, 300, 511, 512)] == [264, 304, 512, 512]
    assert [kernels._kernel_head_dim(d, torch.float32) for d in dims] == [4, 16, 32, 36, 64, 96, 128, 132, 200, 256]
    assert [kernels._kernel_head_dim(d) for d in dims[:7]] == [32, 32, 32, 64, 64, 128, 128]
    q = mk((1, 2, 8, 64), torch.float64)
    with pytest.raises(ValueError, match="bf16, fp16 or fp32"):
        kernels._sp2norm_flash_fwd(q, q, q, 0.1)
    with pytest.raises(ValueError, match="bf16, fp16 or fp32"):
        kernels._sp2norm_flash_bwd(q, q, q, q, q, mk((1, 2, 8), torch.float32), 0.1)
    q32, k16 = mk((1, 2, 8, 64), torch.float32), mk((1, 2, 8, 64), torch.bfloat16)
    with pytest.raises(ValueError, match="of one dtype"):
        kernels._sp2norm_flash_fwd(q32, k16, k16, 0.1)
    qd = torch.zeros(2, 4, 1, 32, dtype=torch.bfloat16)
    kc = torch.zeros(4, 2, 12, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="power of two"):
        smooth_attn.sp2norm_paged_attention(qd, kc, kc, torch.zeros(2, 2, dtype=torch.int32),
                                            torch.ones(2, dtype=torch.int32), block_size=12)
    for D in (4, 12, 516, 1032, 2048):  # paged decode: multiples of 8 in 8..1024
        qd = torch.zeros(2, 4, 1, D, dtype=torch.bfloat16)
        kc = torch.zeros(4, 2, 16, D, dtype=torch.bfloat16)
        with pytest.raises(ValueError, match="multiples of 8 in 8..1024"):
            smooth_attn.sp2norm_paged_attention(qd, kc, kc, torch.zeros(2, 2, dtype=torch.int32),
                                                torch.ones(2, dtype=torch.int32))
    for qdt, cdt in ((torch.float32, torch.float32), (torch.float32, torch.float16), (torch.bfloat16, torch.float16)):
        # caches read as bf16 hi + lo tiles stop at 512
        qd = torch.zeros(2, 4, 1, 520, dtype=qdt)
        kc = torch.zeros(4, 2, 16, 520, dtype=cdt)
        with pytest.raises(ValueError, match="up to 512"):
            smooth_attn.sp2norm_paged_attention(qd, kc, kc, torch.zeros(2, 2, dtype=torch.int32),
                                                torch.ones(2, dtype=torch.int32))
