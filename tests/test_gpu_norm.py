"""Parity of the HIP normalisation kernels with the CPU oracle (GPU).

Tolerances (the path's stated bars): relative error max|HIP - oracle| /
max|oracle| <= 1e-2 for bf16/fp16 outputs and <= 1e-5 for fp32 outputs,
against the float64 oracle on the same seeded inputs; causal zeros exact.
The reference's own test tolerances (tests/test_training_api.py:36-78: atol
5e-3, rtol 5e-2 vs eager) are checked as well where they apply.
"""
import pytest
import torch

import smooth_attn
from oracle import eager
from smooth_attn import FamilyConfig, kernels

pytestmark = pytest.mark.gpu

DEV = "cuda"
REL_TOL = {torch.bfloat16: 1e-2, torch.float16: 1e-2, torch.float32: 1e-5}
FAMILIES = [FamilyConfig(), FamilyConfig(alpha=1.5, theta=0.25, power=3), FamilyConfig(alpha=0.75, theta=-0.5, power=1)]


def _g(seed):
    return torch.Generator().manual_seed(seed)


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


def _randn(shape, dtype, seed, scale=1.0):
    return (torch.randn(shape, generator=_g(seed)) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("L", [1, 7, 64, 100, 512, 1024])
@pytest.mark.parametrize("fam", FAMILIES, ids=["default", "a1.5t.25p3", "a.75t-.5p1"])
def test_causal_forward_matches_oracle(dtype, L, fam):
    x = _randn((2, 3, L, L), dtype, seed=L)
    out = torch.empty(x.shape, dtype=dtype, device=DEV)
    y, meta = smooth_attn.softplus_norm_causal_triton_out(out, x.to(DEV), family=fam, return_meta=True)
    assert y.data_ptr() == out.data_ptr()
    ref = eager.softplus_norm_causal_eager(x.double(), fam.alpha, fam.theta, fam.power)
    assert rel_err(y, ref) <= REL_TOL[dtype]
    yc = y.cpu()
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((yc[..., upper] == 0).all()), "causal zeros must be exact"
    torch.testing.assert_close(yc.float(), ref.float(), atol=7e-3, rtol=5e-2)
    if fam == FamilyConfig():
        assert meta["variant"].startswith("squareplus_winner")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [64, 512, 2048])
def test_rowwise_forward_matches_oracle(dtype, L):
    x = _randn((33, L), dtype, seed=L + 1)
    y = smooth_attn.softplus_norm_triton(x.to(DEV))
    ref = eager.softplus_norm_eager(x.double())
    assert rel_err(y, ref) <= REL_TOL[dtype]
    out = torch.empty(x.shape, dtype=dtype, device=DEV)
    y2 = smooth_attn.softplus_norm_triton_out(out, x.to(DEV), family=FamilyConfig(power=3))
    assert rel_err(y2, eager.softplus_norm_eager(x.double(), power=3)) <= REL_TOL[dtype]
    y3 = smooth_attn.sp2norm_triton(x.to(DEV))
    assert torch.equal(y3, y)


@pytest.mark.parametrize("dtype,gdtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                          (torch.float16, torch.float16), (torch.float32, torch.float32)])
@pytest.mark.parametrize("L", [5, 32, 256, 1024])
@pytest.mark.parametrize("fam", FAMILIES, ids=["default", "a1.5t.25p3", "a.75t-.5p1"])
def test_causal_backward_matches_oracle(dtype, gdtype, L, fam):
    x = _randn((2, 2, L, L), dtype, seed=3 * L)
    dy = _randn((2, 2, L, L), gdtype, seed=3 * L + 1)
    dx = kernels._softplus_norm_causal_backward(x.to(DEV), dy.to(DEV), fam)
    assert dx.dtype == dtype
    ref = eager.softplus_norm_backward(x.double(), dy.double(), fam.alpha, fam.theta, fam.power, causal=True)
    assert rel_err(dx, ref) <= REL_TOL[dtype]
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((dx.cpu()[..., upper] == 0).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [48, 1024])
def test_rowwise_backward_matches_oracle(dtype, L):
    x = _randn((40, L), dtype, seed=5 * L)
    dy = _randn((40, L), dtype, seed=5 * L + 1)
    dx = kernels._softplus_norm_backward(x.to(DEV), dy.to(DEV), FamilyConfig())
    ref = eager.softplus_norm_backward(x.double(), dy.double(), causal=False)
    assert rel_err(dx, ref) <= REL_TOL[dtype]


# Rows long enough to take the split kernels (several waves per row): 8
# chunks of 1 KB -> 4 waves, 16 or more -> 8 waves.  fp32 L=2048 (R=4) and
# L=4096 (R=8) are config 2's row-wise fp32 lengths.
SPLIT_CASES = [
    (torch.float32, 2048, 4), (torch.float32, 4096, 8), (torch.float32, 8192, 8),
    (torch.bfloat16, 4096, 4), (torch.bfloat16, 8192, 8), (torch.float16, 8192, 8),
]
SPLIT_IDS = [f"{str(d).split('.')[-1]}-L{L}-R{r}" for d, L, r in SPLIT_CASES]


def _check_row_kernel(dtype, L, waves, causal):
    """The launch metadata names the split kernel with ``waves`` per row."""
    if causal:
        _, meta = smooth_attn.softplus_norm_causal_triton(_randn((1, 1, L, L), dtype, seed=L).to(DEV),
                                                          return_meta=True)
    else:
        _, meta = smooth_attn.softplus_norm_triton(_randn((2, L), dtype, seed=L).to(DEV), return_meta=True)
    assert meta["kernel"] == "split" and meta["waves_per_row"] == waves


def _gradient_invariant(x, dy, dx, fam):
    """Per-row |sum_j dx_j r_j| / (sum_j |dx_j r_j| + alpha p max_j |dy_j|),
    r_j = sqrt(a_j^2 + 4), a = alpha (x - theta).  Since
    dx_j = alpha p y_j (dy_j - T) / r_j with T = sum_k dy_k y_k, the sum is
    alpha p T (1 - sum_j y_j) = O(eps): every row's ratio is rounding noise.
    The denominator bounds the rounding of the terms and of T (which enters
    every term coherently).  Computed in fp32 on the device."""
    r = fam.alpha * (x.float() - fam.theta)
    r.mul_(r).add_(4.0).sqrt_()
    r.mul_(dx.float())
    num = r.sum(-1, dtype=torch.float64).abs()
    den = r.abs().sum(-1, dtype=torch.float64) + fam.alpha * fam.power * dy.float().abs().amax(-1).double()
    return float((num / den.clamp(min=1e-30)).max())


@pytest.mark.parametrize("dtype,L,waves", SPLIT_CASES, ids=SPLIT_IDS)
@pytest.mark.parametrize("fam", FAMILIES, ids=["default", "a1.5t.25p3", "a.75t-.5p1"])
def test_rowwise_split_kernels_match_oracle(dtype, L, waves, fam):
    """Row-wise forward and backward of the split kernels vs the float64
    oracle on a few full rows (the row-wise gradient is autograd of
    softplus_norm_eager, kernels.py:1332-1346)."""
    _check_row_kernel(dtype, L, waves, causal=False)
    x = _randn((6, L), dtype, seed=7 * L + fam.power, scale=128 ** -0.5)
    dy = _randn((6, L), dtype, seed=7 * L + fam.power + 1)
    y = smooth_attn.softplus_norm_triton(x.to(DEV), family=fam)
    assert rel_err(y, eager.softplus_norm_eager(x.double(), fam.alpha, fam.theta, fam.power)) <= REL_TOL[dtype]
    dx = kernels._softplus_norm_backward(x.to(DEV), dy.to(DEV), fam)
    ref = eager.softplus_norm_backward(x.double(), dy.double(), fam.alpha, fam.theta, fam.power, causal=False)
    assert rel_err(dx, ref) <= REL_TOL[dtype]


# rows across the matrix, including both sides of the 1 KB chunk edges (256
# fp32 / 512 bf16 columns) and of the waves' chunk ranges
SAMPLED_CAUSAL_ROWS = [0, 1, 2, 255, 256, 511, 512, 1023, 1024, 2047, 2048, 3000, 4095, 4096, 6000, 8190, 8191]


@pytest.mark.parametrize("dtype,L,waves", SPLIT_CASES, ids=SPLIT_IDS)
@pytest.mark.parametrize("fam", FAMILIES, ids=["default", "a1.5t.25p3", "a.75t-.5p1"])
def test_causal_split_kernels_match_oracle(dtype, L, waves, fam):
    """Causal forward and backward of the split kernels on one [L, L] matrix:
    exact zeros over the whole upper triangle, and oracle parity on sampled
    rows (causal row i is the row-wise function of its prefix x[i, :i+1])."""
    _check_row_kernel(dtype, L, waves, causal=True)
    gen = torch.Generator(device=DEV).manual_seed(L + fam.power)
    x = (torch.randn(1, 1, L, L, generator=gen, device=DEV) * 128 ** -0.5).to(dtype)
    dy = torch.randn(1, 1, L, L, generator=gen, device=DEV).to(dtype)
    y = smooth_attn.softplus_norm_causal_triton(x, family=fam)
    dx = kernels._softplus_norm_causal_backward(x, dy, fam)
    up = torch.triu(torch.ones(L, L, dtype=torch.bool, device=DEV), 1)
    assert int(y[0, 0][up].count_nonzero()) == 0 and int(dx[0, 0][up].count_nonzero()) == 0
    del up
    # size-independent properties of every row: sum_j y_j = 1, and the
    # gradient invariant sum_j dx_j sqrt(a_j^2 + 4) = 0 (masked entries are
    # exact zeros, so whole rows can be summed)
    sums = y[0, 0].sum(-1, dtype=torch.float64)
    assert float((sums - 1).abs().max()) <= (1e-5 if dtype == torch.float32 else 2e-2)
    assert _gradient_invariant(x[0, 0], dy[0, 0], dx[0, 0], fam) <= REL_TOL[dtype]
    # one relative error over all sampled rows, as over whole tensors elsewhere
    # (row 0's exact gradient is O(eps), so a per-row ratio there is noise)
    rows = [i for i in SAMPLED_CAUSAL_ROWS if i < L]
    xs, dys = x[0, 0, rows].cpu().double(), dy[0, 0, rows].cpu().double()
    ref_y = torch.zeros(len(rows), L, dtype=torch.float64)
    ref_dx = torch.zeros(len(rows), L, dtype=torch.float64)
    for n, i in enumerate(rows):
        ref_y[n, :i + 1] = eager.softplus_norm_eager(xs[n, :i + 1], fam.alpha, fam.theta, fam.power)
        ref_dx[n, :i + 1] = eager.softplus_norm_backward(xs[n:n + 1, :i + 1], dys[n:n + 1, :i + 1], fam.alpha,
                                                         fam.theta, fam.power, causal=False)[0]
    assert rel_err(y[0, 0, rows], ref_y) <= REL_TOL[dtype]
    assert rel_err(dx[0, 0, rows], ref_dx) <= REL_TOL[dtype]


@pytest.mark.parametrize("L", [2048, 4096])
def test_full_size_config2_rowwise_fp32(L):
    """Config 2's row-wise fp32 variant at full size, x = randn/sqrt(128)
    and dy = randn, fp32 [64 L, L]: properties over the whole output
    (rows sum to 1; sum_j dx_j sqrt(a_j^2 + 4) = 0 for every row) and the
    float64 oracle at <= 1e-5 on sampled rows."""
    fam = FamilyConfig()
    n = 64 * L
    gen = torch.Generator(device=DEV).manual_seed(40 + L)
    x = torch.randn(n, L, generator=gen, device=DEV) / 128 ** 0.5
    dy = torch.randn(n, L, generator=gen, device=DEV)
    y = smooth_attn.softplus_norm_triton(x, family=fam)
    assert float((y.sum(-1, dtype=torch.float64) - 1).abs().max()) <= 1e-5
    dx = kernels._softplus_norm_backward(x, dy, fam)
    step = n // 8
    for lo in range(0, n, step):  # the row invariant in slices (bounded temporaries)
        sl = slice(lo, lo + step)
        assert _gradient_invariant(x[sl], dy[sl], dx[sl], fam) <= 1e-5, lo
    rows = torch.tensor([0, 1, L - 1, L, n // 2 + 3, n - 2, n - 1] +
                        torch.randint(0, n, (9,), generator=torch.Generator().manual_seed(L)).tolist())
    xs, dys = x[rows.to(DEV)].cpu().double(), dy[rows.to(DEV)].cpu().double()
    assert rel_err(y[rows.to(DEV)], eager.softplus_norm_eager(xs)) <= 1e-5
    assert rel_err(dx[rows.to(DEV)], eager.softplus_norm_backward(xs, dys, causal=False)) <= 1e-5


def test_autograd_module_matches_reference_test():
    # tests/test_training_api.py:63-78 with a seed
    x = _randn((1, 2, 32, 32), torch.bfloat16, seed=11).to(DEV).requires_grad_(True)
    upstream = torch.randn(1, 2, 32, 32, generator=_g(12)).to(DEV)
    y = smooth_attn.SoftplusNormCausal(family=FamilyConfig())(x)
    assert y.shape == x.shape
    (y.float() * upstream).sum().backward()
    xr = x.detach().cpu().double().requires_grad_(True)
    (eager.softplus_norm_causal_eager(xr) * upstream.cpu().double()).sum().backward()
    torch.testing.assert_close(x.grad.cpu().float(), xr.grad.float(), atol=5e-3, rtol=5e-2)
    assert rel_err(x.grad, xr.grad) <= 1e-2


def test_noncontiguous_out_and_input():
    x = _randn((2, 64, 64), torch.bfloat16, seed=21).to(DEV)
    xt = x.transpose(-1, -2)  # non-contiguous input: copied by the wrapper
    out = torch.empty(2, 64, 64, dtype=torch.bfloat16, device=DEV).transpose(-1, -2)  # non-contiguous out
    y = smooth_attn.softplus_norm_causal_triton_out(out, xt)
    assert y is out
    ref = eager.softplus_norm_causal_eager(xt.cpu().double())
    assert rel_err(y, ref) <= 1e-2


def test_row_stride_wider_than_row():
    base = _randn((16, 160), torch.float32, seed=22).to(DEV)
    x = base[:, :96]  # row stride 160, 16-byte aligned rows
    out = torch.zeros(16, 200, device=DEV)
    kernels._norm_fwd_2d(x, out[:, :96], FamilyConfig(), causal=False)
    assert rel_err(out[:, :96], eager.softplus_norm_eager(x.cpu().double())) <= 1e-5
    assert bool((out[:, 96:] == 0).all()), "columns past n_cols must not be written"
    x2 = base[:, 1:97]  # misaligned rows -> element-wise kernel
    kernels._norm_fwd_2d(x2, out[:, :96], FamilyConfig(), causal=True)
    # causal rows of a non-square 2-D view attend to j <= row mod n_cols: the
    # first 16 rows of a 96 x 96 causal matrix
    sq = torch.zeros(96, 96, dtype=torch.float64)
    sq[:16] = x2.cpu().double()
    assert rel_err(out[:, :96], eager.softplus_norm_causal_eager(sq)[:16]) <= 1e-5


def test_masked_scores_above_diagonal_are_ignored():
    L = 128
    x = _randn((1, 4, L, L), torch.bfloat16, seed=23)
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    xm = x.clone()
    xm[..., upper] = float("-inf")
    y = smooth_attn.softplus_norm_causal_triton(xm.to(DEV))
    assert bool(torch.isfinite(y).all())
    assert torch.equal(y.cpu(), smooth_attn.softplus_norm_causal_triton(x.to(DEV)).cpu())
    dy = _randn((1, 4, L, L), torch.bfloat16, seed=24)
    dy[..., upper] = float("nan")
    dx = kernels._softplus_norm_causal_backward(x.to(DEV), dy.to(DEV), FamilyConfig())
    assert bool(torch.isfinite(dx).all())
    assert bool((dx.cpu()[..., upper] == 0).all())


def test_empty_and_limits():
    x = torch.empty(0, 64, dtype=torch.bfloat16, device=DEV)
    assert smooth_attn.softplus_norm_triton(x).shape == (0, 64)
    with pytest.raises(ValueError, match="too large"):
        smooth_attn.softplus_norm_triton(torch.zeros(2, 8200, device=DEV))
    x = _randn((2, 8192), torch.bfloat16, seed=25)
    y = smooth_attn.softplus_norm_triton(x.to(DEV))
    assert rel_err(y, eager.softplus_norm_eager(x.double())) <= 1e-2


@pytest.mark.parametrize("L", [2048, 4096])
def test_full_size_config2_properties(L):
    """config 2 at full size [4,16,L,L]: size-independent properties
    on the whole output, oracle parity on sampled rows."""
    B, H = 4, 16
    gen = torch.Generator(device=DEV).manual_seed(L)
    x = (torch.randn(B, H, L, L, generator=gen, device=DEV) / 128 ** 0.5).to(torch.bfloat16)
    y = smooth_attn.softplus_norm_causal_triton(x)
    sums = y.float().sum(-1)
    assert float((sums - 1).abs().max()) < 2e-2  # bf16 rounding of up to L terms
    up = torch.triu(torch.ones(L, L, dtype=torch.bool, device=DEV), 1)
    assert int(y[0, 0][up].count_nonzero()) == 0 and int(y[-1, -1][up].count_nonzero()) == 0
    rows = [0, 1, L // 2, L - 2, L - 1]
    for b, h in [(0, 0), (B - 1, H - 1), (2, 7)]:
        ref = eager.softplus_norm_causal_eager(x[b, h].cpu().double())
        assert rel_err(y[b, h, rows], ref[rows]) <= 1e-2
    dy = torch.randn(B, H, L, L, generator=gen, device=DEV).to(torch.bfloat16)
    dx = kernels._softplus_norm_causal_backward(x, dy, FamilyConfig())
    assert int(dx[1, 3][up].count_nonzero()) == 0
    for b, h in [(0, 0), (3, 15)]:
        ref = eager.softplus_norm_backward(x[b, h].cpu().double(), dy[b, h].cpu().double(), causal=True)
        assert rel_err(dx[b, h, rows], ref[rows]) <= 1e-2


@pytest.mark.parametrize("dtype,L,kernel,waves", [
    (torch.bfloat16, 4096, "split", 4),   # 8 chunks of 512 -> 4 waves per row
    (torch.bfloat16, 1024, "vec", 1),
    (torch.bfloat16, 100, "scalar", 1),   # 100 % 8 != 0: element loads
    (torch.float32, 2048, "split", 4),
    (torch.float32, 4096, "split", 8),    # 16 chunks of 256 -> 8 waves per row
])
def test_launch_meta_describes_the_kernel(dtype, L, kernel, waves):
    # return_meta carries the reference's keys (kernels.py:310-317, :423-427),
    # filled from the launch this call made and the compiled kernel
    B, H = 1, 2
    x = _randn((B, H, L, L), dtype, seed=L + 5).to(DEV)
    y, meta = smooth_attn.softplus_norm_causal_triton(x, return_meta=True)
    for key in ["variant", "block_size", "num_warps", "num_stages", "num_programs", "occupancy", "n_regs",
                "shared_mem", "time_us"]:
        assert key in meta
    assert meta["variant"] == "squareplus_winner"
    assert meta["kernel"] == kernel and meta["waves_per_row"] == waves
    rows = B * H * L
    assert meta["num_programs"] == -(-rows // meta["rows_per_program"])
    assert meta["num_warps"] * 64 >= 64 * waves
    assert meta["block_size"] >= (L if kernel != "scalar" else 64)
    assert 0 < meta["n_regs"] <= 512 and meta["occupancy"] >= 1
    assert (meta["shared_mem"] > 0) == (kernel == "split")  # split rows combine partial sums in LDS
    assert meta["time_us"] > 0
    # cached per shape: the same dict values on a second call
    _, meta2 = smooth_attn.softplus_norm_causal_triton(x, return_meta=True)
    assert meta2 == meta
    ref = eager.softplus_norm_causal_eager(x[:1, :1].cpu().double())
    assert rel_err(y[:1, :1], ref) <= REL_TOL[dtype]
