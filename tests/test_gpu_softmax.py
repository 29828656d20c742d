"""Parity of the softmax comparison kernels (HIP) with the CPU oracle, and a
run of the benchmark command line (GPU).

Tolerances: max|HIP - oracle| / max|oracle| <= 1e-5 for fp32 outputs,
<= 1e-2 for bf16 / fp16 outputs (oracle in float64 on the same inputs);
causal zeros exact; the reference suite's row-sum checks (atol 1e-4 fp32,
5e-3 otherwise, kernels.py:2900-2915).
"""
import pytest
import torch

import smooth_attn
from oracle import eager

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


def tol(dtype):
    return 1e-5 if dtype == torch.float32 else 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 33), (64, 256), (300, 1000), (32, 2048), (8, 4096), (4, 8192)])
def test_rowwise_softmax(dtype, rows, cols):
    x = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(rows + cols)) * 3).to(dtype)
    y = smooth_attn.softmax_triton(x.to(DEV))
    ref = eager.softmax_eager(x.double())
    assert y.dtype == dtype and y.shape == x.shape
    assert rel_err(y, ref) <= tol(dtype)
    out = torch.empty_like(y)
    y2, meta = smooth_attn.softmax_triton_out(out, x.to(DEV), return_meta=True)
    assert y2 is out and torch.equal(y2, y) and meta["variant"] == "softmax"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("L", [1, 17, 128, 200, 1024])
def test_causal_softmax(dtype, L):
    x = torch.randn(2, 3, L, L, generator=torch.Generator().manual_seed(L)).to(dtype)
    y = smooth_attn.softmax_causal_triton(x.to(DEV))
    ref = eager.softmax_causal_eager(x.double())
    assert rel_err(y, ref) <= tol(dtype)
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((y.cpu()[..., upper] == 0).all())
    atol = 1e-4 if dtype == torch.float32 else 5e-3
    assert torch.allclose(y.float().sum(-1).cpu(), torch.ones(2, 3, L), atol=atol)


@pytest.mark.parametrize("dtype,L,kernel", [
    (torch.float32, 2048, "vec"), (torch.bfloat16, 2048, "vec"), (torch.bfloat16, 4096, "vec"),
    (torch.float32, 4096, "split"), (torch.bfloat16, 8192, "split"), (torch.float16, 8192, "split"),
])
def test_causal_softmax_long_rows(dtype, L, kernel):
    # rows of 16 or more 1 KB chunks (fp32 L >= 4096, 16-bit L = 8192) run 8
    # waves per row, one row per block; causal rows leave whole waves without
    # a visible chunk.  Shorter rows keep one wave per row.
    x = torch.randn(1, 1, L, L, generator=torch.Generator().manual_seed(L + 1)).to(dtype)
    y, meta = smooth_attn.softmax_causal_triton(x.to(DEV), return_meta=True)
    assert meta["kernel"] == kernel and meta["waves_per_row"] == (8 if kernel == "split" else 1)
    ref = eager.softmax_causal_eager(x.double())
    assert rel_err(y, ref) <= tol(dtype)
    upper = torch.triu(torch.ones(L, L, dtype=torch.bool), 1)
    assert bool((y.cpu()[..., upper] == 0).all())
    atol = 1e-4 if dtype == torch.float32 else 5e-3
    assert torch.allclose(y.float().sum(-1).cpu(), torch.ones(1, 1, L), atol=atol)


def test_softmax_large_values_and_unaligned_rows():
    # |x| up to 200: exp without the max shift would overflow fp32
    x = torch.linspace(-200, 200, 3 * 77).reshape(3, 77)
    y = smooth_attn.softmax_triton(x.to(DEV))
    assert bool(torch.isfinite(y).all())
    assert rel_err(y, eager.softmax_eager(x.double())) <= 1e-5
    # a column slice: rows not 16-byte aligned -> element-strided kernel
    base = torch.randn(50, 131, generator=torch.Generator().manual_seed(3))
    xs = base[:, 1:]
    ys = smooth_attn.softmax_triton(xs.to(DEV))
    assert rel_err(ys, eager.softmax_eager(xs.double())) <= 1e-5
    xc = torch.randn(1, 2, 40, 40, generator=torch.Generator().manual_seed(4)).bfloat16()
    yc = smooth_attn.softmax_causal_triton(xc.to(DEV).transpose(-1, -2).contiguous().transpose(-1, -2))
    assert rel_err(yc, eager.softmax_causal_eager(xc.double())) <= 1e-2


def test_benchmark_cli_quick(capsys):
    # the reference's command line (kernels.py:3078-3128) with a small sweep:
    # every column runs, HIP launches are reported against the HBM roofline,
    # errors, row sums and the backward check come out right
    smooth_attn.main(["--mode", "all", "--quick", "--dtypes", "fp32,bf16", "--lengths", "64,128",
                      "--warmup", "2", "--iters", "3", "--check-backward"])
    text = capsys.readouterr().out
    assert "row-wise fp32" in text and "squareplus family vs torch softmax: geometric mean" in text
    assert text.count("%") >= 2 * 24  # two HIP columns per row-wise shape report a fraction of peak
    assert "fp32: squareplus family vs torch softmax" in text and "bf16: squareplus family vs torch softmax" in text
    assert " NO " not in text and "close: NO" not in text
    assert text.count("close: yes") == 2
    res = smooth_attn.benchmark_causal_suite(smooth_attn.DEFAULT_FAMILY, [torch.bfloat16], [96], warmup=1, iters=2)
    assert res[0].softmax_sums_ok and res[0].family_sums_ok and res[0].softmax_err < 1e-2
    assert res[0].family_meta["kernel"] in ("vec", "scalar", "split")
    rows = smooth_attn.benchmark_rowwise_suite(smooth_attn.DEFAULT_FAMILY, shapes=[(64, 256)], warmup=1, iters=2)
    assert rows[0].shape == (64, 256) and rows[0].family_us > 0 and rows[0].torch_softmax_us > 0
    grads = smooth_attn.kernels.validate_causal_backward(smooth_attn.DEFAULT_FAMILY, [torch.float32], seq_len=32)
    assert grads[0]["grad_close"] and grads[0]["max_abs_grad_err"] < 1e-4
