"""The training step's forward and backward captured in a HIP graph (GPU).

The library allocates no device memory and synchronises with nothing: every
launch goes to the caller's stream, and the backward's workspace is a torch
allocation made by the Python wrapper.  So the whole autograd step of the
causal norm and of fused attention (including the dK/dV split, whose fp32
partials live in that workspace, and GQA with a window) can be captured with
torch.cuda.graph and replayed.  Each replay runs on fresh inputs copied into
the captured tensors, with eager calls of the same entry points and a
synchronisation between replays, and must equal the eager step on the same
inputs bit for bit (every kernel here is deterministic).
"""
import pytest
import torch

import smooth_attn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(step, inputs, grad_out):
    """Warm the step up on a side stream, then capture it; returns the graph
    and its output tensors."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(inputs, grad_out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(inputs, grad_out)
    return graph, outs


def _replay_matches_eager(step, inputs, grad_out, make, n_replays=3):
    graph, outs = _capture(step, inputs, grad_out)
    for i in range(n_replays):
        fresh, fresh_go = make(100 + i)
        with torch.no_grad():
            for dst, src in zip(inputs, fresh):
                dst.copy_(src)
            grad_out.copy_(fresh_go)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        # eager step on the same values (new tensors), between the replays
        want = step([t.detach().clone().requires_grad_(True) for t in fresh], fresh_go.clone())
        torch.cuda.synchronize()
        for j, (g, w) in enumerate(zip(got, want)):
            assert torch.equal(g, w), (i, j)


def test_norm_step_replays():
    def make(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        x = torch.randn(2, 4, 300, 300, generator=g, device=DEV).to(torch.bfloat16)
        return [x], torch.randn(2, 4, 300, 300, generator=g, device=DEV).to(torch.bfloat16)

    def step(inputs, go):
        (x,) = inputs
        y = smooth_attn.softplus_norm_causal(x)
        (dx,) = torch.autograd.grad(y, (x,), go)
        return [y.detach(), dx]

    fresh, go = make(1)
    _replay_matches_eager(step, [fresh[0].requires_grad_(True)], go, make)


@pytest.mark.parametrize("shape,window", [
    ((2, 8, 2, 300, 128), 0),     # GQA 4:1, ragged T
    ((1, 4, 1, 2048, 64), 0),     # one (batch, KV head) pair: dK/dV split over the query tiles
    ((2, 4, 2, 500, 128), 100),   # sliding window
])
def test_attention_step_replays(shape, window):
    B, Hq, Hkv, T, D = shape

    def make(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        q = torch.randn(B, Hq, T, D, generator=g, device=DEV).to(torch.bfloat16)
        k = torch.randn(B, Hkv, T, D, generator=g, device=DEV).to(torch.bfloat16)
        v = torch.randn(B, Hkv, T, D, generator=g, device=DEV).to(torch.bfloat16)
        return [q, k, v], torch.randn(B, Hq, T, D, generator=g, device=DEV).to(torch.bfloat16)

    def step(inputs, go):
        q, k, v = inputs
        o = smooth_attn.sp2norm_flash_attention(q, k, v, window_size=window)
        dq, dk, dv = torch.autograd.grad(o, (q, k, v), go)
        return [o.detach(), dq, dk, dv]

    fresh, go = make(1)
    _replay_matches_eager(step, [t.requires_grad_(True) for t in fresh], go, make)
