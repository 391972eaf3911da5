"""HIP-graph capture of the read ops (torch.cuda.CUDAGraph drives hipGraph on ROCm).

A caller that captures its training step (the reference's published
whole-model numbers are CUDA-graph runs) records these ops' kernel launches
once and replays them.  Each test captures forward + backward, then before
every replay changes the captured inputs in place with eager kernels and
synchronises; every replay must equal an eager run on the same inputs
exactly (same kernels, same launch geometry, deterministic reductions).
The captured regions hold only this library's kernels and element-wise
torch work: no multi-block torch reductions, whose internal memset nodes are
not replay-safe on this platform.
"""

import pytest
import torch

import attnres_ops as ops
from gpu_util import DEV, gen, randn

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _capture(fn):
    """Warm up on a side stream, then capture fn() and return (graph, static outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    torch.cuda.synchronize()
    return graph, outs


def _check_replays(fn, inputs, replays=3):
    graph, static = _capture(fn)
    for i in range(replays):
        with torch.no_grad():
            for t in inputs:  # eager work between replays: new input values
                t.mul_(-0.75 if i % 2 else 1.25).add_(0.125)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static]
        want = fn()
        torch.cuda.synchronize()
        assert len(got) == len(want)
        for k, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {i}: output {k} differs from the eager run"


def test_lr_read_graph_replays_match_eager():
    g = gen(41)
    B, T, D, S, R, H = 2, 48, 1024, 7, 64, 4
    dt = torch.bfloat16
    vals = [randn(g, (B, T, D), dt).to(DEV).requires_grad_(True) for _ in range(S)]
    keys = [randn(g, (B, T, R), dt).to(DEV).requires_grad_(True) for _ in range(S)]
    q = randn(g, (H, R // H), torch.float32, 0.5).to(DEV).requires_grad_(True)
    up = randn(g, (B, T, D), dt).to(DEV)

    def fn():
        out = ops.lrid_attention_residual_read(vals, keys, q, H, 0.25, True, source_counts=[1.0] * (S - 1) + [2.0])
        grads = torch.autograd.grad(out, [*vals, *keys, q], up)
        return [out.detach(), *grads]

    _check_replays(fn, [*vals, *keys, q, up])


@pytest.mark.parametrize("normalize_output", [True, False])  # False: the one-wave packed kernels
def test_base_read_graph_replays_match_eager(normalize_output):
    g = gen(42)
    B, T, D, S = 2, 40, 768, 5
    dt = torch.bfloat16
    vals = [randn(g, (B, T, D), dt).to(DEV).requires_grad_(True) for _ in range(S)]
    q = randn(g, (D,), torch.float32, 0.05).to(DEV).requires_grad_(True)
    up = randn(g, (B, T, D), dt).to(DEV)

    def fn():
        out = ops.attention_residual_read(vals, q, True, normalize_output=normalize_output)
        grads = torch.autograd.grad(out, [*vals, q], up)
        return [out.detach(), *grads]

    _check_replays(fn, [*vals, q, up])


def test_phase_schedule_graph_replays_match_eager():
    g = gen(43)
    B, T, D, S, Q = 2, 32, 768, 4, 3
    dt = torch.bfloat16
    vals = [randn(g, (B, T, D), dt).to(DEV).requires_grad_(True) for _ in range(S)]
    logits = randn(g, (Q, S, B, T), torch.float32, 2.0).to(DEV).requires_grad_(True)
    partial = randn(g, (B, T, D), dt).to(DEV).requires_grad_(True)
    q = randn(g, (D,), dt, 0.05).to(DEV).requires_grad_(True)
    up = randn(g, (B, T, D), dt).to(DEV)
    g_outs = randn(g, (Q, B, T, D), dt).to(DEV)
    g_lse = randn(g, (Q, B, T), torch.float32).to(DEV)

    def fn():
        # upstream gradients are given tensors: the captured region holds only
        # this library's kernels and element-wise gradient accumulation
        outs, lse = ops.attention_residual_phase1_from_logits(vals, logits)
        merged = ops.attention_residual_phase2(partial, q, outs[1], lse[1], True)
        grads = torch.autograd.grad([merged, outs, lse], [*vals, logits, partial, q], [up, g_outs, g_lse])
        return [merged.detach(), *grads]

    _check_replays(fn, [*vals, logits, partial, q, up, g_outs, g_lse])


def test_accumulate_read_graph_replays_match_eager():
    """The fused accumulate-and-read in a captured fwd+bwd, as the graphed
    decoder step runs it: the op's backward reads the forward's descriptor
    from ctx, whose tensors live on as saved tensors only."""
    g = gen(47)
    B, T, D, R, rows = 2, 40, 768, 64, 5
    dt = torch.bfloat16
    y = randn(g, (B, T, D + R), dt).to(DEV).requires_grad_(True)
    pv = randn(g, (B, T, D), dt).to(DEV).requires_grad_(True)
    pk = randn(g, (B, T, R), dt).to(DEV).requires_grad_(True)
    bank = randn(g, (rows, R), dt, 0.1).to(DEV).requires_grad_(True)
    inter = randn(g, (B, T, D), dt).to(DEV).requires_grad_(True)
    lse = randn(g, (B, T), torch.float32).to(DEV).requires_grad_(True)
    go, gv, gk = randn(g, (B, T, D), dt).to(DEV), randn(g, (B, T, D), dt).to(DEV), randn(g, (B, T, R), dt).to(DEV)

    def fn():
        v, k, o = ops.lrid_block_accumulate_read(y, pv, pk, bank, inter, lse, D, R, 0.125, 1, True, lerp=True,
                                                 normalize_output=True, logit_bias=0.4, partial_scale=0.5,
                                                 query_row=2)
        grads = torch.autograd.grad([o, v, k], [y, pv, pk, bank, inter, lse], [go, gv, gk])
        return [v.detach(), k.detach(), o.detach(), *grads]

    _check_replays(fn, [y, pv, pk, bank, inter, lse, go, gv, gk])
