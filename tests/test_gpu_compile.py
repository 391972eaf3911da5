"""torch.compile over the drop-in ops (the reference registers its reads as
torch.library ops so that compiled models keep them as single nodes).

Eager calls run through autograd Functions; while torch.compile traces, the
``attnres_hip::`` library ops with their fake implementations are used.  The
``aot_eager`` backend traces forward and backward through AOTAutograd with
fake tensors and then runs the captured graph eagerly, so these tests check
the library-op path (schemas, fake shapes, autograd registration) without any
code generation; results must equal the eager calls exactly.
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


def _grads(fn, inputs, up):
    for t in inputs:
        t.grad = None
    out = fn(*inputs)
    out.backward(up)
    torch.cuda.synchronize()
    return [out.detach().clone()] + [t.grad.clone() for t in inputs]


def _compare(fn, inputs, up):
    torch._dynamo.reset()
    want = _grads(fn, inputs, up)
    got = _grads(torch.compile(fn, backend="aot_eager", fullgraph=True), inputs, up)
    for k, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"compiled result {k} differs from eager"


def test_compiled_lr_read_matches_eager():
    g = gen(51)
    B, T, D, S, R, H = 2, 24, 512, 5, 32, 2
    vals = [randn(g, (B, T, D), torch.bfloat16).to(DEV).requires_grad_(True) for _ in range(S)]
    keys = [randn(g, (B, T, R), torch.bfloat16).to(DEV).requires_grad_(True) for _ in range(S)]
    q = randn(g, (H, R // H), torch.float32, 0.5).to(DEV).requires_grad_(True)
    up = randn(g, (B, T, D), torch.bfloat16).to(DEV)

    def fn(*t):
        return ops.lrid_attention_residual_read(list(t[:S]), list(t[S:2 * S]), t[-1], H, 0.25, True)

    _compare(fn, [*vals, *keys, q], up)


def test_compiled_lr_read_with_static_keys_matches_eager():
    g = gen(53)
    B, T, D, S, R, H = 2, 24, 512, 5, 32, 2
    vals = [randn(g, (B, T, D), torch.bfloat16).to(DEV).requires_grad_(True) for _ in range(S)]
    keys = [randn(g, (B, T, R), torch.bfloat16).to(DEV).requires_grad_(True) for _ in range(S)]
    sk = randn(g, (S, R), torch.float32, 0.1).to(DEV).requires_grad_(True)
    q = randn(g, (H, R // H), torch.float32, 0.5).to(DEV).requires_grad_(True)
    up = randn(g, (B, T, D), torch.bfloat16).to(DEV)

    def fn(*t):
        return ops.lrid_attention_residual_read(list(t[:S]), list(t[S:2 * S]), t[-1], H, 0.25, False,
                                                static_keys=t[-2])

    _compare(fn, [*vals, *keys, sk, q], up)


def test_compiled_phase_schedule_matches_eager():
    g = gen(52)
    B, T, D, S = 2, 16, 256, 3
    vals = [randn(g, (B, T, D), torch.bfloat16).to(DEV).requires_grad_(True) for _ in range(S)]
    logits = randn(g, (2, S, B, T), torch.float32, 2.0).to(DEV).requires_grad_(True)
    partial = randn(g, (B, T, D), torch.bfloat16).to(DEV).requires_grad_(True)
    q = randn(g, (D,), torch.bfloat16, 0.05).to(DEV).requires_grad_(True)
    up = randn(g, (B, T, D), torch.bfloat16).to(DEV)

    def fn(*t):
        outs, lse = ops.attention_residual_phase1_from_logits(list(t[:S]), t[S])
        return ops.attention_residual_phase2(t[S + 1], t[S + 2], outs[0], lse[0], True) + outs[1]

    _compare(fn, [*vals, logits, partial, q], up)
