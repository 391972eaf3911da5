"""GPU parity of the key-producer epilogue (split of the fused [out | key | pad]
projection, model.py:363-388 with the per-head key norm of model.py:34-37)
against the oracle's eager slice / contiguous / rms-norm form on the CPU.

Forward: the output columns are a copy (bit-exact); the key is one rounding
of an fp32 rms-norm (the gpu_util bound).  Backward: the projection gradient
is grad_out in the output columns (bit-exact), the rms-norm backward of
grad_key in the key columns (the bound) and zero in the padding columns.
"""

import pytest
import torch

import _attnres_hip as H
import attnres_ops as ops
from oracle import attnres_oracle as O
from gpu_util import DEV, assert_close, gen, randn

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


def _split_both(y, D, R, heads, key_norm, g_out, g_key):
    """HIP on the GPU and the oracle on the CPU; returns (out, key, dy) pairs."""
    yh = y.to(DEV).requires_grad_(True)
    out, key = ops.lrid_fused_projection_split(yh, D, R, heads, key_norm)
    yc = y.clone().requires_grad_(True)
    e_out, e_key = O.lrid_fused_projection_split_ref(yc, D, R, heads, key_norm)
    if g_out is not None:
        e_out.backward(g_out, retain_graph=g_key is not None)
    if g_key is not None:
        e_key.backward(g_key)
    if g_out is None and g_key is None:
        return (out, e_out), (key, e_key), (None, None)
    hip_g = []
    if g_out is not None:
        hip_g.append((out, g_out.to(DEV)))
    if g_key is not None:
        hip_g.append((key, g_key.to(DEV)))
    torch.autograd.backward([t for t, _ in hip_g], [g for _, g in hip_g])
    return (out, e_out), (key, e_key), (yh.grad, yc.grad)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,R,P,heads,key_norm", [
    (768, 64, 64, 1, True),     # the whole-model configuration
    (1024, 64, 64, 4, True),    # per-head norm, 16 columns per head
    (2048, 128, 128, 1, True),  # 128-column head: two 64-lane chunks
    (512, 256, 256, 2, True),   # two 128-column heads
    (768, 32, 48, 1, True),     # projection rank above the key rank: padding columns
    (768, 64, 64, 1, False),    # no key norm
    (100, 24, 24, 3, True),     # unaligned rows (scalar path), 8-column heads
])
def test_keyed_split_matches_oracle(dtype, D, R, P, heads, key_norm):
    g = gen(D * 7 + R + heads)
    B, T = 2, 37
    y = randn(g, (B, T, D + P), dtype)
    go = randn(g, (B, T, D), dtype)
    gk = randn(g, (B, T, R), dtype)
    (out, e_out), (key, e_key), (dy, e_dy) = _split_both(y, D, R, heads, key_norm, go, gk)
    assert torch.equal(out.cpu(), e_out)
    assert_close(key, e_key, dtype, "key")
    assert torch.equal(dy[..., :D].cpu(), e_dy[..., :D])
    assert_close(dy[..., D:D + R], e_dy[..., D:D + R], dtype, "dkey")
    if P > R:
        assert float(dy[..., D + R:].abs().max()) == 0.0


@pytest.mark.parametrize("which", ["out", "key"])
def test_keyed_split_one_sided_gradient(which):
    g = gen(3)
    B, T, D, R = 1, 50, 768, 64
    y = randn(g, (B, T, D + R), torch.bfloat16)
    go = randn(g, (B, T, D), torch.bfloat16) if which == "out" else None
    gk = randn(g, (B, T, R), torch.bfloat16) if which == "key" else None
    (_, _), (_, _), (dy, e_dy) = _split_both(y, D, R, 1, True, go, gk)
    if which == "out":
        assert torch.equal(dy[..., :D].cpu(), e_dy[..., :D])
        assert float(dy[..., D:].abs().max()) == 0.0
    else:
        assert float(dy[..., :D].abs().max()) == 0.0
        assert_close(dy[..., D:], e_dy[..., D:], torch.bfloat16, "dkey")


def test_keyed_split_strided_projection_and_model_size():
    """A projection that is a column slice of a wider buffer (rows 896 apart),
    at the whole-model token count (B16 T1024)."""
    g = gen(9)
    B, T, D, R = 16, 1024, 768, 64
    wide = randn(g, (B, T, D + R + 64), torch.bfloat16)
    y = wide[..., :D + R]
    yh = wide.to(DEV)[..., :D + R]
    out, key = ops.lrid_fused_projection_split(yh, D, R, 1, True)
    e_out, e_key = O.lrid_fused_projection_split_ref(y, D, R, 1, True)
    assert torch.equal(out.cpu(), e_out)
    assert_close(key, e_key, torch.bfloat16, "key")


def test_keyed_split_key_is_unit_rms():
    g = gen(4)
    y = randn(g, (3, 5, 256 + 128), torch.float32, 3.0).to(DEV)
    _, key = ops.lrid_fused_projection_split(y, 256, 128, 4, True)
    rms = key.reshape(3, 5, 4, 32).pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-5)


def test_keyed_split_empty():
    y = torch.empty(0, 4, 832, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    out, key = ops.lrid_fused_projection_split(y, 768, 64)
    assert out.shape == (0, 4, 768) and key.shape == (0, 4, 64)
    (out.sum() + key.sum()).backward()
    assert y.grad.shape == y.shape
