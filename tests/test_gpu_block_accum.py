"""GPU parity of the fused block accumulation (a sublayer's fused projection
split, added to the live partial block and, at a block end, turned into the
block source) against the oracle's eager composition on the CPU
(``lrid_block_accumulate_ref``: the split of model.py:363-388, the adds of
model.py:2377-2389 / 2451-2463 and the block source of model.py:990-1028).

Bit-exact where the eager op is one rounding of an fp32 result the kernel
forms the same way (the value add, a python-number scale, the value
gradient); the gpu_util bound where an rms-norm or a token sum enters (keys,
key gradients, value_norm, the learned scale's gradient).
"""

import math

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


def _both(y, pv, pk, D, R, heads, key_norm, g_value, g_key, **kw):
    """HIP on the GPU and the oracle on the CPU, forward and backward.

    ``kw`` may hold ``partial_scale`` as ("tensor", alpha, count): a learned
    alpha whose ``count ** -alpha`` scales the block (a leaf on each side)."""
    sk = kw.pop("partial_scale", 1.0)
    a_h = a_c = None
    if isinstance(sk, tuple):
        _, alpha, count = sk
        a_h = torch.tensor(alpha, device=DEV, requires_grad=True)
        a_c = torch.tensor(alpha, requires_grad=True)
        s_h, s_c = O.block_count_scale(count, a_h), O.block_count_scale(count, a_c)
    else:
        s_h = s_c = sk
    leaves_h = [t.to(DEV).requires_grad_(True) if t is not None else None for t in (y, pv, pk)]
    leaves_c = [t.clone().requires_grad_(True) if t is not None else None for t in (y, pv, pk)]
    v, k = ops.lrid_block_accumulate(leaves_h[0], leaves_h[1], leaves_h[2], D, R, heads, key_norm,
                                     partial_scale=s_h, **kw)
    ev, ek = O.lrid_block_accumulate_ref(leaves_c[0], leaves_c[1], leaves_c[2], D, R, heads, key_norm,
                                         partial_scale=s_c, **kw)
    outs_h, outs_c = [], []
    if g_value is not None:
        outs_h.append((v, g_value.to(DEV)))
        outs_c.append((ev, g_value))
    if g_key is not None:
        outs_h.append((k, g_key.to(DEV)))
        outs_c.append((ek, g_key))
    torch.autograd.backward([t for t, _ in outs_h], [g for _, g in outs_h])
    torch.autograd.backward([t for t, _ in outs_c], [g for _, g in outs_c])
    grads = [(h.grad if h is not None else None, c.grad if c is not None else None)
             for h, c in zip(leaves_h, leaves_c)]
    if a_h is not None:
        grads.append((a_h.grad, a_c.grad))
    return (v, ev), (k, ek), grads


SHAPES = [
    (768, 64, 64, 1, True),     # the whole-model configuration (16-bit: three columns of 8-byte vectors)
    (256, 32, 32, 2, True),     # 16-bit: one column of 8-byte vectors
    (1024, 64, 64, 4, True),    # per-head norm
    (2048, 128, 128, 1, True),  # 128-column head
    (768, 32, 48, 1, False),    # padding columns, no key norm
    (100, 24, 24, 3, True),     # unaligned rows (scalar path)
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,R,P,heads,key_norm", SHAPES)
@pytest.mark.parametrize("first", [False, True])
def test_accumulate_matches_oracle(dtype, D, R, P, heads, key_norm, first):
    """partial' = partial + out, partial_key' = partial_key + key (first: no partial yet)."""
    g = gen(D + 3 * R + heads + first)
    B, T = 2, 37
    y = randn(g, (B, T, D + P), dtype)
    pv = None if first else randn(g, (B, T, D), dtype)
    pk = None if first else randn(g, (B, T, R), dtype)
    gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    (v, ev), (k, ek), grads = _both(y, pv, pk, D, R, heads, key_norm, gv, gk)
    assert torch.equal(v.cpu(), ev.detach())
    assert_close(k, ek, dtype, "key")
    (dy, e_dy), (dpv, e_dpv), (dpk, e_dpk) = grads
    assert torch.equal(dy[..., :D].cpu(), e_dy[..., :D])
    assert_close(dy[..., D:D + R], e_dy[..., D:D + R], dtype, "dkey")
    if P > R:
        assert float(dy[..., D + R:].abs().max()) == 0.0
    if not first:
        assert torch.equal(dpv.cpu(), e_dpv)
        assert torch.equal(dpk.cpu(), e_dpk)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("key_norm", [True, False])
@pytest.mark.parametrize("scale_key", [False, True])
@pytest.mark.parametrize("first", [False, True])
def test_complete_with_count_scale(dtype, key_norm, scale_key, first):
    """Block end, value * count**-alpha (a python number); the key scaled too
    with scale_key (the model's rule for keys without rms-norm)."""
    g = gen(11 + 2 * key_norm + scale_key + 4 * first)
    B, T, D, R = 2, 33, 768, 64
    y = randn(g, (B, T, D + R), dtype)
    pv = None if first else randn(g, (B, T, D), dtype)
    pk = None if first else randn(g, (B, T, R), dtype)
    gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    s = 3.0 ** -0.5
    (v, ev), (k, ek), grads = _both(y, pv, pk, D, R, 1, key_norm, gv, gk, complete=True, partial_scale=s,
                                    scale_key=scale_key)
    assert torch.equal(v.cpu(), ev.detach())
    assert_close(k, ek, dtype, "key")
    (dy, e_dy), (dpv, e_dpv), (dpk, e_dpk) = grads
    assert torch.equal(dy[..., :D].cpu(), e_dy[..., :D])
    assert_close(dy[..., D:], e_dy[..., D:], dtype, "dkey")
    if not first:
        assert torch.equal(dpv.cpu(), e_dpv)
        assert torch.equal(dpk.cpu(), e_dpk)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale_key", [False, True])
def test_complete_with_learned_scale(dtype, scale_key):
    """A learned alpha: the scale tensor takes the value dtype before it scales
    (model.py:983-985, 1016-1018), and its gradient is a token sum of the
    rounded products (value side, plus key side with scale_key)."""
    g = gen(21 + scale_key)
    B, T, D, R = 4, 300, 768, 64
    y = randn(g, (B, T, D + R), dtype)
    pv, pk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    (v, ev), (k, ek), grads = _both(y, pv, pk, D, R, 1, False, gv, gk, complete=True,
                                    partial_scale=("tensor", 0.7, 3), scale_key=scale_key)
    assert_close(v, ev, dtype, "value")
    assert_close(k, ek, dtype, "key")
    (dy, e_dy), (dpv, e_dpv), (dpk, e_dpk), (da, e_da) = grads
    assert_close(dy, e_dy, dtype, "dy")
    assert_close(dpv, e_dpv, dtype, "dpartial")
    assert_close(dpk, e_dpk, dtype, "dpartial_key")
    if dtype == torch.float32:
        assert_close(da.reshape(1), e_da.reshape(1), dtype, "dalpha", reduced=True)
    else:
        # the scale's gradient is a token sum rounded to the dtype on both sides (the
        # reference's scale is a dtype tensor): summation order may move it by one
        # ulp, which the fp32 chain rule to alpha carries over as a relative error
        mant = 7 if dtype == torch.bfloat16 else 10
        a, e = float(da), float(e_da)
        assert abs(a - e) <= 2.0 ** -mant * abs(e) * (1 + 1e-5), (a, e)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [768, 100])
def test_complete_with_value_norm(dtype, D):
    """Block end with value_norm: rms_norm(partial + out), the key unscaled."""
    g = gen(31 + D)
    B, T, R = 2, 41, 24
    y = randn(g, (B, T, D + R), dtype)
    pv, pk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    (v, ev), (k, ek), grads = _both(y, pv, pk, D, R, 3, True, gv, gk, complete=True, value_norm=True)
    assert_close(v, ev, dtype, "value")
    assert_close(k, ek, dtype, "key")
    (dy, e_dy), (dpv, e_dpv), (dpk, e_dpk) = grads
    assert_close(dy, e_dy, dtype, "dy")
    assert_close(dpv, e_dpv, dtype, "dpartial")
    assert torch.equal(dpk.cpu(), e_dpk)


@pytest.mark.parametrize("which", ["value", "key"])
@pytest.mark.parametrize("value_norm", [False, True])
def test_one_sided_gradient(which, value_norm):
    g = gen(41 + value_norm)
    B, T, D, R = 1, 50, 768, 64
    dtype = torch.bfloat16
    y = randn(g, (B, T, D + R), dtype)
    pv, pk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    gv = randn(g, (B, T, D), dtype) if which == "value" else None
    gk = randn(g, (B, T, R), dtype) if which == "key" else None
    kw = dict(value_norm=True) if value_norm else dict(partial_scale=0.5, scale_key=True)
    _, _, grads = _both(y, pv, pk, D, R, 1, value_norm, gv, gk, complete=True, **kw)
    (dy, e_dy), (dpv, e_dpv), (dpk, e_dpk) = grads
    assert_close(dy, e_dy, dtype, "dy")
    if which == "value":
        assert_close(dpv, e_dpv, dtype, "dpartial")
        assert dpk is None and e_dpk is None
    else:
        assert dpv is None and e_dpv is None
        assert_close(dpk, e_dpk, dtype, "dpartial_key")


def test_strided_value_gradient():
    """The value's incoming gradient as a row-strided view (a cat downstream)."""
    g = gen(51)
    B, T, D, R = 2, 64, 768, 64
    dtype = torch.bfloat16
    y = randn(g, (B, T, D + R), dtype)
    pv, pk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    gc = randn(g, (B, T, D + R), dtype)
    yh, pvh, pkh = (t.to(DEV).requires_grad_(True) for t in (y, pv, pk))
    v, k = ops.lrid_block_accumulate(yh, pvh, pkh, D, R, 1, True, complete=True, partial_scale=0.5)
    torch.cat([v, k], -1).backward(gc.to(DEV))
    yc, pvc, pkc = (t.clone().requires_grad_(True) for t in (y, pv, pk))
    ev, ek = O.lrid_block_accumulate_ref(yc, pvc, pkc, D, R, 1, True, complete=True, partial_scale=0.5)
    torch.cat([ev, ek], -1).backward(gc)
    assert torch.equal(yh.grad[..., :D].cpu(), yc.grad[..., :D])
    assert_close(yh.grad, yc.grad, dtype, "dy")
    assert torch.equal(pvh.grad.cpu(), pvc.grad)
    assert torch.equal(pkh.grad.cpu(), pkc.grad)


def test_a_whole_block_matches_the_eager_sublayer_chain():
    """Two sublayers of a block at a model-sized shape (B4 T1024 d768 r64): the
    first starts the partial block, the second completes it with count**-alpha;
    gradients reach both projections and match the eager chain."""
    g = gen(61)
    B, T, D, R = 4, 1024, 768, 64
    dtype = torch.bfloat16
    ys = [randn(g, (B, T, D + R), dtype) for _ in range(2)]
    gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    s = 2.0 ** -1.0
    yh = [t.to(DEV).requires_grad_(True) for t in ys]
    pv, pk = ops.lrid_block_accumulate(yh[0], None, None, D, R, 1, True)
    v, k = ops.lrid_block_accumulate(yh[1], pv, pk, D, R, 1, True, complete=True, partial_scale=s)
    torch.autograd.backward([v, k], [gv.to(DEV), gk.to(DEV)])
    yc = [t.clone().requires_grad_(True) for t in ys]
    epv, epk = O.lrid_block_accumulate_ref(yc[0], None, None, D, R, 1, True)
    ev, ek = O.lrid_block_accumulate_ref(yc[1], epv, epk, D, R, 1, True, complete=True, partial_scale=s)
    torch.autograd.backward([ev, ek], [gv, gk])
    assert torch.equal(v.cpu(), ev.detach())
    assert_close(k, ek, dtype, "key")
    for i in range(2):
        assert torch.equal(yh[i].grad[..., :D].cpu(), yc[i].grad[..., :D]), i
        assert_close(yh[i].grad, yc[i].grad, dtype, f"dy{i}")
    assert math.isfinite(float(v.float().abs().max()))
