"""GPU parity of the LR read with per-source static keys fused in (config 4's
[N, R] static source key; the model adds it eagerly, model.py:2046-2049)
against the oracle's read of the summed keys, on the CPU: output, value and
key gradients, the query / gate gradients and the static keys' gradient (the
token sum of the key gradient, rounded to the key dtype once).

Covers the fast kernels (the static-key instantiations with a static query,
with a gated per-token query at config 4's shape, and with the output norm)
and the general kernel (unaligned rows), fp32 and bf16, key norm on and off.
"""

import pytest
import torch

import _attnres_hip as H
import attnres_ops as ops
from oracle import attnres_oracle as O
from gpu_util import DEV, assert_close, gen, leaf, randn

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


def _case(seed, B, T, D, S, R, Hh, dtype):
    g = gen(seed)
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    keys = [randn(g, (B, T, R), dtype) for _ in range(S)]
    sk = randn(g, (S, R), torch.float32, 0.02 if dtype != torch.float32 else 0.5)
    up = randn(g, (B, T, D), dtype)
    return g, vals, keys, sk, up


def _ref(vals, keys, sk, read):
    vc = [x.clone().requires_grad_(True) for x in vals]
    kc = [x.clone().requires_grad_(True) for x in keys]
    skc = sk.clone().requires_grad_(True)
    out = read(vc, O.static_key_add_ref(kc, skc))
    return out, vc, kc, skc


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("key_norm", [True, False])
@pytest.mark.parametrize("shape", [
    (2, 64, 1024, 13, 64, 4),   # C3's rows: fast kernels, static query
    (1, 70, 102, 5, 24, 3),     # unaligned rows: general kernel
])
def test_static_query_read_with_static_keys(dtype, key_norm, shape):
    B, T, D, S, R, Hh = shape
    g, vals, keys, sk, up = _case(11 + S + key_norm, B, T, D, S, R, Hh, dtype)
    q = randn(g, (Hh, R // Hh), dtype, 0.5)
    vd, kd, qd, skd = [leaf(x) for x in vals], [leaf(x) for x in keys], leaf(q), leaf(sk)
    out = ops.lrid_attention_residual_read(vd, kd, qd, Hh, 0.25, key_norm, static_keys=skd)
    out.backward(up.to(DEV))
    qc = q.clone().requires_grad_(True)
    ref, vc, kc, skc = _ref(vals, keys, sk, lambda v, k: O.lrid_attention_residual_read_ref(v, k, qc, Hh, 0.25,
                                                                                              key_norm))
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
        assert_close(kd[s].grad, kc[s].grad, dtype, f"dk{s}")
    assert_close(qd.grad, qc.grad, dtype, "dq", reduced=True)
    assert skd.grad.dtype == torch.float32 and skd.grad.shape == (S, R)
    assert_close(skd.grad, skc.grad, dtype, "dstatic", reduced=True)


@pytest.mark.parametrize("key_norm", [True, False])
def test_config4_gated_read_with_static_keys(key_norm):
    """Config 4's read (gated per-token query, N17 r128 H8, d2048) with its
    [N, 128] static source key, on a token subset of its shape."""
    B, T, D, S, R, Hh = 1, 256, 2048, 17, 128, 8
    dtype = torch.bfloat16
    g, vals, keys, sk, up = _case(44 + key_norm, B, T, D, S, R, Hh, dtype)
    qs = randn(g, (Hh, R // Hh), dtype, 0.02)
    qdyn = randn(g, (B, T, R), dtype)
    gate = randn(g, (B, T, Hh), dtype)
    vd, kd, skd = [leaf(x) for x in vals], [leaf(x) for x in keys], leaf(sk)
    qsd, qdd, gd = leaf(qs), leaf(qdyn), leaf(gate)
    out = ops.lrid_attention_residual_read_gated(vd, kd, qsd, qdd, gd, Hh, 0.25, key_norm,
                                                 gate_activation="sigmoid", static_keys=skd)
    out.backward(up.to(DEV))
    qsc, qdc, gc = (x.clone().requires_grad_(True) for x in (qs, qdyn, gate))
    qq = O.gated_query_ref(qsc.float(), qdc.float(), gc.float(), Hh, "sigmoid")
    ref, vc, kc, skc = _ref(vals, keys, sk, lambda v, k: O.lrid_attention_residual_read_ref(v, k, qq, Hh, 0.25,
                                                                                              key_norm))
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
        assert_close(kd[s].grad, kc[s].grad, dtype, f"dk{s}")
    assert_close(qdd.grad, qdc.grad, dtype, "dq_dyn")
    assert_close(gd.grad, gc.grad, dtype, "dgate")
    assert_close(qsd.grad, qsc.grad, dtype, "dq_static", reduced=True)
    assert_close(skd.grad, skc.grad, dtype, "dstatic", reduced=True)


def test_static_keys_with_output_norm_and_a_bias():
    """The instantiation with every optional code path (output norm), a
    per-source bias, and static keys given as a list of [R] tensors."""
    B, T, D, S, R, Hh = 2, 33, 512, 6, 32, 2
    dtype = torch.bfloat16
    g, vals, keys, sk, up = _case(71, B, T, D, S, R, Hh, dtype)
    q = randn(g, (Hh, R // Hh), dtype, 0.5)
    vd, kd, qd = [leaf(x) for x in vals], [leaf(x) for x in keys], leaf(q)
    skl = [leaf(sk[s]) for s in range(S)]
    out = ops.lrid_attention_residual_read(vd, kd, qd, Hh, 0.25, True, normalize_output=True,
                                           source_logit_biases=[0.1 * s for s in range(S)], static_keys=skl)
    out.backward(up.to(DEV))
    qc = q.clone().requires_grad_(True)
    ref, vc, kc, skc = _ref(vals, keys, sk, lambda v, k: O.lrid_attention_residual_read_ref(
        v, k, qc, Hh, 0.25, True, normalize_output=True, source_logit_biases=[0.1 * s for s in range(S)]))
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
        assert_close(kd[s].grad, kc[s].grad, dtype, f"dk{s}")
        assert_close(skl[s].grad, skc.grad[s], dtype, f"dstatic{s}", reduced=True)
