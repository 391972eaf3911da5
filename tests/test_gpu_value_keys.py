"""GPU parity of config 4's key producer -- keys projected from the sources'
values, ``rms_norm(v_s) @ W^T`` (model.py:420-428) -- and of config 4's read
by its full definition: keys from that projection plus a static source key
[N, 128] ~ N(0, 0.02), W_k [2048, 128] ~ N(0, 0.02), a sigmoid-gated
per-token query; against the oracle (the model's eager norm + Linear, the
broadcast static-key add and the eager read) on the CPU.

The projection GEMM is a library GEMM on both sides (hipBLASLt here, the CPU
BLAS in the oracle), so keys match within the bf16 bound, not bit for bit;
the weight gradient is a sum over all sources' tokens (reduced bound).
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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,R", [(2048, 128), (768, 64), (100, 16)])
@pytest.mark.parametrize("value_norm", [True, False])
def test_value_key_projection_matches_oracle(dtype, D, R, value_norm):
    g = gen(D + R + value_norm)
    B, T, S = 1, 64, 5
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    w = randn(g, (R, D), dtype, 0.02)
    gk = [randn(g, (B, T, R), dtype) for _ in range(S)]
    vd, wd = [leaf(x) for x in vals], leaf(w)
    keys = ops.lrid_value_key_projection(vd, wd, value_norm)
    torch.autograd.backward(keys, [x.to(DEV) for x in gk])
    vc, wc = [x.clone().requires_grad_(True) for x in vals], w.clone().requires_grad_(True)
    ref = O.lrid_value_key_projection_ref(vc, wc, value_norm)
    torch.autograd.backward(ref, gk)
    for s in range(S):
        assert_close(keys[s], ref[s], dtype, f"key{s}")
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
    assert_close(wd.grad, wc.grad, dtype, "dW", reduced=True)


def test_value_key_projection_key_subset_gradient():
    """Only some keys used downstream: the others' gradients count as zero."""
    g = gen(5)
    B, T, S, D, R = 2, 16, 3, 512, 32
    dtype = torch.bfloat16
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    w = randn(g, (R, D), dtype, 0.02)
    gk = randn(g, (B, T, R), dtype)
    vd, wd = [leaf(x) for x in vals], leaf(w)
    keys = ops.lrid_value_key_projection(vd, wd)
    keys[1].backward(gk.to(DEV))
    vc, wc = [x.clone().requires_grad_(True) for x in vals], w.clone().requires_grad_(True)
    ref = O.lrid_value_key_projection_ref(vc, wc)
    ref[1].backward(gk)
    assert vd[0].grad is not None and float(vd[0].grad.abs().max()) == 0.0
    assert_close(vd[1].grad, vc[1].grad, dtype, "dv1")
    assert_close(wd.grad, wc.grad, dtype, "dW", reduced=True)


def test_config4_by_its_full_definition():
    """Config 4 (B4 T4096 d2048 N17 r128 H8, bf16) on a B1 T1024 token subset:
    keys = rms_norm(v_s) @ W_k + static key, gated query, fwd + bwd; gradients
    reach the values through the read and the key projection."""
    g = gen(404)
    B, T, D, S, R, Hh = 1, 1024, 2048, 17, 128, 8
    dtype = torch.bfloat16
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    w = randn(g, (R, D), dtype, 0.02)
    sk = randn(g, (S, R), torch.float32, 0.02)
    qs = randn(g, (Hh, R // Hh), dtype, 0.02)
    qdyn = randn(g, (B, T, R), dtype)
    gate = randn(g, (B, T, Hh), dtype)
    up = randn(g, (B, T, D), dtype)

    vd, wd, skd = [leaf(x) for x in vals], leaf(w), leaf(sk)
    qsd, qdd, gd = leaf(qs), leaf(qdyn), leaf(gate)
    keys = ops.lrid_value_key_projection(vd, wd)
    out = ops.lrid_attention_residual_read_gated(vd, keys, qsd, qdd, gd, Hh, 0.25, False,
                                                 gate_activation="sigmoid", static_keys=skd)
    out.backward(up.to(DEV))

    vc = [x.clone().requires_grad_(True) for x in vals]
    wc, skc = w.clone().requires_grad_(True), sk.clone().requires_grad_(True)
    qsc, qdc, gc = (x.clone().requires_grad_(True) for x in (qs, qdyn, gate))
    kc = O.static_key_add_ref(O.lrid_value_key_projection_ref(vc, wc), skc)
    qq = O.gated_query_ref(qsc.float(), qdc.float(), gc.float(), Hh, "sigmoid")
    ref = O.lrid_attention_residual_read_ref(vc, kc, qq, Hh, 0.25, False)
    ref.backward(up)

    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
    assert_close(wd.grad, wc.grad, dtype, "dW", reduced=True)
    assert_close(skd.grad, skc.grad, dtype, "dstatic", reduced=True)
    assert_close(qdd.grad, qdc.grad, dtype, "dq_dyn")
    assert_close(gd.grad, gc.grad, dtype, "dgate")
    assert_close(qsd.grad, qsc.grad, dtype, "dq_static", reduced=True)
