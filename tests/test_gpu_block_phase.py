"""GPU parity of the block decoder's per-source logit path: the site-logits
kernels (one completed source's logits for every later read site, split into
the block phases that read them) and phase 1 from per-source logits with
per-site outputs.

Phase 1 from per-source logits runs the same kernels as phase 1 from a stacked
[Q, S, n] tensor, so it must agree with it bit for bit, forward and backward
(per-source logit gradients against the stacked gradient's slices), also when
some sites have no lse gradient.  The site logits are checked against the
oracle's restatement of the reference's eager chain (``make_source_logits``,
``model.py:1843-1865``) on the CPU, forward and backward, to the tolerances of
gpu_util.assert_close.
"""

import pytest
import torch

from oracle import attnres_oracle as O
import attnres_ops as ops
import _attnres_hip as H
from gpu_util import DEV, assert_close, gen, leaf, randn

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


# ------------------------------------------------- phase 1 from per-source logits

@pytest.mark.parametrize("S,Q,D,dtype,ldt", [
    (2, 3, 768, torch.bfloat16, torch.float32),      # one-wave kernels
    (4, 12, 1024, torch.bfloat16, torch.float32),    # column-split kernels (the published block)
    (7, 4, 768, torch.bfloat16, torch.bfloat16),     # bf16 logits
    (5, 6, 96, torch.float32, torch.float32),        # general kernels
    (3, 16, 512, torch.float16, torch.float32),
])
def test_block_phase1_matches_stacked_phase1(S, Q, D, dtype, ldt):
    g = gen(1000 + S * 31 + Q)
    B, T = 2, 45
    vals = [randn(g, (B, T, D), dtype).to(DEV) for _ in range(S)]
    lgs = [(randn(g, (Q, B, T), torch.float32) * 2).to(ldt).to(DEV) for _ in range(S)]
    gout = [randn(g, (B, T, D), dtype).to(DEV) for _ in range(Q)]
    # every third site's lse carries no gradient (a site read without a partial block)
    glse = [None if q % 3 == 1 else randn(g, (B, T), torch.float32).to(DEV) for q in range(Q)]

    v1 = [leaf(v) for v in vals]
    l1 = [leaf(lg) for lg in lgs]
    outs, lses = ops.lrid_block_phase1(v1, l1)
    terms = [(o, go) for o, go in zip(outs, gout)] + [(l, gl) for l, gl in zip(lses, glse) if gl is not None]
    torch.autograd.backward([t for t, _ in terms], [g_ for _, g_ in terms])

    v2 = [leaf(v) for v in vals]
    l2 = leaf(torch.stack(lgs, dim=1))
    out, lse = ops.attention_residual_phase1_from_logits(v2, l2)
    glse_st = torch.stack([gl if gl is not None else torch.zeros((B, T), device=DEV) for gl in glse])
    torch.autograd.backward([out, lse], [torch.stack(gout), glse_st])

    for q in range(Q):
        assert torch.equal(outs[q], out[q]), f"out[{q}]"
        assert torch.equal(lses[q], lse[q]), f"lse[{q}]"
    for s in range(S):
        assert torch.equal(v1[s].grad, v2[s].grad), f"dvalues[{s}]"
        assert torch.equal(l1[s].grad, l2.grad[:, s]), f"dlogits[{s}]"


def test_block_phase1_rejects_mismatched_logits():
    vals = [torch.zeros((1, 4, 256), device=DEV, dtype=torch.bfloat16) for _ in range(2)]
    lgs = [torch.zeros((3, 1, 4), device=DEV), torch.zeros((2, 1, 4), device=DEV)]
    with pytest.raises(RuntimeError, match="logits must all be"):
        ops.lrid_block_phase1(vals, lgs)


def test_block_phase1_promotes_mixed_logit_dtypes():
    """The embedding's logits stay 16-bit (no count prior) beside fp32 block
    logits: the pieces are promoted as torch.stack promotes them."""
    g = gen(1300)
    B, T, D, Q = 1, 37, 768, 4
    vals = [randn(g, (B, T, D), torch.bfloat16).to(DEV) for _ in range(3)]
    lgs = [randn(g, (Q, B, T), torch.float32).to(DEV) for _ in range(3)]
    lgs[0] = lgs[0].to(torch.bfloat16)
    gout = [randn(g, (B, T, D), torch.bfloat16).to(DEV) for _ in range(Q)]
    l1 = [leaf(lg) for lg in lgs]
    outs, lses = ops.lrid_block_phase1(vals, l1)
    torch.autograd.backward(list(outs), gout)
    l2 = [leaf(lg) for lg in lgs]
    out, lse = ops.attention_residual_phase1_from_logits(vals, torch.stack(l2, dim=1))
    out.backward(torch.stack(gout))
    for q in range(Q):
        assert torch.equal(outs[q], out[q]) and torch.equal(lses[q], lse[q])
    for a, b in zip(l1, l2):
        assert a.grad.dtype == b.grad.dtype and torch.equal(a.grad, b.grad)


# ------------------------------------------------------------------ site logits

def _site_case(seed, B, T, R, L, first, sizes, dtype, key_norm, bias, scale=0.125):
    g = gen(seed)
    key = randn(g, (B, T, R), dtype)
    queries = randn(g, (L, R), dtype, 0.5)
    grads = [randn(g, (n, B, T), torch.float32 if bias != 0.0 else dtype) for n in sizes]

    kd, qd = leaf(key), leaf(queries)
    parts = ops.lrid_site_logits(kd, qd, first, sizes, scale, bias, key_norm)
    torch.autograd.backward(list(parts), [x.to(DEV) for x in grads])

    kc = key.clone().requires_grad_(True)
    qc = queries.clone().requires_grad_(True)
    ref = O.lrid_site_logits_ref(kc, qc, first, sizes, scale, bias, key_norm)
    torch.autograd.backward(list(ref), grads)

    assert len(parts) == len(ref)
    for i, (a, e) in enumerate(zip(parts, ref)):
        assert a.dtype == e.dtype, (i, a.dtype, e.dtype)
        assert_close(a, e, dtype, f"logits[{i}]")
    assert_close(kd.grad, kc.grad, dtype, "dkey")
    assert_close(qd.grad, qc.grad, dtype, "dqueries", reduced=True)
    assert torch.count_nonzero(qd.grad[:first]) == 0


@pytest.mark.parametrize("R,dtype,key_norm,bias", [
    (32, torch.bfloat16, True, 0.0), (32, torch.bfloat16, True, 0.6931),
    (64, torch.bfloat16, True, 1.0986), (64, torch.bfloat16, False, 0.0),
    (128, torch.float16, True, 0.6931), (32, torch.float32, True, 0.6931),
    (40, torch.bfloat16, True, 0.6931),  # a rank whose rows are not 16-byte vectors
])
def test_site_logits_match_oracle(R, dtype, key_norm, bias):
    # 24 sites from query row 5 on, in phases of 7 / 6 / 6 / 5
    _site_case(2000 + R, 2, 83, R, 29, 5, (7, 6, 6, 5), dtype, key_norm, bias)


def test_site_logits_single_phase_and_many_tokens():
    _site_case(2100, 4, 1024, 64, 48, 0, (48,), torch.bfloat16, True, 0.0, scale=0.25)


def test_site_logits_limits():
    key = torch.zeros((1, 4, 160), device=DEV, dtype=torch.bfloat16)
    q = torch.zeros((4, 160), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="rank 160 exceeds"):
        ops.lrid_site_logits(key, q, 0, (4,), 1.0)
    with pytest.raises(RuntimeError, match="must cover"):
        ops.lrid_site_logits(key[..., :32], q[:, :32], 1, (4,), 1.0)
