"""Pin the oracle with checks the mathematics fixes (CPU).

* the eager restatement (run in float64) equals the independent fp64 numpy
  formulation, forward and backward (autograd vs closed-form gradients);
* the vectorised fp64 formulation equals element-by-element loops;
* closed forms from the reference's own tests: zero query -> uniform average,
  count prior -> count-weighted average (tests/test_attnres_ops.py:479-512),
  single source -> identity, huge bias -> that source;
* invariants: weights sum to 1, a common bias shift changes nothing,
  permutation equivariance over sources, linearity in the values, heads are
  independent, key rescaling is invisible under key_norm;
* ``torch.autograd.gradcheck`` on the restatement in float64.

Each check is chosen so that a plausible slip (dropped term, wrong sign,
transposed operand, head/source index swap) fails at least one.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attnres_oracle as O
from oracle import fp64 as F64

EPS64 = float(np.finfo(np.float64).eps)


def _close32(a, b):
    """fp32-level agreement, scaled to the reference magnitude (reductions
    over many terms carry absolute error proportional to their size)."""
    b = np.asarray(b)
    np.testing.assert_allclose(a, b, rtol=2e-6, atol=2e-7 * max(1.0, float(np.abs(b).max())))


def _t(x):
    return torch.tensor(np.asarray(x), dtype=torch.float64)


def _lr_inputs(seed, S=5, n=6, D=32, R=16, H=2, dynamic=False):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((S, n, D))
    k = rng.standard_normal((S, n, R))
    q = rng.standard_normal((n, H, R // H) if dynamic else (H, R // H)) * 0.7
    g = rng.standard_normal((n, D))
    return v, k, q, g


def _lr_torch(v, k, q, H, scale, key_norm, bias=None, normalize_output=False):
    S, n, D = v.shape
    vt = _t(v).reshape(S, 1, n, D).requires_grad_(True)
    kt = _t(k).reshape(S, 1, n, -1).requires_grad_(True)
    if q.ndim == 3:
        qt = _t(q).reshape(1, n, H, -1).requires_grad_(True)
    else:
        qt = _t(q).requires_grad_(True)
    bt = None if bias is None else _t(bias).requires_grad_(True)
    out = O.lrid_attention_residual_read_torch(vt, kt, qt, H, scale, key_norm, source_logit_biases=bt)
    if normalize_output:
        out = O.norm(out)
    return out, vt, kt, qt, bt


@pytest.mark.parametrize("H,key_norm,dynamic,use_bias,normalize_output", [
    (1, True, False, False, False),
    (2, True, False, True, False),
    (4, False, False, False, False),
    (2, True, True, False, False),
    (2, True, False, True, True),
    (4, False, True, True, True),
])
def test_lr_restatement_equals_fp64_math(H, key_norm, dynamic, use_bias, normalize_output):
    v, k, q, g = _lr_inputs(7 + H, H=H, dynamic=dynamic)
    bias = np.array([0.0, 0.4, -0.9, 1.3, 0.2]) if use_bias else None
    scale = 0.37
    out, vt, kt, qt, bt = _lr_torch(v, k, q, H, scale, key_norm, bias, normalize_output)
    # the reference norms LR keys in fp32 (``keys.float()``, attnres_ops.py:4180)
    # and always runs the softmax in fp32 (``logits.float()``, :4190), so a
    # float64 run of the restatement carries fp32 rounding in those steps
    eps = float(np.finfo(np.float32).eps) if key_norm else EPS64
    ref_out, p, _ = F64.lr_forward(v, k, q, H, scale, key_norm, bias, eps, normalize_output)
    _close32(out.detach().numpy().reshape(ref_out.shape), ref_out)
    out.backward(_t(g).reshape(out.shape))
    grads = F64.lr_backward(v, k, q, H, scale, key_norm, g, bias, eps, normalize_output)
    _close32(vt.grad.numpy().reshape(grads["dv"].shape), grads["dv"])
    _close32(kt.grad.numpy().reshape(grads["dk"].shape), grads["dk"])
    _close32(qt.grad.numpy().reshape(grads["dq"].shape), grads["dq"])
    if use_bias:
        _close32(bt.grad.numpy(), grads["dbias"])


@pytest.mark.parametrize("key_norm,use_bias,normalize_output", [
    (True, False, False), (False, False, False), (True, True, False), (True, False, True), (False, True, True)])
def test_base_restatement_equals_fp64_math(key_norm, use_bias, normalize_output):
    rng = np.random.default_rng(3)
    S, n, D = 4, 7, 24
    v = rng.standard_normal((S, n, D))
    q = rng.standard_normal(D) * 0.5
    g = rng.standard_normal((n, D))
    bias = np.array([0.1, -0.6, 0.8, 0.0]) if use_bias else None
    vt = _t(v).reshape(S, 1, n, D).requires_grad_(True)
    qt = _t(q).requires_grad_(True)
    bt = None if bias is None else _t(bias).requires_grad_(True)
    out = O.attention_residual_read_torch(vt, qt, key_norm, source_logit_biases=bt)
    if normalize_output:
        out = O.norm(out)
    # softmax is fp32 in the reference (attnres_ops.py:2189): fp32-level tolerance
    ref_out, p, _ = F64.base_forward(v, q, key_norm, bias, EPS64, normalize_output)
    _close32(out.detach().numpy().reshape(n, D), ref_out)
    out.backward(_t(g).reshape(out.shape))
    grads = F64.base_backward(v, q, key_norm, g, bias, EPS64, normalize_output)
    _close32(vt.grad.numpy().reshape(S, n, D), grads["dv"])
    _close32(qt.grad.numpy(), grads["dq"])
    if use_bias:
        _close32(bt.grad.numpy(), grads["dbias"])


@pytest.mark.parametrize("dynamic", [False, True])
def test_fp64_vectorised_equals_loops(dynamic):
    v, k, q, _ = _lr_inputs(11, S=3, n=4, D=8, R=6, H=2, dynamic=dynamic)
    bias = np.array([0.3, -0.2, 0.5])
    a, _, _ = F64.lr_forward(v, k, q, 2, 0.8, True, bias)
    b = F64.lr_forward_loops(v, k, q, 2, 0.8, True, bias)
    np.testing.assert_allclose(a, b, rtol=1e-13, atol=1e-13)


# ----------------------------------------------------------- closed forms

def test_zero_query_count_prior_is_weighted_average_base():
    # the reference's own known answer, tests/test_attnres_ops.py:479-492
    emb = torch.full((1, 2, 4), 1.0)
    blk = torch.full((1, 2, 4), 7.0)
    out = O.attention_residual_read_ref([emb, blk], torch.zeros(4), key_norm=False, source_counts=[1, 3])
    assert torch.allclose(out, (emb + 3 * blk) / 4)


def test_zero_query_count_prior_is_weighted_average_lr():
    # tests/test_attnres_ops.py:495-512
    emb = torch.full((1, 2, 8), 2.0)
    blk = torch.full((1, 2, 8), 10.0)
    keys = [torch.zeros(1, 2, 4), torch.zeros(1, 2, 4)]
    out = O.lrid_attention_residual_read_ref([emb, blk], keys, torch.zeros(1, 4), 1, 1.0, False,
                                             source_counts=[1, 3])
    assert torch.allclose(out, (emb + 3 * blk) / 4)


def test_zero_query_is_uniform_average():
    torch.manual_seed(0)
    vs = [torch.randn(2, 3, 16, dtype=torch.float64) for _ in range(5)]
    ks = [torch.randn(2, 3, 8, dtype=torch.float64) for _ in range(5)]
    out = O.lrid_attention_residual_read_ref(vs, ks, torch.zeros(2, 4, dtype=torch.float64), 2, 0.5, True)
    assert torch.allclose(out, torch.stack(vs).mean(0), atol=1e-14)
    out_b = O.attention_residual_read_ref(vs, torch.zeros(16, dtype=torch.float64), True)
    assert torch.allclose(out_b, torch.stack(vs).mean(0), atol=1e-14)


def test_single_source_is_identity():
    v = torch.randn(2, 3, 8)
    assert O.attention_residual_read_ref([v], torch.randn(8), True) is v
    assert O.lrid_attention_residual_read_ref([v], [torch.randn(2, 3, 4)], torch.randn(1, 4), 1, 1.0, True) is v


def test_huge_bias_selects_source():
    torch.manual_seed(1)
    vs = [torch.randn(1, 4, 8, dtype=torch.float64) for _ in range(4)]
    ks = [torch.randn(1, 4, 4, dtype=torch.float64) for _ in range(4)]
    bias = [0.0, 0.0, 200.0, 0.0]
    out = O.lrid_attention_residual_read_ref(vs, ks, torch.randn(1, 4, dtype=torch.float64), 1, 1.0, True,
                                             source_logit_biases=bias)
    assert torch.allclose(out, vs[2], atol=1e-12)


# ----------------------------------------------------------- invariants

def test_weights_sum_to_one_and_bias_shift_invariance():
    v, k, q, _ = _lr_inputs(5, H=4)
    _, p, _ = F64.lr_forward(v, k, q, 4, 0.5, True)
    np.testing.assert_allclose(p.sum(axis=0), 1.0, atol=1e-14)
    w = O.softmax_weights_ref(_t(k).unsqueeze(1), _t(q), 4, 0.5, True, base=False)
    assert torch.allclose(w.sum(0), torch.ones_like(w[0]), atol=1e-12)
    a, _, _ = F64.lr_forward(v, k, q, 4, 0.5, True, bias=np.full(5, 3.7))
    b, _, _ = F64.lr_forward(v, k, q, 4, 0.5, True)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_permutation_equivariance_over_sources():
    v, k, q, _ = _lr_inputs(6, H=2)
    perm = np.array([3, 0, 4, 1, 2])
    bias = np.array([0.1, 0.2, -0.3, 0.4, -0.5])
    a, _, _ = F64.lr_forward(v, k, q, 2, 0.5, True, bias)
    b, _, _ = F64.lr_forward(v[perm], k[perm], q, 2, 0.5, True, bias[perm])
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-13)
    out1 = O.lrid_attention_residual_read_torch(_t(v).unsqueeze(1), _t(k).unsqueeze(1), _t(q), 2, 0.5, True,
                                                source_logit_biases=list(bias))
    out2 = O.lrid_attention_residual_read_torch(_t(v[perm]).unsqueeze(1), _t(k[perm]).unsqueeze(1), _t(q), 2, 0.5,
                                                True, source_logit_biases=list(bias[perm]))
    assert torch.allclose(out1, out2, atol=1e-13)


def test_linearity_in_values_and_head_independence():
    v, k, q, _ = _lr_inputs(8, H=2)
    v2 = np.random.default_rng(9).standard_normal(v.shape)
    a, _, _ = F64.lr_forward(2.0 * v - 0.5 * v2, k, q, 2, 0.5, True)
    b1, _, _ = F64.lr_forward(v, k, q, 2, 0.5, True)
    b2, _, _ = F64.lr_forward(v2, k, q, 2, 0.5, True)
    np.testing.assert_allclose(a, 2.0 * b1 - 0.5 * b2, rtol=1e-12, atol=1e-12)
    # changing head 1's keys leaves head 0's output untouched
    k2 = k.copy()
    k2[..., 8:] = np.random.default_rng(10).standard_normal(k2[..., 8:].shape)
    c, _, _ = F64.lr_forward(v, k2, q, 2, 0.5, True)
    np.testing.assert_allclose(c[:, :16], b1[:, :16], rtol=1e-13, atol=1e-13)
    assert not np.allclose(c[:, 16:], b1[:, 16:])
    out_t = O.lrid_attention_residual_read_torch(_t(v).unsqueeze(1), _t(k2).unsqueeze(1), _t(q), 2, 0.5, True)
    c32, _, _ = F64.lr_forward(v, k2, q, 2, 0.5, True, eps=float(np.finfo(np.float32).eps))
    np.testing.assert_allclose(out_t.numpy().reshape(c.shape), c32, rtol=2e-6, atol=2e-7)


def test_key_scale_invariance_under_key_norm():
    v, k, q, _ = _lr_inputs(12, H=2)
    a, _, _ = F64.lr_forward(v, k, q, 2, 0.5, True, eps=0.0)
    b, _, _ = F64.lr_forward(v, 3.5 * k, q, 2, 0.5, True, eps=0.0)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)
    c, _, _ = F64.lr_forward(v, 3.5 * k, q, 2, 0.5, False)
    assert not np.allclose(a, c)


# ----------------------------------------------------------- gradcheck

@pytest.mark.parametrize("dynamic", [False, True])
def test_gradcheck_lr_restatement(dynamic):
    torch.manual_seed(2)
    H = 2
    v = torch.randn(3, 1, 2, 8, dtype=torch.float64, requires_grad=True)
    k = torch.randn(3, 1, 2, 6, dtype=torch.float64, requires_grad=True)
    q = torch.randn((1, 2, H, 3) if dynamic else (H, 3), dtype=torch.float64, requires_grad=True)
    b = torch.randn(3, dtype=torch.float64, requires_grad=True)

    def f(v, k, q, b):
        return O.norm(O.lrid_attention_residual_read_torch(v, k, q, H, 0.7, True, source_logit_biases=b))

    # the restatement runs its softmax in fp32, so finite differences are
    # only good to ~1e-4; sign / dropped-term errors are O(1)
    assert torch.autograd.gradcheck(f, (v, k, q, b), eps=1e-3, atol=2e-3, rtol=2e-3)


def test_gradcheck_base_restatement():
    torch.manual_seed(3)
    v = torch.randn(3, 1, 2, 6, dtype=torch.float64, requires_grad=True)
    q = torch.randn(6, dtype=torch.float64, requires_grad=True)
    b = torch.randn(3, dtype=torch.float64, requires_grad=True)

    def f(v, q, b):
        return O.attention_residual_read_torch(v, q, True, source_logit_biases=b)

    assert torch.autograd.gradcheck(f, (v, q, b), eps=1e-3, atol=2e-3, rtol=2e-3)


def _fd(fun, x, eps=1e-6):
    """Central finite differences of a scalar function of an array."""
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp = x.copy()
        xm = x.copy()
        xp[i] += eps
        xm[i] -= eps
        g[i] = (fun(xp) - fun(xm)) / (2 * eps)
    return g


@pytest.mark.parametrize("key_norm,normalize_output,dynamic", [(True, False, False), (False, True, True),
                                                               (True, True, False)])
def test_fp64_closed_form_lr_grads_equal_finite_differences(key_norm, normalize_output, dynamic):
    v, k, q, g = _lr_inputs(21, S=3, n=2, D=8, R=4, H=2, dynamic=dynamic)
    bias = np.array([0.2, -0.1, 0.4])
    args = (2, 0.9, key_norm)

    def loss(v_=v, k_=k, q_=q, b_=bias):
        out, _, _ = F64.lr_forward(v_, k_, q_, *args, bias=b_, normalize_output=normalize_output)
        return float(np.sum(out * g))

    grads = F64.lr_backward(v, k, q, *args, grad_out=g, bias=bias, normalize_output=normalize_output)
    np.testing.assert_allclose(grads["dv"], _fd(lambda x: loss(v_=x), v), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(grads["dk"], _fd(lambda x: loss(k_=x), k), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(grads["dq"], _fd(lambda x: loss(q_=x), q), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(grads["dbias"], _fd(lambda x: loss(b_=x), bias), rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("key_norm,normalize_output", [(True, False), (False, True), (True, True)])
def test_fp64_closed_form_base_grads_equal_finite_differences(key_norm, normalize_output):
    rng = np.random.default_rng(22)
    v = rng.standard_normal((3, 2, 6))
    q = rng.standard_normal(6) * 0.6
    g = rng.standard_normal((2, 6))
    bias = np.array([0.3, 0.0, -0.2])

    def loss(v_=v, q_=q, b_=bias):
        out, _, _ = F64.base_forward(v_, q_, key_norm, b_, normalize_output=normalize_output)
        return float(np.sum(out * g))

    grads = F64.base_backward(v, q, key_norm, g, bias, normalize_output=normalize_output)
    np.testing.assert_allclose(grads["dv"], _fd(lambda x: loss(v_=x), v), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(grads["dq"], _fd(lambda x: loss(q_=x), q), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(grads["dbias"], _fd(lambda x: loss(b_=x), bias), rtol=1e-6, atol=1e-8)


# ----------------------------------------------------------- block summaries (model.py known answers)

@pytest.mark.parametrize("alpha,denominator", [(1.0, 4.0), (0.5, 2.0)])
def test_block_summary_known_answers(alpha, denominator):
    # tests/test_attnres_ops.py:21-47: count 4 -> /4 (count), /2 (sqrt)
    value = torch.full((1, 2, 8), 8.0)
    key = torch.full((1, 2, 4), 4.0)
    assert torch.allclose(O.block_summary(value, 4, alpha), value / denominator)
    v, k = O.lrid_block_source(value, key, 4, alpha, key_norm=False)
    assert torch.allclose(v, value / denominator) and torch.allclose(k, key / denominator)
    v, k = O.lrid_block_source(value, key, 4, alpha, key_norm=True)
    assert torch.equal(k, key)


def test_block_value_norm_known_answer():
    # tests/test_attnres_ops.py:95-126: value_norm gives RMS 1 and leaves keys alone
    value = torch.arange(1, 17, dtype=torch.float32).reshape(1, 2, 8)
    key = torch.full((1, 2, 4), 4.0)
    v, k = O.lrid_block_source(value, key, 4, 1.0, value_norm=True)
    rms = v.pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-6)
    assert torch.equal(k, key)


def test_block_ends_and_count_bias():
    # model.py:828-836 for 12 layers / 6 blocks: every second sublayer ends a block
    assert O.make_block_ends(12, 6) == frozenset({4, 8, 12, 16, 20, 24})
    assert O.make_block_ends(3, 2) == frozenset({3, 6})
    assert O.block_count_logit_bias(1, 1.0) == 0.0
    assert O.block_count_logit_bias(4, 1.0) == pytest.approx(math.log(4))
    assert O.block_count_logit_bias(3, 0.0) == 0.0


def test_phase1_phase2_composition_equals_full_read():
    # tests/test_attnres_ops.py:582-610: phase1 over completed blocks, then the
    # sigmoid merge of the partial block, equals the full read with counts
    torch.manual_seed(11)
    values = [torch.randn(2, 3, 6) for _ in range(2)]
    partial = torch.randn(2, 3, 6)
    query = torch.randn(6)
    counts = [1, 4]
    logits = torch.stack([torch.sum(v * query, -1) + math.log(c) for v, c in zip(values, counts)]).unsqueeze(0)
    out, lse = O.phase1_from_logits_ref(values, logits)
    merged = O.attention_residual_phase2_ref(partial, query, out[0], lse[0], False, logit_bias=math.log(2.0))
    full = O.attention_residual_read_torch(values + [partial], query, False, source_counts=counts + [2])
    assert torch.allclose(merged, full, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("key_norm", [True, False])
def test_phase1_query_bank_single_query_is_the_read(key_norm):
    # one query row: phase 1 from a query bank is the base read with that query
    # (both are _attnres_*_read_torch in the reference); fp64, so the two
    # einsum contractions agree to rounding
    torch.manual_seed(12)
    values = [torch.randn(2, 3, 8, dtype=torch.float64) for _ in range(4)]
    q = torch.randn(8, dtype=torch.float64)
    out, lse = O.attention_residual_phase1_ref(values, q[None], key_norm)
    read = O.attention_residual_read_torch(values, q, key_norm)
    assert torch.allclose(out[0], read, atol=1e-12, rtol=1e-12)
    assert lse.shape == (1, 2, 3)


def test_phase1_query_bank_closed_form():
    # fp64 brute force: out[q] = sum_s softmax_s(<q, v_s / rms(v_s)>) v_s and
    # lse[q] = log sum_s exp(<q, v_s / rms(v_s)>), query by query
    torch.manual_seed(13)
    S, Q, B, T, D = 3, 3, 2, 2, 5
    v = torch.randn(S, B, T, D, dtype=torch.float64)
    qs = torch.randn(Q, D, dtype=torch.float64)
    out, lse = O.attention_residual_phase1_ref(v, qs, True)
    vn = v.numpy()
    eps = float(torch.finfo(torch.float64).eps)
    for qi in range(Q):
        for b in range(B):
            for t in range(T):
                ks = [vn[s, b, t] / np.sqrt(np.mean(vn[s, b, t] ** 2) + eps) for s in range(S)]
                lg = np.array([float(np.dot(qs[qi].numpy(), k)) for k in ks])
                w = np.exp(lg - lg.max())
                w /= w.sum()
                expect = sum(w[s] * vn[s, b, t] for s in range(S))
                assert np.allclose(out[qi, b, t].numpy(), expect, atol=1e-12)
                # the reference takes the lse of float(logits): fp32 precision
                ref = lg.max() + np.log(np.exp(lg - lg.max()).sum())
                assert abs(float(lse[qi, b, t]) - ref) < 1e-6 * max(1.0, abs(ref))


def test_gated_query_closed_forms():
    qs = torch.randn(2, 4)
    qd = torch.randn(1, 3, 8)
    gate0 = torch.zeros(2)
    q = O.gated_query_ref(qs, qd, gate0, 2, "linear")
    assert torch.allclose(q, qs.view(1, 1, 2, 4).expand(1, 3, 2, 4))
    q = O.gated_query_ref(qs, qd, torch.zeros(1, 3, 2), 2, "sigmoid")
    assert torch.allclose(q, qs.view(1, 1, 2, 4) + 0.5 * qd.view(1, 3, 2, 4))
