"""GPU parity of the cached-logit block schedule (phase 1 / phase 2 kernels)
against the reference's golden vectors and the CPU oracle, forward and backward.

Tolerances are those of gpu_util.assert_close.  Quantities derived from
dtype-rounded intermediates (logit gradients, the lse gradient, learned bias
and scale gradients) are compared at the value dtype's bound even when they
are stored in fp32, because one storage ulp of an intermediate (e.g. the
rounded weight gradient) moves them by more than fp32 noise.
"""

import math

import pytest
import torch

from oracle import attnres_oracle as O
import attnres_ops as ops
import _attnres_hip as H
from _golden import load, names
from gpu_util import DEV, assert_close, leaf, gen, randn
from test_oracle_golden import _phase2_oracle

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


# ------------------------------------------------------------------ phase 1

def _phase1_hip(values, logits, g, glse, normalize_output):
    v = [leaf(x) for x in values]
    lg = leaf(logits)
    out, lse = ops.attention_residual_phase1_from_logits(v, lg, normalize_output=normalize_output)
    torch.autograd.backward([out, lse], [g.to(DEV), glse.to(DEV)])
    return out, lse, [x.grad for x in v], lg.grad


def _phase1_oracle(values, logits, g, glse, normalize_output):
    v = torch.stack(values).clone().requires_grad_(True)
    lg = logits.clone().requires_grad_(True)
    out, lse = O.phase1_from_logits_ref(v, lg, normalize_output=normalize_output)
    torch.autograd.backward([out, lse], [g, glse])
    return out.detach(), lse.detach(), list(v.grad.unbind(0)), lg.grad


@pytest.mark.parametrize("name", names("phase1"))
def test_phase1_golden(name):
    t, m = load(name)
    dt = DT[m["dtype"]]
    out, lse, dv, dl = _phase1_hip(list(t["values"].unbind(0)), t["logits"], t["grad_out"], t["grad_lse"],
                                   m["normalize_output"])
    assert_close(out, t["out"], dt, "out")
    assert_close(lse, t["lse"], torch.float32, "lse")
    for s in range(m["S"]):
        assert_close(dv[s], t["dvalues"][s], dt, f"dv{s}")
    assert_close(dl, t["dlogits"], dt, "dlogits", reduced=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,Q,D,ldt,norm", [
    (1, 1, 64, torch.float32, False),
    (3, 4, 256, torch.float32, False),
    (7, 4, 768, torch.float32, True),
    (5, 6, 1024, torch.bfloat16, False),
    (9, 11, 512, torch.float32, False),
    (13, 16, 128, torch.float32, True),
    (20, 3, 2048, torch.float32, False),
    (6, 2, 100, torch.float32, False),    # unaligned rows: scalar path
    (4, 8, 4096, torch.float32, False),
    (4, 3, 1280, torch.bfloat16, True),   # 16-bit rows: five waves of 8-byte vectors
])
def test_phase1_matches_oracle(dtype, S, Q, D, ldt, norm):
    g = gen(1000 + S * 31 + Q * 7 + D)
    B, T = 2, 9
    values = [randn(g, (B, T, D), dtype) for _ in range(S)]
    logits = randn(g, (Q, S, B, T), ldt, 2.0)
    go = randn(g, (Q, B, T, D), dtype)
    glse = randn(g, (Q, B, T), torch.float32)
    out, lse, dv, dl = _phase1_hip(values, logits, go, glse, norm)
    e_out, e_lse, e_dv, e_dl = _phase1_oracle(values, logits, go, glse, norm)
    assert_close(out, e_out, dtype, "out")
    assert_close(lse, e_lse, torch.float32, "lse")
    for s in range(S):
        assert_close(dv[s], e_dv[s], dtype, f"dv{s}")
    assert_close(dl, e_dl, dtype if dtype != torch.float32 else ldt, "dlogits", reduced=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,Q,D,ldt,T", [
    (7, 4, 768, torch.float32, 9),
    (8, 2, 1024, torch.bfloat16, 9),
    (2, 1, 512, torch.float16, 9),
    (5, 3, 256, torch.float32, 9),
    (1, 4, 768, torch.float32, 9),
    (6, 4, 768, torch.float32, 2100),   # more tokens than token streams
])
def test_phase1_one_wave_rows_backward(dtype, S, Q, D, ldt, T):
    """16-bit rows one wave covers exactly, <= 4 sites, <= 8 sources, no
    output norm: the packed-arithmetic phase-1 backward (every column layout,
    both source slot counts, 16-bit and fp32 logits)."""
    g = gen(3000 + S * 31 + Q * 7 + D + T)
    B = 2
    values = [randn(g, (B, T, D), dtype) for _ in range(S)]
    logits = randn(g, (Q, S, B, T), ldt, 2.0)
    go = randn(g, (Q, B, T, D), dtype)
    glse = randn(g, (Q, B, T), torch.float32)
    out, lse, dv, dl = _phase1_hip(values, logits, go, glse, False)
    e_out, e_lse, e_dv, e_dl = _phase1_oracle(values, logits, go, glse, False)
    assert_close(out, e_out, dtype, "out")
    for s in range(S):
        assert_close(dv[s], e_dv[s], dtype, f"dv{s}")
    assert_close(dl, e_dl, dtype, "dlogits", reduced=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,Q,D,ldt,T", [
    (4, 12, 1024, torch.float32, 9),     # the reference's published block (24 layers, 4 blocks)
    (8, 6, 1024, torch.bfloat16, 9),     # 24 layers, 8 blocks
    (16, 4, 768, torch.float32, 9),      # 16 sources
    (2, 16, 512, torch.float16, 9),      # 16 sites, two lanes per softmax row
    (5, 8, 256, torch.float32, 9),       # one wave per token
    (3, 16, 1536, torch.float32, 9),     # six waves per token
    (1, 9, 2048, torch.float32, 9),      # eight waves per token, one source
    (12, 4, 768, torch.float32, 4200),   # more tokens than workgroups
])
def test_phase1_split_rows(dtype, S, Q, D, ldt, T):
    """16-bit rows of a multiple of 256 elements, up to 16 sites: the column-
    split phase-1 kernels (D / 256 waves per token), forward and backward,
    every lane-layout width (np = 2 / 4 / 8 / 16) and fp32 / 16-bit logits."""
    g = gen(5000 + S * 31 + Q * 7 + D + T)
    B = 2
    values = [randn(g, (B, T, D), dtype) for _ in range(S)]
    logits = randn(g, (Q, S, B, T), ldt, 2.0)
    go = randn(g, (Q, B, T, D), dtype)
    glse = randn(g, (Q, B, T), torch.float32)
    print(f"phase-1 split: S{S} Q{Q} D{D} T{T} {dtype} logits {ldt}", flush=True)
    out, lse, dv, dl = _phase1_hip(values, logits, go, glse, False)
    e_out, e_lse, e_dv, e_dl = _phase1_oracle(values, logits, go, glse, False)
    assert_close(out, e_out, dtype, "out")
    assert_close(lse, e_lse, torch.float32, "lse")
    for s in range(S):
        assert_close(dv[s], e_dv[s], dtype, f"dv{s}")
    assert_close(dl, e_dl, dtype, "dlogits", reduced=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,Q,D,key_norm", [(3, 2, 256, True), (5, 4, 768, True), (6, 16, 100, False),
                                            (2, 1, 1024, True), (9, 3, 4096, False)])
def test_phase1_query_bank_matches_oracle(dtype, S, Q, D, key_norm):
    """attention_residual_phase1: logits of a query bank against the sources'
    keys (keyed-logits kernels), then the cached-logit read; gradients into
    the values (both paths) and the fp32 query bank."""
    g = gen(4000 + S * 31 + Q * 7 + D)
    B, T = 2, 7
    values = [randn(g, (B, T, D), dtype) for _ in range(S)]
    queries = randn(g, (Q, D), torch.float32, 2.0 / math.sqrt(D))  # logits of order 2
    go = randn(g, (Q, B, T, D), dtype)
    glse = randn(g, (Q, B, T), torch.float32)
    vd = [leaf(x) for x in values]
    qd = leaf(queries)
    out, lse = ops.attention_residual_phase1(vd, qd, key_norm)
    torch.autograd.backward([out, lse], [go.to(DEV), glse.to(DEV)])
    vc = torch.stack(values).clone().requires_grad_(True)
    qc = queries.clone().requires_grad_(True)
    e_out, e_lse = O.attention_residual_phase1_ref(vc, qc, key_norm)
    torch.autograd.backward([e_out, e_lse], [go, glse])
    assert_close(out, e_out, dtype, "out")
    assert_close(lse, e_lse, torch.float32 if dtype == torch.float32 else dtype, "lse", reduced=True)
    for s in range(S):
        assert_close(vd[s].grad, vc.grad[s], dtype, f"dv{s}")
    assert_close(qd.grad, qc.grad, dtype, "dqueries", reduced=True)


def test_phase1_unused_lse_and_strided_sources():
    # sources that are strided views (last-dim slices of a wider tensor) and a
    # backward through the output only
    g = gen(7)
    B, T, D, S, Q = 2, 5, 256, 4, 3
    wide = [randn(g, (B, T, D + 64), torch.bfloat16) for _ in range(S)]
    values = [w[..., :D] for w in wide]
    logits = randn(g, (Q, S, B, T), torch.float32, 2.0)
    go = randn(g, (Q, B, T, D), torch.bfloat16)
    v = [leaf(x) for x in wide]
    lg = leaf(logits)
    out, lse = ops.attention_residual_phase1_from_logits([x[..., :D] for x in v], lg)
    out.backward(go.to(DEV))
    e_out, _, e_dv, e_dl = _phase1_oracle(values, logits, go, torch.zeros(Q, B, T), False)
    assert_close(out, e_out, torch.bfloat16, "out")
    for s in range(S):
        assert_close(v[s].grad[..., :D], e_dv[s], torch.bfloat16, f"dv{s}")
        assert float(v[s].grad[..., D:].abs().max()) == 0.0
    assert_close(lg.grad, e_dl, torch.bfloat16, "dlogits", reduced=True)


def test_phase1_weights_are_a_softmax():
    # uniform logits -> the phase-1 output is the mean of the sources; lse = log S
    g = gen(11)
    B, T, D, S, Q = 1, 7, 512, 5, 2
    values = [randn(g, (B, T, D), torch.float32) for _ in range(S)]
    logits = torch.full((Q, S, B, T), 0.3)
    out, lse = ops.attention_residual_phase1_from_logits([v.to(DEV) for v in values], logits.to(DEV))
    mean = torch.stack(values).mean(0)
    for q in range(Q):
        assert_close(out[q], mean, torch.float32, "mean")
    assert torch.allclose(lse.cpu(), torch.full((Q, B, T), 0.3 + math.log(S)), atol=1e-6)


# ------------------------------------------------------------------ phase 2

def _phase2_hip(t, m):
    p = leaf(t["partial"])
    it = leaf(t["inter"])
    ls = leaf(t["lse"])
    bias = m["bias"]
    bt = None
    if m["bias_tensor"] and m["variant"] != "logit":
        bt = torch.tensor(bias, dtype=torch.float32, device=DEV).requires_grad_(True)
        bias = bt
    grads = {}
    if m["variant"] == "base":
        q = leaf(t["query"])
        out = ops.attention_residual_phase2_torch(p, q, it, ls, m["key_norm"], normalize_output=m["normalize_output"],
                                                  logit_bias=bias)
    elif m["variant"] in ("lrid", "lrid_addcmul"):
        k = leaf(t["partial_key"])
        q = leaf(t["query"])
        fn = ops.lrid_attention_residual_phase2_torch if m["variant"] == "lrid" else ops.lrid_attention_residual_phase2
        out = fn(p, k, q, it, ls, m["scale"], m["key_norm"], normalize_output=m["normalize_output"], logit_bias=bias)
    else:
        q = leaf(t["logit"])
        out = ops.attention_residual_phase2_from_logit(p, q, it, ls, normalize_output=m["normalize_output"])
    out.backward(t["grad_out"].to(DEV))
    grads.update(dpartial=p.grad, dinter=it.grad, dlse=ls.grad)
    grads["dlogit" if m["variant"] == "logit" else "dquery"] = q.grad
    if m["variant"] in ("lrid", "lrid_addcmul"):
        grads["dpartial_key"] = k.grad
    if bt is not None:
        grads["dbias"] = bt.grad.reshape(1)
    return out, grads


def _check_phase2(out, grads, ref_out, ref_grads, dt):
    assert_close(out, ref_out, dt, "out")
    for key, g in grads.items():
        reduced = key in ("dquery", "dbias", "dscale")
        assert_close(g, ref_grads[key], dt, key, reduced=reduced or key in ("dlse", "dlogit"))


@pytest.mark.parametrize("name", names("phase2"))
def test_phase2_golden(name):
    t, m = load(name)
    out, grads = _phase2_hip(t, m)
    _check_phase2(out, grads, t["out"], {k: t[k] for k in grads}, DT[m["dtype"]])


def _phase2_case(seed, dtype, B, T, D, variant, R=64):
    g = gen(seed)
    t = {"partial": randn(g, (B, T, D), dtype), "inter": randn(g, (B, T, D), dtype),
         "lse": randn(g, (B, T), torch.float32), "grad_out": randn(g, (B, T, D), dtype)}
    if variant == "base":
        t["query"] = randn(g, (D,), dtype, 0.5)
    elif variant in ("lrid", "lrid_addcmul"):
        t["partial_key"] = randn(g, (B, T, R), dtype)
        t["query"] = randn(g, (1, R), dtype, 0.5)
    else:
        t["logit"] = randn(g, (B, T), torch.float32, 2.0)
    return t


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("variant", ["base", "lrid", "lrid_addcmul", "logit"])
@pytest.mark.parametrize("D,key_norm,bias,bias_tensor,norm", [
    (768, True, None, False, False),
    (1024, False, 0.693, False, True),
    (2048, True, 1.2, True, False),
    (100, True, -0.4, True, True),   # unaligned rows
    (4096, True, None, False, False),
])
def test_phase2_matches_oracle(dtype, variant, D, key_norm, bias, bias_tensor, norm):
    seed = {"base": 1, "lrid": 2, "lrid_addcmul": 3, "logit": 4}[variant] * 10000 + D
    t = _phase2_case(seed, dtype, 2, 7, D, variant)
    m = dict(variant=variant, key_norm=key_norm, bias=0.0 if bias is None else bias, bias_tensor=bias_tensor,
             normalize_output=norm, scale=0.125)
    out, grads = _phase2_hip(t, m)
    ref_out, ref_grads = _phase2_oracle(t, m)
    _check_phase2(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,key_norm,bias_tensor", [(256, True, False), (512, False, True), (768, True, True),
                                                    (1024, True, False), (768, False, False)])
def test_phase2_one_wave_rows(dtype, D, key_norm, bias_tensor):
    """Base keys on 16-bit rows one wave covers exactly, no output norm: the
    packed-arithmetic phase-2 kernels (every column layout, with and without
    key norm); 111 tokens leave part of the last workgroup idle."""
    t = _phase2_case(5000 + D + int(key_norm), dtype, 3, 37, D, "base")
    m = dict(variant="base", key_norm=key_norm, bias=0.3, bias_tensor=bias_tensor, normalize_output=False,
             scale=0.125)
    out, grads = _phase2_hip(t, m)
    ref_out, ref_grads = _phase2_oracle(t, m)
    _check_phase2(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,R,variant,key_norm,norm", [
    (256, 64, "lrid", True, True), (256, 32, "lrid_addcmul", False, False),
    (512, 128, "lrid", True, False), (512, 100, "lrid_addcmul", True, True),
    (768, 64, "lrid", True, True), (768, 256, "lrid_addcmul", True, False),
    (1024, 64, "lrid", False, True), (1024, 200, "lrid", True, True)])
def test_lrid_phase2_one_wave_rows(dtype, D, R, variant, key_norm, norm):
    """LR keys on 16-bit rows one wave covers exactly: the packed-arithmetic
    phase-2 kernels (every column layout, 1, 2 and 4 key elements per lane,
    both merges, with and without key norm and the fused output norm); 111
    tokens leave part of the last workgroup idle."""
    t = _phase2_case(6000 + D + R, dtype, 3, 37, D, variant, R=R)
    m = dict(variant=variant, key_norm=key_norm, bias=0.3, bias_tensor=True, normalize_output=norm, scale=0.25)
    out, grads = _phase2_hip(t, m)
    ref_out, ref_grads = _phase2_oracle(t, m)
    _check_phase2(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("R", [16, 64, 128, 200, 256, 1024])
def test_lrid_phase2_key_widths(R):
    t = _phase2_case(40 + R, torch.bfloat16, 1, 6, 512, "lrid", R=R)
    m = dict(variant="lrid", key_norm=True, bias=0.3, bias_tensor=False, normalize_output=False, scale=0.25)
    out, grads = _phase2_hip(t, m)
    ref_out, ref_grads = _phase2_oracle(t, m)
    _check_phase2(out, grads, ref_out, ref_grads, torch.bfloat16)


@pytest.mark.parametrize("variant,dtype", [("lrid", torch.bfloat16), ("base", torch.float32),
                                           ("lrid_addcmul", torch.float32)])
def test_phase2_many_tokens_matches_oracle(variant, dtype):
    """More tokens than workgroups x waves (16400 > 2048 x 4): each wave walks
    several tokens and the cross-token sums go through many partial rows.
    (At this many tokens a 16-bit base-key case meets one-ulp flips of a
    per-token scalar -- dprob, the logit -- whose fp32 sum order differs from
    the oracle's; that case is covered by the layout test below.)"""
    t = _phase2_case(300 + len(variant), dtype, 4, 4100, 768, variant)
    m = dict(variant=variant, key_norm=True, bias=0.4, bias_tensor=True, normalize_output=True, scale=0.125)
    out, grads = _phase2_hip(t, m)
    ref_out, ref_grads = _phase2_oracle(t, m)
    _check_phase2(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("variant", ["base", "lrid", "lrid_addcmul", "logit"])
@pytest.mark.parametrize("D", [512, 1024])
def test_phase2_wave_layout_matches_block_layout(variant, D):
    """For rows one wave covers with 16-byte vectors, phase 2 runs one wave
    per token; the workgroup-per-token kernels (selected through the test
    hook attnres_test_phase2_block_layout) sum each row in the same order, so every per-token output and gradient
    is bit-identical in bf16.  Cross-token sums (query, bias) walk tokens in
    another order and are compared at the reduced bound.  (D=768 uses 8-byte
    vectors, whose sums associate differently; it is checked against the
    oracle by the tests above.)"""
    t = _phase2_case(700 + D + len(variant), torch.bfloat16, 4, 4100, D, variant)
    m = dict(variant=variant, key_norm=True, bias=0.4, bias_tensor=True, normalize_output=True, scale=0.125)
    out_w, g_w = _phase2_hip(t, m)
    lib = H.load()
    assert lib.attnres_test_phase2_block_layout(1) == 0
    try:
        out_b, g_b = _phase2_hip(t, m)
    finally:
        assert lib.attnres_test_phase2_block_layout(0) == 0
    assert torch.equal(out_w, out_b)
    for key in g_w:
        if key in ("dquery", "dbias"):
            assert_close(g_w[key], g_b[key], torch.bfloat16, key, reduced=True)
        else:
            assert torch.equal(g_w[key], g_b[key]), key


# ------------------------------------------------------------------ block summaries folded into phase 2

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("variant", ["base", "lrid", "lrid_addcmul"])
@pytest.mark.parametrize("scale_kind", ["float", "tensor"])
@pytest.mark.parametrize("key_norm", [True, False])
def test_phase2_partial_scale_is_the_block_summary(dtype, variant, scale_kind, key_norm):
    """phase2(partial_block, partial_scale=s) == phase2(block_summary(partial_block)),
    the model's summary being ``partial * count**-alpha`` (model.py:990-1018;
    LR keys scaled only without key_norm)."""
    g = gen(77)
    B, T, D, R = 2, 5, 768, 64
    count, alpha = 3, 0.5
    pb = randn(g, (B, T, D), dtype)
    it = randn(g, (B, T, D), dtype)
    lse = randn(g, (B, T), torch.float32)
    go = randn(g, (B, T, D), dtype)
    pk = randn(g, (B, T, R), dtype)
    q = randn(g, (D,) if variant == "base" else (1, R), dtype, 0.5)
    scale_key = variant != "base" and not key_norm

    # oracle: materialise the summary, then the reference merge (CPU)
    a_t = torch.tensor(alpha, requires_grad=True)
    s_ref = O.block_count_scale(count, a_t) if scale_kind == "tensor" else O.block_count_scale(count, alpha)
    pb_c = pb.clone().requires_grad_(True)
    it_c = it.clone().requires_grad_(True)
    ls_c = lse.clone().requires_grad_(True)
    q_c = q.clone().requires_grad_(True)
    if variant == "base":
        v_sum = O.block_summary(pb_c, count, scale=s_ref)
        ref = O.attention_residual_phase2_ref(v_sum, q_c, it_c, ls_c, key_norm, logit_bias=math.log(count))
    else:
        pk_c = pk.clone().requires_grad_(True)
        v_sum, k_sum = O.lrid_block_source(pb_c, pk_c, count, key_norm=key_norm, scale=s_ref)
        ref = O.lrid_attention_residual_phase2_ref(v_sum, k_sum, q_c, it_c, ls_c, 0.25, key_norm,
                                                   logit_bias=math.log(count),
                                                   merge="lerp" if variant == "lrid" else "addcmul")
    ref.backward(go)

    # HIP: raw partial block + scale inside the kernel
    a_d = torch.tensor(alpha, device=DEV, requires_grad=True)
    s_hip = torch.exp(-a_d * math.log(count)) if scale_kind == "tensor" else float(count) ** -alpha
    p_d, it_d, ls_d, q_d = leaf(pb), leaf(it), leaf(lse), leaf(q)
    if variant == "base":
        out = ops.attention_residual_phase2_torch(p_d, q_d, it_d, ls_d, key_norm, logit_bias=math.log(count),
                                                  partial_scale=s_hip)
    else:
        k_d = leaf(pk)
        fn = ops.lrid_attention_residual_phase2_torch if variant == "lrid" else ops.lrid_attention_residual_phase2
        out = fn(p_d, k_d, q_d, it_d, ls_d, 0.25, key_norm, logit_bias=math.log(count), partial_scale=s_hip,
                 scale_key=scale_key)
    out.backward(go.to(DEV))
    assert_close(out, ref, dtype, "out")
    assert_close(p_d.grad, pb_c.grad, dtype, "dpartial_block")
    assert_close(it_d.grad, it_c.grad, dtype, "dinter")
    assert_close(ls_d.grad, ls_c.grad, dtype, "dlse", reduced=True)
    assert_close(q_d.grad, q_c.grad, dtype, "dquery", reduced=True)
    if variant != "base":
        assert_close(k_d.grad, pk_c.grad, dtype, "dpartial_key")
    if scale_kind == "tensor":
        assert_close(a_d.grad.reshape(1), a_t.grad.reshape(1), dtype, "dalpha", reduced=True)


# ------------------------------------------------------------------ query bank rows

@pytest.mark.parametrize("variant", ["lrid", "lrid_addcmul"])
@pytest.mark.parametrize("row", [0, 5, 47])
@pytest.mark.parametrize("T", [37, 2048])
def test_lrid_phase2_query_bank_row(variant, row, T):
    """phase2(query=bank, query_row=i) is phase2(query=bank[i]) bit for bit, and
    the bank's gradient is the select's: the row's gradient in row i, zeros
    elsewhere (written by the reduction, no fill or copy)."""
    g = gen(4100 + row)
    B, D, R, L = 1, 1024, 32, 48
    dt = torch.bfloat16
    pv, it, go = (randn(g, (B, T, D), dt) for _ in range(3))
    pk = randn(g, (B, T, R), dt)
    lse = randn(g, (B, T), torch.float32)
    bank = randn(g, (L, R), dt, 0.5)
    fn = ops.lrid_attention_residual_phase2_torch if variant == "lrid" else ops.lrid_attention_residual_phase2
    kw = dict(normalize_output=True, logit_bias=0.6931, partial_scale=0.5)

    b1 = leaf(bank)
    a = [leaf(x) for x in (pv, pk, it, lse)]
    out1 = fn(a[0], a[1], b1, a[2], a[3], 0.125, True, query_row=row, **kw)
    out1.backward(go.to(DEV))

    b2 = leaf(bank)
    c = [leaf(x) for x in (pv, pk, it, lse)]
    out2 = fn(c[0], c[1], b2[row], c[2], c[3], 0.125, True, **kw)
    out2.backward(go.to(DEV))

    assert torch.equal(out1, out2)
    assert torch.equal(b1.grad, b2.grad)
    assert int(torch.count_nonzero(b1.grad[torch.arange(L, device=DEV) != row])) == 0
    for x, y in zip(a, c):
        assert torch.equal(x.grad, y.grad)


def test_lrid_phase2_query_bank_row_limits():
    B, T, D, R = 1, 4, 256, 32
    pv = torch.zeros((B, T, D), device=DEV, dtype=torch.bfloat16)
    pk = torch.zeros((B, T, R), device=DEV, dtype=torch.bfloat16)
    lse = torch.zeros((B, T), device=DEV)
    with pytest.raises(RuntimeError, match="query_row=6 outside"):
        ops.lrid_attention_residual_phase2(pv, pk, torch.zeros((6, R), device=DEV, dtype=torch.bfloat16), pv, lse,
                                           0.125, True, query_row=6)
    with pytest.raises(RuntimeError, match="query bank must be"):
        ops.lrid_attention_residual_phase2(pv, pk, torch.zeros((6, R + 1), device=DEV, dtype=torch.bfloat16), pv,
                                           lse, 0.125, True, query_row=1)
    # no tokens: the bank's gradient is all zeros
    e = torch.empty((1, 0, D), device=DEV, dtype=torch.bfloat16)
    bank = torch.ones((6, R), device=DEV, dtype=torch.bfloat16, requires_grad=True)
    out = ops.lrid_attention_residual_phase2(e, torch.empty((1, 0, R), device=DEV, dtype=torch.bfloat16), bank, e,
                                             torch.empty((1, 0), device=DEV), 0.125, True, query_row=2)
    out.sum().backward()
    assert bank.grad.shape == (6, R) and float(bank.grad.abs().sum()) == 0.0


# ------------------------------------------------------------------ composition and sizes

def test_phase1_phase2_compose_to_the_full_read():
    """phase1 over completed sources, then the phase-2 merge of the partial
    block, equals one read over all sources (tests/test_attnres_ops.py:582-610)
    -- here both sides on the GPU, at a model-sized shape."""
    g = gen(5)
    B, T, D, S = 2, 512, 768, 6
    dtype = torch.float32
    completed = [randn(g, (B, T, D), dtype) for _ in range(S)]
    partial = randn(g, (B, T, D), dtype)
    q = randn(g, (D,), dtype, 0.5)
    cd = [c.to(DEV) for c in completed]
    pd, qd = partial.to(DEV), q.to(DEV)
    keys = torch.nn.functional.rms_norm(torch.stack(cd), (D,))
    logits = torch.einsum("d,sbtd->sbt", qd, keys).unsqueeze(0).contiguous()
    inter, lse = ops.attention_residual_phase1_from_logits(cd, logits)
    merged = ops.attention_residual_phase2(pd, qd, inter[0], lse[0], True)
    full = ops.attention_residual_read(cd + [pd], qd, True)
    assert_close(merged, full, dtype, "merged")


def test_phase_model_scale_subset_matches_oracle():
    """Config-5-like shape (B16 T1024 d768, 6 completed blocks, 4 read sites)
    on the GPU; the oracle checks a token subset (tokens are independent)."""
    g = gen(21)
    B, T, D, S, Q = 16, 1024, 768, 6, 4
    dtype = torch.bfloat16
    values = [randn(g, (B, T, D), dtype).to(DEV) for _ in range(S)]
    logits = randn(g, (Q, S, B, T), torch.float32, 2.0).to(DEV)
    out, lse = ops.attention_residual_phase1_from_logits(values, logits)
    idx = torch.tensor([0, 1, 777, 5000, B * T - 1])
    sub_v = [v.reshape(B * T, D)[idx].cpu().reshape(1, -1, D) for v in values]
    sub_l = logits.reshape(Q, S, B * T)[:, :, idx].cpu().reshape(Q, S, 1, -1)
    e_out, e_lse = O.phase1_from_logits_ref(sub_v, sub_l)
    assert_close(out.reshape(Q, B * T, D)[:, idx], e_out.reshape(Q, -1, D), dtype, "out")
    assert_close(lse.reshape(Q, B * T)[:, idx], e_lse.reshape(Q, -1), torch.float32, "lse")


def test_phase_empty_tokens():
    v = [torch.empty(0, 3, 64, device=DEV, requires_grad=True) for _ in range(3)]
    lg = torch.empty(2, 3, 0, 3, device=DEV, requires_grad=True)
    out, lse = ops.attention_residual_phase1_from_logits(v, lg)
    assert out.shape == (2, 0, 3, 64) and lse.shape == (2, 0, 3)
    (out.sum() + lse.sum()).backward()
    p = torch.empty(0, 3, 64, device=DEV, requires_grad=True)
    q = torch.randn(64, device=DEV, requires_grad=True)
    o2 = ops.attention_residual_phase2(p, q, p.detach(), torch.empty(0, 3, device=DEV), True)
    o2.sum().backward()
    assert float(q.grad.abs().sum()) == 0.0


def test_phase_backward_is_deterministic():
    t = _phase2_case(9, torch.bfloat16, 4, 256, 1024, "base")
    m = dict(variant="base", key_norm=True, bias=0.5, bias_tensor=True, normalize_output=False, scale=1.0)
    _, g1 = _phase2_hip(t, m)
    _, g2 = _phase2_hip(t, m)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
