"""GPU parity: the HIP kernels (through the drop-in API and its C ABI) against
the CPU oracle and the reference's golden vectors, forward and backward."""

import math

import pytest
import torch

from oracle import attnres_oracle as O
import attnres_ops as ops
import _attnres_hip as H
from _golden import load, names
from gpu_util import DEV, assert_close, leaf, gen, randn

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


# ------------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("name", names("lr"))
def test_lr_golden(name):
    t, m = load(name)
    dt = DT[m["dtype"]]
    S = m["S"]
    v = [leaf(x) for x in t["values"].unbind(0)]
    k = [leaf(x) for x in t["keys"].unbind(0)]
    q = leaf(t["query"])
    kw = {}
    b = None
    if m["has_bias"]:
        b = leaf(t["bias"])
        kw["source_logit_biases"] = b
    if m["has_counts"]:
        kw["source_counts"] = t["counts"].tolist()
    out = ops.lrid_attention_residual_read(v, k, q, m["H"], m["scale"], m["key_norm"],
                                           normalize_output=m["normalize_output"], **kw)
    out.backward(t["grad_out"].to(DEV))
    assert_close(out, t["out"], dt, "out")
    for s in range(S):
        assert_close(v[s].grad, t["dvalues"][s], dt, f"dv{s}")
        assert_close(k[s].grad, t["dkeys"][s], dt, f"dk{s}")
    assert_close(q.grad, t["dquery"], dt, "dq", reduced=not m["dynamic"])
    if b is not None:
        assert_close(b.grad, t["dbias"], dt, "dbias", reduced=True)


@pytest.mark.parametrize("name", names("base"))
def test_base_golden(name):
    t, m = load(name)
    dt = DT[m["dtype"]]
    v = [leaf(x) for x in t["values"].unbind(0)]
    q = leaf(t["query"])
    kw = {}
    b = None
    if m["has_bias"]:
        b = leaf(t["bias"])
        kw["source_logit_biases"] = b
    if m["has_counts"]:
        kw["source_counts"] = t["counts"].tolist()
    out = ops.attention_residual_read(v, q, m["key_norm"], normalize_output=m["normalize_output"], **kw)
    out.backward(t["grad_out"].to(DEV))
    assert_close(out, t["out"], dt, "out")
    for s in range(m["S"]):
        assert_close(v[s].grad, t["dvalues"][s], dt, f"dv{s}")
    assert_close(q.grad, t["dquery"], dt, "dq", reduced=True)
    if b is not None:
        assert_close(b.grad, t["dbias"], dt, "dbias", reduced=True)


@pytest.mark.parametrize("name", names("average"))
def test_average_golden(name):
    t, m = load(name)
    out = ops.attention_residual_average_read([x.to(DEV) for x in t["values"].unbind(0)], m["normalize_output"])
    assert_close(out, t["out"], DT[m["dtype"]], "out")


# ------------------------------------------------------------------ oracle sweeps

def _lr_case(seed, dtype, B, T, D, S, R, Hh, scale, key_norm, dynamic=False, bias=None, counts=None,
             normalize_output=False, stacked=False):
    g = gen(seed)
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    keys = [randn(g, (B, T, R), dtype) for _ in range(S)]
    qshape = (B, T, Hh, R // Hh) if dynamic else (Hh, R // Hh)
    query = randn(g, qshape, torch.float32, 0.5)
    up = randn(g, (B, T, D), dtype)
    kw = {}
    bias_c = bias_d = None
    if bias is not None:
        bias_c = torch.tensor(bias, dtype=torch.float32, requires_grad=True)
        bias_d = leaf(bias_c)
    if counts is not None:
        kw["source_counts"] = counts
    # GPU
    vd = [leaf(x) for x in vals]
    kd = [leaf(x) for x in keys]
    qd = leaf(query)
    vin = torch.stack(vd) if stacked else vd
    out = ops.lrid_attention_residual_read(vin, kd, qd, Hh, scale, key_norm, normalize_output=normalize_output,
                                           source_logit_biases=bias_d, **kw)
    out.backward(up.to(DEV))
    # oracle (CPU)
    vc = [x.clone().requires_grad_(True) for x in vals]
    kc = [x.clone().requires_grad_(True) for x in keys]
    qc = query.clone().requires_grad_(True)
    ref = O.lrid_attention_residual_read_ref(vc, kc, qc, Hh, scale, key_norm, normalize_output=normalize_output,
                                             source_logit_biases=bias_c, **kw)
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
        assert_close(kd[s].grad, kc[s].grad, dtype, f"dk{s}")
    assert_close(qd.grad, qc.grad, dtype, "dq", reduced=not dynamic)
    if bias is not None:
        assert_close(bias_d.grad, bias_c.grad, dtype, "dbias", reduced=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Hh,key_norm", [(1, True), (4, True), (4, False), (2, True)])
def test_lr_matches_oracle(dtype, Hh, key_norm):
    _lr_case(100 + Hh + 10 * int(key_norm), dtype, 2, 7, 128, 6, 32, Hh, 0.25, key_norm)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lr_options_dynamic_bias_norm(dtype):
    _lr_case(201, dtype, 2, 6, 128, 4, 32, 2, 0.5, True, dynamic=True)
    _lr_case(202, dtype, 1, 9, 64, 5, 16, 2, 0.25, True, bias=[0.0, 0.69, -0.3, 1.2, 0.1])
    _lr_case(203, dtype, 1, 9, 64, 5, 16, 2, 0.25, True, counts=[1, 2, 3, 4, 2])
    _lr_case(204, dtype, 2, 5, 256, 5, 64, 1, 0.125, True, normalize_output=True)
    _lr_case(205, dtype, 2, 5, 256, 5, 64, 4, 0.125, True, normalize_output=True, bias=[0.1, 0.2, 0.3, 0.4, 0.5])


@pytest.mark.parametrize("S", [2, 9, 13, 16, 17, 21, 24, 33, 64])
def test_lr_source_counts(S):
    _lr_case(300 + S, torch.bfloat16, 1, 5, 128, S, 32, 2, 0.25, True)


@pytest.mark.parametrize("D,R,Hh", [(40, 6, 2), (24, 12, 3), (2048, 128, 8), (1024, 512, 1), (520, 16, 2)])
def test_lr_odd_and_large_shapes(D, R, Hh):
    # D=40/24: not a multiple of 8 -> one-element path; R/H=3: scalar key path;
    # R=512/H=1: long key rows; D=2048: two waves per token; D=520: partial column
    _lr_case(400 + D, torch.bfloat16, 1, 5, D, 5, R, Hh, 1.0 / math.sqrt(R // Hh), True)


def test_lr_stacked_and_unaligned_keys():
    _lr_case(501, torch.bfloat16, 2, 4, 128, 5, 32, 2, 0.25, True, stacked=True)
    # keys as views of the value tails (model.py lrid_key_from_output_tail): not 16-byte aligned rows
    g = gen(502)
    vals = [randn(g, (2, 4, 128), torch.float32) for _ in range(5)]
    vd = [leaf(x) for x in vals]
    kd = [x[..., -24:] for x in vd]
    q = leaf(randn(g, (2, 12), torch.float32, 0.5))
    out = ops.lrid_attention_residual_read(vd, kd, q, 2, 0.3, True)
    up = randn(g, (2, 4, 128), torch.float32)
    out.backward(up.to(DEV))
    vc = [x.clone().requires_grad_(True) for x in vals]
    qc = q.detach().cpu().clone().requires_grad_(True)
    ref = O.lrid_attention_residual_read_ref(vc, [x[..., -24:] for x in vc], qc, 2, 0.3, True)
    ref.backward(up)
    assert_close(out, ref, torch.float32, "out")
    for s in range(5):
        assert_close(vd[s].grad, vc[s].grad, torch.float32, f"dv{s}")
    assert_close(q.grad, qc.grad, torch.float32, "dq")


def test_lr_aliased_sources_and_row_strides():
    g = gen(503)
    base = randn(g, (2, 4, 256), torch.bfloat16)
    vd_base = leaf(base)
    a = vd_base[..., :128]          # row stride 256 (not dense)
    b = vd_base[..., 128:]
    keys = [randn(g, (2, 4, 32), torch.bfloat16) for _ in range(3)]
    kd = [leaf(x) for x in keys]
    q = leaf(randn(g, (2, 16), torch.float32, 0.5))
    out = ops.lrid_attention_residual_read([a, b, a], kd, q, 2, 0.25, True)   # `a` twice
    up = randn(g, (2, 4, 128), torch.bfloat16)
    out.backward(up.to(DEV))
    vc = base.clone().requires_grad_(True)
    kc = [x.clone().requires_grad_(True) for x in keys]
    qc = q.detach().cpu().clone().requires_grad_(True)
    ref = O.lrid_attention_residual_read_ref([vc[..., :128], vc[..., 128:], vc[..., :128]], kc, qc, 2, 0.25, True)
    ref.backward(up)
    assert_close(out, ref, torch.bfloat16, "out")
    assert_close(vd_base.grad, vc.grad, torch.bfloat16, "dvalues (aliased)")


def _base_case(seed, dtype, B, T, D, S, key_norm, bias=None, counts=None, normalize_output=False, qstd=0.5):
    g = gen(seed)
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    query = randn(g, (D,), torch.float32, qstd)
    up = randn(g, (B, T, D), dtype)
    kw = {}
    bias_c = bias_d = None
    if bias is not None:
        bias_c = torch.tensor(bias, dtype=torch.float32, requires_grad=True)
        bias_d = leaf(bias_c)
    if counts is not None:
        kw["source_counts"] = counts
    vd = [leaf(x) for x in vals]
    qd = leaf(query)
    out = ops.attention_residual_read(vd, qd, key_norm, normalize_output=normalize_output,
                                      source_logit_biases=bias_d, **kw)
    out.backward(up.to(DEV))
    vc = [x.clone().requires_grad_(True) for x in vals]
    qc = query.clone().requires_grad_(True)
    ref = O.attention_residual_read_ref(vc, qc, key_norm, normalize_output=normalize_output,
                                        source_logit_biases=bias_c, **kw)
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
    assert_close(qd.grad, qc.grad, dtype, "dq", reduced=True)
    if bias is not None:
        assert_close(bias_d.grad, bias_c.grad, dtype, "dbias", reduced=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("key_norm", [True, False])
def test_base_matches_oracle(dtype, key_norm):
    _base_case(600 + int(key_norm), dtype, 2, 6, 256, 5, key_norm)


@pytest.mark.parametrize("S,D", [(2, 64), (7, 768), (13, 768), (9, 256), (12, 1024), (16, 2048), (17, 256),
                                 (40, 128), (5, 40)])
def test_base_shapes(S, D):
    _base_case(700 + S, torch.bfloat16, 1, 5, D, S, True)


# every slot count of the one-wave base kernels (exact up to 8 sources, then
# 10 / 12 / 14 / 16 with a spare slot for odd counts), cycling through the four
# column layouts, both dtypes, key norm on and off, and a learned logit bias
_ONE_WAVE_CASES = [(S, (768, 512, 1024, 256)[i % 4], (torch.bfloat16, torch.float16)[i % 2], i % 3 != 2, i % 4 in (1, 2))
                   for i, S in enumerate(range(2, 17))] + [(7, 768, torch.bfloat16, False, False),
                                                           (7, 768, torch.float16, True, True),
                                                           (5, 768, torch.bfloat16, True, True)]


@pytest.mark.parametrize("S,D,dtype,key_norm,bias", _ONE_WAVE_CASES)
def test_base_one_wave_rows(S, D, dtype, key_norm, bias):
    """16-bit rows one wave covers exactly (D = 256, 512, 768, 1024): every
    column layout and slot count of the one-wave base kernels, with and
    without key norm and a learned logit bias; 74 tokens leave part of the
    last workgroup's streams idle."""
    b = [0.3 * ((i % 3) - 1) for i in range(S)] if bias else None
    _base_case(900 + S + D, dtype, 2, 37, D, S, key_norm, bias=b)


@pytest.mark.parametrize("T", [1, 3, 6])
def test_base_one_wave_rows_few_tokens(T):
    """One to six tokens with a logit bias: the per-workgroup partial sums
    (768 query + 5 bias slots) fall back from 16-slot tiles to slot-major rows
    when the padded tiles would not fit the workspace."""
    _base_case(960 + T, torch.bfloat16, 1, T, 768, 5, True, bias=[0.2, -0.1, 0.0, 0.4, -0.3])


def test_base_one_wave_rows_strided_and_aliased_sources():
    """Sources that are column slices of wider tensors (row stride 832, not
    768) and one source passed twice: the one-wave base kernels address every
    row through the per-source stride table; the aliased source's gradient is
    the sum of its two slots."""
    g = gen(970)
    B, T, D, S = 2, 33, 768, 5
    wide = [randn(g, (B, T, D + 64), torch.bfloat16) for _ in range(S - 1)]
    q = randn(g, (D,), torch.float32, 0.1)
    up = randn(g, (B, T, D), torch.bfloat16)
    wd = [leaf(x) for x in wide]
    qd = leaf(q)
    src_d = [w[..., :D] for w in wd]
    out = ops.attention_residual_read(src_d + [src_d[1]], qd, True)
    out.backward(up.to(DEV))
    wc = [x.clone().requires_grad_(True) for x in wide]
    qc = q.clone().requires_grad_(True)
    src_c = [w[..., :D] for w in wc]
    ref = O.attention_residual_read_ref(src_c + [src_c[1]], qc, True)
    ref.backward(up)
    assert_close(out, ref, torch.bfloat16, "out")
    for s in range(S - 1):
        assert_close(wd[s].grad[..., :D], wc[s].grad[..., :D], torch.bfloat16, f"dv{s}")
        assert float(wd[s].grad[..., D:].abs().max()) == 0.0
    assert_close(qd.grad, qc.grad, torch.bfloat16, "dq", reduced=True)


def test_base_one_wave_rows_many_tokens():
    """More tokens than token streams (each stream walks several tokens); the
    query gradient sums every token."""
    g = gen(950)
    B, T, D, S = 4, 4500, 256, 5
    vals = [torch.randn(B, T, D, generator=g).to(torch.bfloat16) for _ in range(S)]
    q = torch.randn(D, generator=g) * 0.1
    up = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    vd = [leaf(x) for x in vals]
    qd = leaf(q)
    out = ops.attention_residual_read(vd, qd, True, source_counts=[1, 2, 2, 2, 1])
    out.backward(up.to(DEV))
    torch.cuda.synchronize()
    vc = [x.clone().requires_grad_(True) for x in vals]
    qc = q.clone().requires_grad_(True)
    ref = O.attention_residual_read_ref(vc, qc, True, source_counts=[1, 2, 2, 2, 1])
    ref.backward(up)
    assert_close(out, ref, torch.bfloat16, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, torch.bfloat16, f"dv{s}")
    assert_close(qd.grad, qc.grad, torch.bfloat16, "dq", reduced=True)


def test_base_row768_fp16_norm_counts():
    """768-element 16-bit rows (three 8-byte columns per wave) with output norm and counts."""
    _base_case(805, torch.float16, 2, 4, 768, 7, True, normalize_output=True, counts=[1, 2, 2, 2, 2, 2, 2])


def test_base_options():
    _base_case(801, torch.bfloat16, 2, 3, 64, 3, True, counts=[1, 3, 2])
    _base_case(802, torch.float32, 1, 4, 32, 4, True, bias=[0.0, 0.7, -0.3, 1.1])
    _base_case(803, torch.bfloat16, 1, 4, 128, 6, True, normalize_output=True)
    _base_case(804, torch.bfloat16, 2, 4, 1536, 20, True, normalize_output=True, bias=[0.1] * 20)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("normalize_output", [False, True])
def test_average_forward_backward(dtype, normalize_output):
    g = gen(900)
    vals = [randn(g, (2, 3, 96), dtype) for _ in range(5)]
    up = randn(g, (2, 3, 96), dtype)
    vd = [leaf(x) for x in vals]
    out = ops.attention_residual_average_read(vd, normalize_output=normalize_output)
    out.backward(up.to(DEV))
    vc = [x.clone().requires_grad_(True) for x in vals]
    ref = O.attention_residual_average_read_ref(vc, normalize_output)
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(5):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")


@pytest.mark.parametrize("act,per_token", [("sigmoid", True), ("linear", False)])
def test_gated_query_matches_oracle(act, per_token):
    dtype = torch.bfloat16
    g = gen(1000 + int(per_token))
    B, T, D, S, R, Hh = 2, 5, 256, 5, 64, 4
    vals = [randn(g, (B, T, D), dtype) for _ in range(S)]
    keys = [randn(g, (B, T, R), dtype) for _ in range(S)]
    qs = randn(g, (Hh, R // Hh), dtype, 0.3)
    qdyn = randn(g, (B, T, R), dtype)
    gate = randn(g, (B, T, Hh) if per_token else (Hh,), dtype)
    up = randn(g, (B, T, D), dtype)
    vd, kd = [leaf(x) for x in vals], [leaf(x) for x in keys]
    qsd, qdd, gd = leaf(qs), leaf(qdyn), leaf(gate)
    out = ops.lrid_attention_residual_read_gated(vd, kd, qsd, qdd, gd, Hh, 0.25, True, gate_activation=act)
    out.backward(up.to(DEV))
    vc, kc = [x.clone().requires_grad_(True) for x in vals], [x.clone().requires_grad_(True) for x in keys]
    qsc, qdc, gc = (x.clone().requires_grad_(True) for x in (qs, qdyn, gate))
    # the kernel composes in fp32 and rounds once; the oracle composes in fp32 too
    q = O.gated_query_ref(qsc.float(), qdc.float(), gc.float(), Hh, act)
    ref = O.lrid_attention_residual_read_ref(vc, kc, q, Hh, 0.25, True)
    ref.backward(up)
    assert_close(out, ref, dtype, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, dtype, f"dv{s}")
        assert_close(kd[s].grad, kc[s].grad, dtype, f"dk{s}")
    assert_close(qdd.grad, qdc.grad, dtype, "dq_dyn")
    assert_close(qsd.grad, qsc.grad, dtype, "dq_static", reduced=True)
    assert_close(gd.grad, gc.grad, dtype, "dgate", reduced=not per_token)


# ------------------------------------------------------------------ properties

def test_weights_sum_to_one_and_match_oracle():
    g = gen(1100)
    B, T, D, S, R, Hh = 2, 64, 1024, 13, 64, 4
    vals = [randn(g, (B, T, D), torch.bfloat16) for _ in range(S)]
    keys = [randn(g, (B, T, R), torch.bfloat16) for _ in range(S)]
    q = randn(g, (Hh, R // Hh), torch.bfloat16, 0.5)
    vd, kd, qd = [x.to(DEV) for x in vals], [x.to(DEV) for x in keys], q.to(DEV)
    desc = H.Desc(vd, kd, qd, None, None, None, Hh, 0.25, True, False, H.MODE_SOFTMAX, 0, False)
    out, w, _, _ = H.forward(desc, vd[0].device, torch.bfloat16, True, False, True)
    torch.cuda.synchronize()
    sums = w.double().sum(-1)
    assert float((sums - 1).abs().max()) <= 1e-6
    ref = O.softmax_weights_ref(keys, q, Hh, 0.25, True, base=False)  # [S,B,T,H]
    ref = ref.permute(1, 2, 3, 0).reshape(B * T, Hh, S)
    assert float((w.cpu() - ref).abs().max()) <= 1e-6



def test_kernel_timing_records_one_pair_per_call_and_changes_no_result():
    import ctypes
    g = gen(1150)
    B, T, D, S, R, Hh = 2, 64, 1024, 13, 64, 4
    vd = [randn(g, (B, T, D), torch.bfloat16).to(DEV) for _ in range(S)]
    kd = [randn(g, (B, T, R), torch.bfloat16).to(DEV) for _ in range(S)]
    qd = randn(g, (Hh, R // Hh), torch.bfloat16, 0.5).to(DEV)
    go = randn(g, (B * T, D), torch.bfloat16).to(DEV)
    desc = H.Desc(vd, kd, qd, None, None, None, Hh, 0.25, True, False, H.MODE_SOFTMAX, 0, False)

    def run():
        out, w, inv, pre = H.forward(desc, DEV, torch.bfloat16, True, False, True)
        grads = H.backward(desc, DEV, torch.bfloat16, go, pre, inv, w, want_dquery=True, want_dgate=False,
                           want_dbias=False, query_shape=tuple(qd.shape), gate_shape=(0,), lr=True,
                           has_query_dyn=False)
        return out, grads[0], grads[1], grads[2]

    plain = run()
    lib = H.load()
    assert lib.attnres_kernel_timing(1) == 0
    try:
        timed = run()
        timed2 = run()
        buf = (ctypes.c_float * 8)()
        n = lib.attnres_kernel_times(buf, 8)
        assert n == 4, lib.attnres_last_error()  # fwd, bwd, fwd, bwd
        assert all(0.0 < buf[i] < 1000.0 for i in range(n))
        assert lib.attnres_kernel_times(buf, 8) == 0  # read resets the recording
    finally:
        assert lib.attnres_kernel_timing(0) == 0
    torch.cuda.synchronize()
    for a, b in ((plain, timed), (plain, timed2)):
        assert torch.equal(a[0], b[0])
        for x, y in zip(a[1] + a[2], b[1] + b[2]):
            assert torch.equal(x, y)
        assert torch.equal(a[3], b[3])

def test_backward_is_deterministic():
    g = gen(1200)
    B, T, D, S, R, Hh = 4, 256, 1024, 13, 64, 4
    vals = [randn(g, (B, T, D), torch.bfloat16).to(DEV) for _ in range(S)]
    keys = [randn(g, (B, T, R), torch.bfloat16).to(DEV) for _ in range(S)]
    q = randn(g, (Hh, R // Hh), torch.float32, 0.5).to(DEV)
    bias = torch.randn(S, generator=g).to(DEV)
    up = randn(g, (B, T, D), torch.bfloat16).to(DEV)
    grads = []
    for _ in range(2):
        vd = [x.clone().requires_grad_(True) for x in vals]
        kd = [x.clone().requires_grad_(True) for x in keys]
        qd = q.clone().requires_grad_(True)
        bd = bias.clone().requires_grad_(True)
        ops.lrid_attention_residual_read(vd, kd, qd, Hh, 0.25, True, source_logit_biases=bd).backward(up)
        grads.append((qd.grad.clone(), bd.grad.clone(), vd[3].grad.clone(), kd[5].grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_empty_and_single_source():
    v = [torch.randn(2, 0, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True) for _ in range(3)]
    k = [torch.randn(2, 0, 16, device=DEV, dtype=torch.bfloat16, requires_grad=True) for _ in range(3)]
    q = torch.randn(2, 8, device=DEV, requires_grad=True)
    out = ops.lrid_attention_residual_read(v, k, q, 2, 0.25, True)
    assert out.shape == (2, 0, 64)
    out.sum().backward()
    assert q.grad is not None and float(q.grad.abs().sum()) == 0.0
    x = torch.randn(1, 3, 64, device=DEV)
    assert ops.lrid_attention_residual_read([x], [torch.randn(1, 3, 16, device=DEV)], q, 2, 0.25, True) is x
    with pytest.raises(RuntimeError, match="at most 64"):
        ops.attention_residual_read([x] * 65, torch.randn(64, device=DEV), True)


def test_bf16_rounding_ties_match_torch():
    """The kernels round to bf16 in hardware (v_cvt_pk_bf16_f32); check exact
    round-half-to-even ties against torch's rounding.  With a zero query the
    two-source weights are exactly 0.5, so out = (a + b) / 2 is exact in fp32
    and lands on a bf16 tie when a and b differ by one ulp."""
    base = torch.tensor([1.0, 1.0078125, -3.0, 0.5, 2.0 ** -20, 1.5, 100.0, 7.0], dtype=torch.float32)
    a = base.to(torch.bfloat16)
    ulp = torch.ldexp(torch.ones_like(base), torch.frexp(base)[1] - 8)  # one bf16 ulp of |base|
    b = (base + ulp).to(torch.bfloat16)
    D = 64
    va = a.repeat(D // a.numel()).view(1, 1, D)
    vb = b.repeat(D // b.numel()).view(1, 1, D)
    keys = [torch.zeros(1, 1, 16, dtype=torch.bfloat16) for _ in range(2)]
    q = torch.zeros(1, 16)
    out = ops.lrid_attention_residual_read([va.to(DEV), vb.to(DEV)], [k.to(DEV) for k in keys], q.to(DEV), 1, 1.0,
                                           False)
    ref = O.lrid_attention_residual_read_ref([va, vb], keys, q, 1, 1.0, False)
    assert torch.equal(out.cpu(), ref), (out.cpu(), ref)
    # the same through the output rounding of the base read
    out_b = ops.attention_residual_read([va.to(DEV), vb.to(DEV)], torch.zeros(D, device=DEV), False)
    ref_b = O.attention_residual_read_ref([va, vb], torch.zeros(D), False)
    assert torch.equal(out_b.cpu(), ref_b)


# ------------------------------------------------------------------ mixed dtypes

@pytest.mark.parametrize("kdt,vdt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.float16)])
@pytest.mark.parametrize("key_norm", [True, False])
@pytest.mark.parametrize("dynamic", [False, True])
def test_lr_keys_in_another_dtype(kdt, vdt, key_norm, dynamic):
    """Keys in another dtype than the values stay in their dtype: the eager
    read norms them in fp32 and rounds them to the value dtype, so the logits
    are a value-dtype contraction with key_norm and a key-dtype one without
    it (attnres_ops.py:4179-4186); key gradients come back in the key dtype."""
    g = gen(1300 + int(key_norm) + 2 * int(dynamic))
    B, T, D, S, R, Hh = 2, 9, 256, 5, 64, 4
    vals = [randn(g, (B, T, D), vdt) for _ in range(S)]
    keys = [randn(g, (B, T, R), kdt) for _ in range(S)]
    q = randn(g, (B, T, Hh, R // Hh) if dynamic else (Hh, R // Hh), torch.float32, 0.5)
    up = randn(g, (B, T, D), vdt)
    vd, kd, qd = [leaf(x) for x in vals], [leaf(x) for x in keys], leaf(q)
    out = ops.lrid_attention_residual_read(vd, kd, qd, Hh, 0.25, key_norm)
    out.backward(up.to(DEV))
    vc = [x.clone().requires_grad_(True) for x in vals]
    kc = [x.clone().requires_grad_(True) for x in keys]
    qc = q.clone().requires_grad_(True)
    ref = O.lrid_attention_residual_read_ref(vc, kc, qc, Hh, 0.25, key_norm)
    ref.backward(up)
    assert out.dtype == vdt and kd[0].grad.dtype == kdt
    # every result is downstream of a 16-bit rounding (weights, dW, or the
    # logits / rounded keys): the 16-bit bound of the coarser dtype applies
    tol = torch.bfloat16 if torch.bfloat16 in (kdt, vdt) else torch.float16
    assert_close(out, ref, tol, "out")
    for s in range(S):
        assert_close(vd[s].grad, vc[s].grad, tol, f"dv{s}")
        assert_close(kd[s].grad, kc[s].grad, tol, f"dk{s}")
    assert_close(qd.grad, qc.grad, tol, "dq", reduced=not dynamic)


def test_mixed_dtype_source_lists_are_promoted():
    """An fp32 embedding next to bf16 block summaries (what a bf16-autocast
    model hands the read): the sources are read in their common dtype, as the
    reference's eager read stacks them (attnres_ops.py:58-61, :2224, :3940),
    for the base read, the LR read (bf16 keys) and phase 1 from logits."""
    g = gen(1320)
    B, T, D, S, R, Hh = 2, 6, 256, 5, 32, 2
    vals = [randn(g, (B, T, D), torch.float32)] + [randn(g, (B, T, D), torch.bfloat16) for _ in range(S - 1)]
    keys = [randn(g, (B, T, R), torch.bfloat16) for _ in range(S)]
    qb = randn(g, (D,), torch.float32, 0.1)
    ql = randn(g, (Hh, R // Hh), torch.float32, 0.5)
    logits = randn(g, (3, S, B, T), torch.float32, 2.0)
    up = randn(g, (B, T, D), torch.float32)
    up1 = randn(g, (3, B, T, D), torch.float32)

    def check(run_gpu, run_ref, name, with_keys=False, upstream=up):
        vd, kd = [leaf(x) for x in vals], [leaf(x) for x in keys]
        vc, kc = [x.clone().requires_grad_(True) for x in vals], [x.clone().requires_grad_(True) for x in keys]
        out = run_gpu(vd, kd)
        ref = run_ref(vc, kc)
        assert out.dtype == torch.float32
        out.backward(upstream.to(DEV))
        ref.backward(upstream)
        assert_close(out, ref, torch.float32, f"{name} out")
        for s in range(S):
            assert vd[s].grad.dtype == vals[s].dtype
            assert_close(vd[s].grad, vc[s].grad, vals[s].dtype, f"{name} dv{s}")
            if with_keys:
                assert_close(kd[s].grad, kc[s].grad, torch.bfloat16, f"{name} dk{s}")

    check(lambda v, k: ops.attention_residual_read(v, leaf(qb), True),
          lambda v, k: O.attention_residual_read_ref(v, qb, True), "base")
    check(lambda v, k: ops.lrid_attention_residual_read(v, k, leaf(ql), Hh, 0.25, True),
          lambda v, k: O.lrid_attention_residual_read_ref(v, k, ql, Hh, 0.25, True), "lr", with_keys=True)
    check(lambda v, k: ops.attention_residual_phase1_from_logits(v, logits.to(DEV))[0],
          lambda v, k: O.phase1_from_logits_ref(v, logits)[0], "phase1", upstream=up1)
