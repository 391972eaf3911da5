"""GPU parity of the fused accumulate-and-read (``lrid_block_accumulate_read``):
a sublayer's projection grows the live partial block and the next read
site's LR merge reads the grown block, in one pass.

Bit for bit against the composition it replaces -- ``lrid_block_accumulate``
then ``lrid_attention_residual_phase2[_torch]`` on the grown block, both HIP
(the accumulation of model.py:363-388 / 2377-2389, the merge of
attnres_ops.py:4075-4160) -- in the forward and in every gradient autograd
forms there, including the sums where the grown block also feeds later
consumers; and within the gpu_util bound of the oracle's eager composition
on the CPU.
"""

import pytest
import torch

import _attnres_hip as H
import attnres_ops as ops
from decoder_util import OracleOps
from gpu_util import DEV, assert_close, gen, randn

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


@pytest.fixture
def fused_calls(monkeypatch):
    """Counts the fused entry point's forward calls (the op composes the two
    calls for shapes the fused kernels do not take)."""
    calls = []
    real = H.accum_read_forward

    def counting(*a, **k):
        calls.append(1)
        return real(*a, **k)

    monkeypatch.setattr(H, "accum_read_forward", counting)
    return calls


def _inputs(g, B, T, D, R, P, dtype, first, rows):
    y = randn(g, (B, T, P), dtype)
    pv = None if first else randn(g, (B, T, D), dtype)
    pk = None if first else randn(g, (B, T, R), dtype)
    bank = randn(g, (rows, R), dtype)
    inter = randn(g, (B, T, D), dtype)
    lse = randn(g, (B, T), torch.float32) + 1.0
    return [y, pv, pk, bank, inter, lse]


def _run(fused, leaves, D, R, heads, key_norm, kw, go, gv, gk):
    y, pv, pk, bank, inter, lse = leaves
    scale = 0.125
    if fused:
        v, k, o = ops.lrid_block_accumulate_read(y, pv, pk, bank, inter, lse, D, R, scale, heads, key_norm, **kw)
    else:
        kw = dict(kw)
        lerp = kw.pop("lerp")
        v, k = ops.lrid_block_accumulate(y, pv, pk, D, R, heads, key_norm)
        fn = ops.lrid_attention_residual_phase2_torch if lerp else ops.lrid_attention_residual_phase2
        o = fn(v, k, bank, inter, lse, scale, key_norm, **kw)
    outs = [(o, go)] + [(t, g) for t, g in ((v, gv), (k, gk)) if g is not None]
    torch.autograd.backward([t for t, _ in outs], [g for _, g in outs])
    return v, k, o


def _leaves(ts, device, extra=()):
    out = [t.to(device).requires_grad_(True) if t is not None else None for t in ts]
    return out + [e.to(device).requires_grad_(True) for e in extra]


CASES = [
    # D, R, P, heads, key_norm
    (768, 64, 64, 1, True),    # the whole-model configuration
    (256, 32, 32, 2, True),    # two key heads of 16
    (1024, 64, 64, 4, True),   # per-head norm, 16-byte vectors
    (512, 64, 80, 1, False),   # no key norm (the key scaled with the block), padding columns
    (768, 16, 16, 1, True),    # a narrow key
    (1024, 128, 128, 1, True),  # two key elements per lane, one 128-column head
    (512, 128, 128, 4, True),  # two key elements per lane, heads of 32
    (768, 256, 256, 2, True),  # four key elements per lane, heads of 128
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,R,P,heads,key_norm", CASES)
@pytest.mark.parametrize("first", [False, True])
@pytest.mark.parametrize("lerp,normalize_output", [(True, True), (False, False), (True, False)])
def test_accumulate_read_matches_the_composition(fused_calls, dtype, D, R, P, heads, key_norm, first, lerp,
                                                 normalize_output):
    g = gen(D + 7 * R + P + heads + 3 * first + 5 * lerp + 11 * normalize_output)
    B, T, rows, row = 2, 37, 6, 3
    ins = _inputs(g, B, T, D, R, D + P, dtype, first, rows)
    go, gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    kw = dict(lerp=lerp, normalize_output=normalize_output, logit_bias=0.37, partial_scale=3.0 ** -0.5,
              scale_key=not key_norm, query_row=row)
    lf, lc = _leaves(ins, DEV), _leaves(ins, DEV)
    v, k, o = _run(True, lf, D, R, heads, key_norm, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
    assert len(fused_calls) == 1
    ev, ek, eo = _run(False, lc, D, R, heads, key_norm, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
    assert torch.equal(v, ev)
    assert torch.equal(k, ek)
    assert torch.equal(o, eo)
    for name, a, b in zip(("y", "pv", "pk", "query", "inter", "lse"), lf, lc):
        if a is None:
            continue
        assert torch.equal(a.grad, b.grad), name
    if P > R:
        assert float(lf[0].grad[..., D + R:].abs().max()) == 0.0
    # the query bank's gradient sits in the read row only
    others = torch.cat([lf[3].grad[:row], lf[3].grad[row + 1:]])
    assert float(others.abs().max()) == 0.0
    # and the oracle's eager composition agrees to the gpu_util bound
    cpu = [t.detach().cpu() if t is not None else None for t in ins]
    e_v, e_k, e_o = OracleOps.lrid_block_accumulate_read(cpu[0], cpu[1], cpu[2], cpu[3], cpu[4], cpu[5], D, R, 0.125,
                                                         heads, key_norm, **kw)
    assert torch.equal(v.cpu(), e_v)
    assert_close(k, e_k, dtype, "grown key")
    assert_close(o, e_o, dtype, "read")


@pytest.mark.parametrize("others", ["none", "value", "key"])
def test_accumulate_read_gradients_without_other_consumers(fused_calls, others):
    """The grown block's other gradients may be absent (a block's last fused
    read before its end feeds only the completing accumulation): each missing
    one counts as zero, as autograd's sum has it."""
    dtype = torch.bfloat16
    g = gen(91 + len(others))
    B, T, D, R = 2, 45, 768, 64
    ins = _inputs(g, B, T, D, R, D + R, dtype, False, 4)
    go = randn(g, (B, T, D), dtype)
    gv = randn(g, (B, T, D), dtype).to(DEV) if others == "value" else None
    gk = randn(g, (B, T, R), dtype).to(DEV) if others == "key" else None
    kw = dict(lerp=True, normalize_output=True, logit_bias=0.0, partial_scale=0.5, scale_key=False, query_row=1)
    lf, lc = _leaves(ins, DEV), _leaves(ins, DEV)
    _run(True, lf, D, R, 1, True, kw, go.to(DEV), gv, gk)
    assert len(fused_calls) == 1
    _run(False, lc, D, R, 1, True, kw, go.to(DEV), gv, gk)
    for name, a, b in zip(("y", "pv", "pk", "query", "inter", "lse"), lf, lc):
        assert torch.equal(a.grad, b.grad), name


def test_accumulate_read_learned_bias_and_scale(fused_calls):
    """Logit bias and block scale as learned scalars: their gradients are
    token sums the merge's reduction forms in the same order either way."""
    dtype = torch.bfloat16
    g = gen(57)
    B, T, D, R = 2, 200, 768, 64
    ins = _inputs(g, B, T, D, R, D + R, dtype, False, 8)
    go, gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    extra = (torch.tensor(0.3), torch.tensor(0.6))
    res = []
    for fused in (True, False):
        lv = _leaves(ins, DEV, extra)
        kw = dict(lerp=False, normalize_output=False, logit_bias=lv[6], partial_scale=lv[7], scale_key=False,
                  query_row=5)
        _run(fused, lv[:6], D, R, 1, True, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
        res.append(lv)
    assert len(fused_calls) == 1
    for name, a, b in zip(("y", "pv", "pk", "query", "inter", "lse", "bias", "scale"), *res):
        assert torch.equal(a.grad, b.grad), name


def test_accumulate_read_at_the_model_size(fused_calls):
    """8192 tokens of the whole-model configuration: every wave walks several
    tokens.  Per-token results equal the composition bit for bit; the query
    bank's gradient, a cross-token sum whose fp32 partial rows follow each
    kernel's own grid (the fused backward runs one resident round at its 3
    waves per SIMD, the plain merge backward at 4), within the cross-token
    bound."""
    dtype = torch.bfloat16
    g = gen(4)
    B, T, D, R = 4, 2048, 768, 64
    ins = _inputs(g, B, T, D, R, D + R, dtype, False, 24)
    go, gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    kw = dict(lerp=True, normalize_output=True, logit_bias=0.69, partial_scale=0.5, scale_key=False, query_row=17)
    lf, lc = _leaves(ins, DEV), _leaves(ins, DEV)
    v, k, o = _run(True, lf, D, R, 1, True, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
    assert len(fused_calls) == 1
    ev, ek, eo = _run(False, lc, D, R, 1, True, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
    assert torch.equal(v, ev) and torch.equal(k, ek) and torch.equal(o, eo)
    for name, a, b in zip(("y", "pv", "pk", "inter", "lse"), [lf[i] for i in (0, 1, 2, 4, 5)],
                          [lc[i] for i in (0, 1, 2, 4, 5)]):
        assert torch.equal(a.grad, b.grad), name
    assert_close(lf[3].grad, lc[3].grad.float(), dtype, "query bank gradient (cross-token sum)", reduced=True)


def test_accumulate_read_composes_where_the_fused_kernels_do_not_reach(fused_calls):
    """fp32 rows and rows one wave does not cover (d800) take the two calls;
    the results are the composition's by construction."""
    for dtype, D in ((torch.float32, 768), (torch.bfloat16, 800)):
        R = 64
        g = gen(D)
        B, T = 1, 19
        ins = _inputs(g, B, T, D, R, D + R, dtype, False, 2)
        v, k, o = ops.lrid_block_accumulate_read(*[t.to(DEV) for t in ins], D, R, 0.1, 1, True, query_row=1)
        assert o.shape == (B, T, D)
    assert len(fused_calls) == 0


@pytest.mark.parametrize("T", [1, 5])
def test_accumulate_read_few_tokens(fused_calls, T):
    """Fewer tokens than a workgroup's waves: idle waves, one partial row."""
    dtype = torch.bfloat16
    g = gen(70 + T)
    B, D, R = 1, 768, 64
    ins = _inputs(g, B, T, D, R, D + R, dtype, False, 3)
    go, gv, gk = randn(g, (B, T, D), dtype), randn(g, (B, T, D), dtype), randn(g, (B, T, R), dtype)
    kw = dict(lerp=True, normalize_output=True, logit_bias=0.2, partial_scale=0.5, scale_key=False, query_row=2)
    lf, lc = _leaves(ins, DEV), _leaves(ins, DEV)
    v, k, o = _run(True, lf, D, R, 1, True, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
    assert len(fused_calls) == 1
    ev, ek, eo = _run(False, lc, D, R, 1, True, kw, go.to(DEV), gv.to(DEV), gk.to(DEV))
    assert torch.equal(v, ev) and torch.equal(k, ek) and torch.equal(o, eo)
    for name, a, b in zip(("y", "pv", "pk", "query", "inter", "lse"), lf, lc):
        assert torch.equal(a.grad, b.grad), name


def test_accumulate_read_empty_batch(fused_calls):
    """No tokens: empty outputs, zero gradients for the query bank (the two calls' behaviour)."""
    dtype = torch.bfloat16
    g = gen(80)
    ins = _inputs(g, 2, 0, 768, 64, 832, dtype, False, 3)
    lf = _leaves(ins, DEV)
    v, k, o = ops.lrid_block_accumulate_read(*lf, 768, 64, 0.125, 1, True, lerp=True, query_row=1)
    assert v.shape == (2, 0, 768) and k.shape == (2, 0, 64) and o.shape == (2, 0, 768)
    o.sum().backward()
    assert float(lf[3].grad.abs().max()) == 0.0
    assert len(fused_calls) == 0
