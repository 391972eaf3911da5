"""CPU check of the fused accumulate-and-read's autograd wiring
(``attnres_ops.lrid_block_accumulate_read`` / ``_AccumReadFn``), with the two
library calls answered by the oracle's eager composition on the CPU.

The library's kernels are not involved (their parity is the GPU tests'); this
pins the host side: which saved tensors the backward hands over, which
gradient goes to which input (the old partial value's is the projection
gradient's value columns, a strided view), the query bank's row, and the
decoder's schedule around the op.  The decoder with the fused op must give
the reference model's golden hidden state, loss and gradients bit for bit --
under ``loss.backward()`` and under ``torch.autograd.grad`` over the
parameters, as graph-capture harnesses call it.
"""

import contextlib
import weakref

import pytest
import torch

import _attnres_hip as H
import attnres_decoder as AD
import attnres_ops as ops
from decoder_util import OracleOps, build_from_case, lm_step, load_model_case, model_index
from oracle import attnres_oracle as O


class _Desc:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _compose(a, r, y, pv, pk, q, inter, lse):
    """The composition the fused op stands for, on tensors."""
    v, k = O.lrid_block_accumulate_ref(y, pv, pk, a.dim, a.rank, a.heads, a.key_norm)
    bias = r.bias_t.reshape(()) if r.bias_t is not None else r.bias_value
    scale = r.scale_t.reshape(()) if r.scale_t is not None else r.scale_value
    pv_s, pk_s = v * scale, (k * scale if r.scale_key else k)
    one = lambda t: t.unsqueeze(0)  # noqa: E731  (rows as a batch of one)
    out = O.lrid_attention_residual_phase2_ref(one(pv_s), one(pk_s), q, one(inter), one(lse), r.logit_scale,
                                               r.key_norm, r.normalize_output, bias,
                                               merge="lerp" if r.merge == H.MERGE_LERP else "addcmul")
    return v, k, out.squeeze(0)


@pytest.fixture
def oracle_kernels(monkeypatch):
    """Descriptors that keep their tensors, and forward / backward entry points
    computed by the oracle: the op's host code runs unchanged on the CPU."""
    calls = {"fwd": 0, "bwd": 0}

    def block_accum_desc(y, dim, rank, heads, key_norm, pv, pk, complete, value_norm, scale_key, scale_value,
                         scale_t):
        assert not complete and not value_norm and not scale_key and scale_t is None
        return _Desc(y=y, dim=dim, rank=rank, heads=heads, key_norm=key_norm, pv=pv, pk=pk)

    class Phase2:
        # the grown block (the op's own outputs) by weak reference, as the real
        # descriptor holds only its address: a strong one would be a cycle
        def __init__(self, pv, pk, q, pl, inter, lse, merge, key_norm, normalize_output, logit_scale, bias_value,
                     bias_t, scale_value, scale_t, scale_key):
            self.__dict__.update(pv=weakref.ref(pv), pk=weakref.ref(pk), q=q, inter=inter, lse=lse, merge=merge,
                                 key_norm=key_norm,
                                 normalize_output=normalize_output, logit_scale=logit_scale,
                                 bias_value=bias_value, bias_t=bias_t, scale_value=scale_value, scale_t=scale_t,
                                 scale_key=scale_key)

    def accum_read_forward(d, value, key, kinv, out, device):
        calls["fwd"] += 1
        a, r = d.acc, d.read
        assert r.pv() is value and r.pk() is key  # the merge reads the block this call grows
        v, k, o = _compose(a, r, a.y, a.pv, a.pk, r.q, r.inter, r.lse)
        value.copy_(v)
        key.copy_(k)
        out.copy_(o)

    def accum_read_backward(d, device, dtype, grad_out, grad_value, grad_key, kinv, want_dquery, query_shape,
                            query_row, want_dbias, want_dscale, want_dpk_old):
        calls["bwd"] += 1
        a, r = d.acc, d.read
        leaf = lambda t: t.detach().clone().requires_grad_(True) if t is not None else None  # noqa: E731
        y, pv, pk, q, inter, lse = (leaf(t) for t in (a.y, a.pv, a.pk, r.q, r.inter, r.lse))
        r2 = _Desc(**r.__dict__)
        r2.bias_t, r2.scale_t = leaf(r.bias_t), leaf(r.scale_t)
        with torch.enable_grad():
            v, k, o = _compose(a, r2, y, pv, pk, q, inter, lse)
            outs = [(o, grad_out)] + [(t, g) for t, g in ((v, grad_value), (k, grad_key)) if g is not None]
            ins = [y, q, inter, lse] + [t for t in (pk, r2.bias_t, r2.scale_t) if t is not None]
            grads = torch.autograd.grad([t for t, _ in outs], ins, [g for _, g in outs], allow_unused=True)
        gy, dq_row, di, dl = grads[:4]
        rest = list(grads[4:])
        dpk = rest.pop(0) if pk is not None else None
        db = rest.pop(0) if r2.bias_t is not None else None
        ds = rest.pop(0) if r2.scale_t is not None else None
        dq = None
        if want_dquery:
            dq = torch.zeros(query_shape, dtype=dtype)
            dq[query_row] = dq_row
        return (gy, dpk if want_dpk_old else None, dq, di, dl, db if want_dbias else None,
                ds if want_dscale else None)

    monkeypatch.setattr(H, "block_accum_desc", block_accum_desc)
    monkeypatch.setattr(H, "Phase2", Phase2)
    monkeypatch.setattr(H, "accum_read_desc", lambda acc, read: _Desc(acc=acc, read=read))
    monkeypatch.setattr(H, "accum_read_forward", accum_read_forward)
    monkeypatch.setattr(H, "accum_read_backward", accum_read_backward)
    monkeypatch.setattr(ops, "_check_gpu", lambda tensors, what: tensors[0].device)
    monkeypatch.setattr(ops, "_device_ctx", lambda dev: contextlib.nullcontext())
    monkeypatch.setattr(ops, "_accum_read_fits", lambda *a: True)  # any shape reaches the op
    return calls


class _FusedOps(OracleOps):
    """Oracle reads, with the op under test for the accumulate-and-read."""
    lrid_block_accumulate_read = staticmethod(ops.lrid_block_accumulate_read)


# the cases whose sublayers hand over their projections (pre-norm LR-AttnRes)
_CASES = sorted(n for n, m in model_index().items() if m["config"].get("use_attnres", True)
                and m["config"].get("lrid_rank") and m["config"].get("norm_pos", "before") == "before")


@pytest.mark.parametrize("name", _CASES)
def test_decoder_with_the_fused_read_matches_reference_model(oracle_kernels, name):
    t, meta = load_model_case(name)
    model = build_from_case(t, meta, _FusedOps, fold_block_summary=True, fuse_block_accumulation=True,
                            fuse_accumulate_read=True)
    hidden, loss = lm_step(model, t["idx"], t["targets"])
    assert oracle_kernels["fwd"] > 0 and oracle_kernels["bwd"] == oracle_kernels["fwd"]
    assert torch.equal(hidden, t["hidden"])
    assert torch.equal(loss.reshape(1), t["loss"])
    for pname, p in model.named_parameters():
        assert torch.equal(p.grad, t[f"grad.{pname}"]), pname


def _small_decoder(ops_cls, fuse_read):
    cfg = AD.DecoderConfig(n_layer=3, n_head=4, n_embd=256, mlp_hidden_dim=256, vocab_size=128, block_size=24,
                           attnres_num_blocks=2, lrid_rank=32, attn_res_query_init="normal",
                           fuse_accumulate_read=fuse_read)
    torch.manual_seed(3)
    return AD.Decoder(cfg, ops=ops_cls).to(torch.bfloat16)


def test_fused_read_under_autograd_grad_over_parameters(oracle_kernels):
    """Warmup-style ``torch.autograd.grad`` over the body's input and every
    parameter with an arbitrary output gradient, repeated, then an ordinary
    step: the gradients equal the composed path's."""
    fused, split = _small_decoder(_FusedOps, True), _small_decoder(OracleOps, False)
    split.load_state_dict(fused.state_dict())
    idx = torch.randint(0, 128, (2, 24), generator=torch.Generator().manual_seed(4))
    res = []
    for model in (fused, split):
        x0 = model.transformer.wte(idx).detach().requires_grad_(True)
        params = tuple(model.parameters())
        g_h = torch.randn(2, 24, 256, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
        got = []
        for _ in range(3):
            h = model._forward_block_lrid(x0)
            got.append(torch.autograd.grad((h,), (x0,) + params, (g_h,), allow_unused=True))
        res.append(got)
    assert oracle_kernels["fwd"] == oracle_kernels["bwd"] > 0
    for got_f, got_s in zip(*res):
        for a, b in zip(got_f, got_s):
            assert (a is None) == (b is None)
            if a is not None:
                assert torch.equal(a, b)


def test_fused_read_leaves_no_graph_behind(oracle_kernels):
    """After a step, nothing of its autograd graph survives: the op's outputs
    (and through their grad_fn the parameters' gradient accumulators, which
    carry the stream they were made on) must die with the step.  A forward
    that kept its outputs on ctx held every step's graph alive, so a later
    HIP-graph capture met accumulators of an eager step on another stream."""
    model = _small_decoder(_FusedOps, True)
    idx = torch.randint(0, 128, (2, 24), generator=torch.Generator().manual_seed(6))
    seen = []
    real = ops._AccumReadFn.apply

    def spy(*a):
        out = real(*a)
        seen.append(weakref.ref(out[0]))
        return out

    ops._AccumReadFn.apply = spy
    try:
        x0 = model.transformer.wte(idx).detach().requires_grad_(True)
        h = model._forward_block_lrid(x0)
        h.float().square().mean().backward()
        del h, x0
    finally:
        ops._AccumReadFn.apply = real
    assert seen
    assert all(r() is None for r in seen)
