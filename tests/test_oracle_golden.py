"""The eager oracle reproduces the reference's own eager op on its golden vectors.

The vectors come from the reference's eager functions (see
tests/golden/make_golden.py); the oracle restates them, so forward outputs and
every gradient must agree bit for bit on the same torch build, and to a few
ulps of the storage dtype on another one.
"""

import pytest
import torch

from oracle import attnres_oracle as O
from _golden import load, names

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.fixture(autouse=True)
def _one_thread():
    # the vectors were written with one intra-op thread; fp32 reductions
    # (e.g. dquery over all tokens) are only bit-exact with the same order
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


def _close(a, b, dtype):
    # same torch build -> bit-exact; other builds -> one storage ulp
    if torch.equal(a, b):
        return
    tol = {"fp32": 1e-6, "bf16": 8e-3, "fp16": 1e-3}[dtype]
    torch.testing.assert_close(a.float(), b.float(), rtol=tol, atol=tol)


@pytest.mark.parametrize("name", names("lr"))
def test_lr_oracle_matches_reference_vectors(name):
    t, m = load(name)
    dt = DT[m["dtype"]]
    v = t["values"].clone().requires_grad_(True)
    k = t["keys"].clone().requires_grad_(True)
    q = t["query"].clone().requires_grad_(True)
    kw = {}
    b = None
    if m["has_bias"]:
        b = t["bias"].clone().requires_grad_(True)
        kw["source_logit_biases"] = b
    if m["has_counts"]:
        kw["source_counts"] = t["counts"].tolist()
    out = O.lrid_attention_residual_read_torch(list(v.unbind(0)), list(k.unbind(0)), q.to(dt), m["H"],
                                               m["scale"], m["key_norm"], **kw)
    if m["normalize_output"]:
        out = O.norm(out)
    out.backward(t["grad_out"])
    _close(out.detach(), t["out"], m["dtype"])
    _close(v.grad, t["dvalues"], m["dtype"])
    _close(k.grad, t["dkeys"], m["dtype"])
    _close(q.grad, t["dquery"], "fp32" if m["dtype"] == "fp32" else m["dtype"])
    if b is not None:
        _close(b.grad, t["dbias"], "fp32")


@pytest.mark.parametrize("name", names("base"))
def test_base_oracle_matches_reference_vectors(name):
    t, m = load(name)
    dt = DT[m["dtype"]]
    v = t["values"].clone().requires_grad_(True)
    q = t["query"].clone().requires_grad_(True)
    kw = {}
    b = None
    if m["has_bias"]:
        b = t["bias"].clone().requires_grad_(True)
        kw["source_logit_biases"] = b
    if m["has_counts"]:
        kw["source_counts"] = t["counts"].tolist()
    out = O.attention_residual_read_torch(list(v.unbind(0)), q.to(dt), m["key_norm"], **kw)
    if m["normalize_output"]:
        out = O.norm(out)
    out.backward(t["grad_out"])
    _close(out.detach(), t["out"], m["dtype"])
    _close(v.grad, t["dvalues"], m["dtype"])
    _close(q.grad, t["dquery"], m["dtype"])
    if b is not None:
        _close(b.grad, t["dbias"], "fp32")


@pytest.mark.parametrize("name", names("average"))
def test_average_oracle_matches_reference_vectors(name):
    t, m = load(name)
    out = O.attention_residual_average_read_ref(list(t["values"].unbind(0)), m["normalize_output"])
    _close(out, t["out"], m["dtype"])


@pytest.mark.parametrize("name", names("phase"))
def test_phase_oracle_matches_reference_vectors(name):
    t, m = load(name)
    out, lse = O.phase1_from_logits_ref(t["values"], t["logits"])
    _close(out, t["out"], m["dtype"])
    _close(lse, t["lse"], "fp32")
    p2 = O.attention_residual_phase2_ref(t["partial"], t["query"], out[0], lse[0], True)
    _close(p2, t["phase2_out"], m["dtype"])
    lp2 = O.lrid_attention_residual_phase2_ref(t["partial"], t["partial_key"], t["lrid_query"], out[0], lse[0],
                                               0.25, True)
    _close(lp2, t["lrid_phase2_out"], m["dtype"])


def _phase2_oracle(t, m, dev="cpu"):
    """Run the oracle's phase-2 merge on a golden case; returns (out, grads dict)."""
    p = t["partial"].to(dev).clone().requires_grad_(True)
    it = t["inter"].to(dev).clone().requires_grad_(True)
    ls = t["lse"].to(dev).clone().requires_grad_(True)
    bias = m["bias"]
    bt = None
    if m["bias_tensor"] and m["variant"] != "logit":
        bt = torch.tensor(bias, dtype=torch.float32, device=dev).requires_grad_(True)
        bias = bt
    grads = {}
    if m["variant"] == "base":
        q = t["query"].to(dev).clone().requires_grad_(True)
        out = O.attention_residual_phase2_ref(p, q, it, ls, m["key_norm"], logit_bias=bias,
                                              normalize_output=m["normalize_output"])
    elif m["variant"] in ("lrid", "lrid_addcmul"):
        k = t["partial_key"].to(dev).clone().requires_grad_(True)
        q = t["query"].to(dev).clone().requires_grad_(True)
        out = O.lrid_attention_residual_phase2_ref(p, k, q, it, ls, m["scale"], m["key_norm"],
                                                   normalize_output=m["normalize_output"], logit_bias=bias,
                                                   merge="lerp" if m["variant"] == "lrid" else "addcmul")
    else:
        q = t["logit"].to(dev).clone().requires_grad_(True)
        out = O.phase2_from_logit_ref(p, q, it, ls, normalize_output=m["normalize_output"])
    out.backward(t["grad_out"].to(dev))
    grads.update(dpartial=p.grad, dinter=it.grad, dlse=ls.grad)
    grads["dlogit" if m["variant"] == "logit" else "dquery"] = q.grad
    if m["variant"] in ("lrid", "lrid_addcmul"):
        grads["dpartial_key"] = k.grad
    if bt is not None:
        grads["dbias"] = bt.grad.reshape(1)
    return out.detach(), grads


@pytest.mark.parametrize("name", names("phase1"))
def test_phase1_oracle_matches_reference_vectors(name):
    t, m = load(name)
    v = t["values"].clone().requires_grad_(True)
    lg = t["logits"].clone().requires_grad_(True)
    out, lse = O.phase1_from_logits_ref(v, lg, normalize_output=m["normalize_output"])
    torch.autograd.backward([out, lse], [t["grad_out"], t["grad_lse"]])
    _close(out.detach(), t["out"], m["dtype"])
    _close(lse.detach(), t["lse"], "fp32")
    _close(v.grad, t["dvalues"], m["dtype"])
    _close(lg.grad, t["dlogits"], m["logits_dtype"])


@pytest.mark.parametrize("name", names("phase2"))
def test_phase2_oracle_matches_reference_vectors(name):
    t, m = load(name)
    out, grads = _phase2_oracle(t, m)
    _close(out, t["out"], m["dtype"])
    for key, g in grads.items():
        ref_dtype = "fp32" if key in ("dlse", "dbias", "dlogit") else m["dtype"]
        _close(g, t[key], ref_dtype)
