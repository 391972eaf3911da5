"""The oracle's key producers reproduce the reference model's own modules on their golden vectors.

The vectors come from the reference's ``LRIDSourceKeyProjection``
(``model.py:391-428``, with ``lrid_key_from_value``) and from its shared static
source key (``LRIDStaticKey`` ``model.py:275-289`` added by
``OBPM._add_static_lrid_source_key`` ``:2046-2049`` to every source but the
embedding) followed by the reference's eager LR read
(tests/golden/make_producer_golden.py).  On the same torch build every output
and gradient must agree bit for bit; the fp32 static-key parameter's gradient,
a sum over the sources in fp32 whose order autograd picks, within 1e-6.
"""

import pytest
import torch

from oracle import attnres_oracle as O
from _golden import load_producer, producer_names

DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


@pytest.fixture(autouse=True)
def _one_thread():
    # the vectors were written with one intra-op thread (fixed reduction order)
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


def _same(a, b, dtype):
    if torch.equal(a, b):
        return
    tol = {"fp32": 1e-6, "bf16": 8e-3}[dtype]  # another torch build: one storage ulp
    torch.testing.assert_close(a.float(), b.float(), rtol=tol, atol=tol)


def test_producer_vectors_present():
    assert len(producer_names("value_key")) >= 4 and len(producer_names("static_key")) >= 3


@pytest.mark.parametrize("name", producer_names("value_key"))
def test_value_key_projection_matches_reference_module(name):
    t, m = load_producer(name)
    x = t["values"].clone().requires_grad_(True)
    w = t["weight"].clone().requires_grad_(True)
    keys = O.lrid_value_key_projection_ref(list(x.unbind(0)), w, m["value_norm"])
    # one backward through all sources, as the vectors were written: autograd
    # then sums the per-source bf16 weight gradients in its own order
    sum((k.float() * g.float()).sum() for k, g in zip(keys, t["grad_keys"].unbind(0))).backward()
    _same(torch.stack([k.detach() for k in keys]), t["keys"], m["dtype"])
    _same(x.grad, t["dvalues"], m["dtype"])
    _same(w.grad, t["dweight"], m["dtype"])


@pytest.mark.parametrize("name", producer_names("value_key"))
def test_value_key_projection_pin_catches_a_key_norm(name):
    """A per-head key norm after the projection (what the fused projection does,
    model.py:376-377, but this path must not, :408) changes the keys."""
    t, m = load_producer(name)
    keys = O.lrid_value_key_projection_ref(list(t["values"].unbind(0)), t["weight"], m["value_norm"])
    normed = torch.stack([O.norm(k) for k in keys])
    assert not torch.equal(normed, t["keys"])


@pytest.mark.parametrize("name", producer_names("static_key"))
def test_shared_static_key_matches_reference_model(name):
    t, m = load_producer(name)
    dt = DT[m["dtype"]]
    N = m["N"]
    v = t["values"].clone().requires_grad_(True)
    k = t["keys"].clone().requires_grad_(True)
    q = t["query"].clone().requires_grad_(True)
    p = t["static_key"].clone().requires_grad_(True)  # the model's fp32 parameter
    table = O.shared_static_key_table_ref(p, N, dt)
    keyed = O.static_key_add_ref(list(k.unbind(0)), table)
    _same(torch.stack([x.detach() for x in keyed]), t["keys_with_static"], m["dtype"])
    out = O.lrid_attention_residual_read_torch(list(v.unbind(0)), keyed, q.to(dt), m["H"], m["scale"],
                                               m["key_norm"])
    out.backward(t["grad_out"])
    _same(out.detach(), t["out"], m["dtype"])
    _same(v.grad, t["dvalues"], m["dtype"])
    _same(k.grad, t["dkeys"], m["dtype"])
    _same(q.grad, t["dquery"], "fp32")
    torch.testing.assert_close(p.grad, t["dstatic_key"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", producer_names("static_key"))
def test_static_key_pin_catches_the_embedding_row(name):
    """Adding the static key to the embedding source too (a plausible slip:
    the model skips it there) is caught by the vectors."""
    t, m = load_producer(name)
    dt = DT[m["dtype"]]
    p = t["static_key"]
    everywhere = torch.stack([p.to(dt)] * m["N"])
    keyed = O.static_key_add_ref(list(t["keys"].unbind(0)), everywhere)
    assert not torch.equal(torch.stack(keyed), t["keys_with_static"])


@pytest.mark.parametrize("name", producer_names("static_key"))
def test_static_key_pin_catches_the_rounding_point(name):
    """Adding the fp32 key before rounding (key.float() + static, one rounding)
    instead of the model's add in the key dtype differs in bf16."""
    t, m = load_producer(name)
    if m["dtype"] == "fp32":
        pytest.skip("one rounding either way in fp32")
    dt = DT[m["dtype"]]
    ks = t["keys"].unbind(0)
    late = [ks[0]] + [(ks[s].float() + t["static_key"]).to(dt) for s in range(1, m["N"])]
    other = torch.stack([(ks[s].float() + t["static_key"].to(dt).float()).to(dt) for s in range(1, m["N"])])
    ref = t["keys_with_static"][1:]
    assert torch.equal(other, ref)  # the reference's rounding: both operands in the dtype, one rounding of the sum
    assert not torch.equal(torch.stack(late[1:]), ref)
