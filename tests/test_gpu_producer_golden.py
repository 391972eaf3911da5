"""GPU parity of the key producers against vectors written by the reference model's own modules.

* ``lrid_value_key_projection`` (one HIP rms-norm pass + one library GEMM over
  all sources) against ``LRIDSourceKeyProjection`` with ``lrid_key_from_value``
  (``model.py:391-428``), value norm on and off, fp32 and bf16: keys, value
  gradients and the weight gradient.  The weight gradient here is one GEMM over
  every source's rows (fp32 accumulation, one rounding); the model's autograd
  rounds each source's ``nn.Linear`` weight gradient to the dtype and adds
  them in the dtype, so that gradient is held to the bounds relative to
  ``max(1, max|e|)`` (the cross-token sums' bound).
* the LR read with ``static_keys`` set up as the reference model has it -- one
  shared fp32 ``[R]`` parameter (``LRIDStaticKey``, ``model.py:275-289``),
  added to every source key but the embedding's (``model.py:2046-2049,
  2062-2063, 2070-2078``): a table whose row 0 is zero and whose other rows
  are the parameter cast to the key dtype.  Output, value / key / query
  gradients and the fp32 parameter's gradient (the per-row gradients the read
  returns, summed back by autograd) against the model's.

Vectors: tests/golden/make_producer_golden.py.
"""

import pytest
import torch

import _attnres_hip as H
import attnres_ops as ops
from _golden import load_producer, producer_names
from gpu_util import DEV, assert_close, leaf

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


@pytest.mark.parametrize("name", producer_names("value_key"))
def test_value_key_projection_matches_reference_vectors(name):
    t, m = load_producer(name)
    dt = DT[m["dtype"]]
    xd = [leaf(x) for x in t["values"].unbind(0)]
    wd = leaf(t["weight"])
    keys = ops.lrid_value_key_projection(xd, wd, m["value_norm"])
    torch.autograd.backward(keys, [g.to(DEV) for g in t["grad_keys"].unbind(0)])
    for s in range(m["N"]):
        assert_close(keys[s], t["keys"][s], dt, f"key{s}")
        assert_close(xd[s].grad, t["dvalues"][s], dt, f"dv{s}")
    assert_close(wd.grad, t["dweight"], dt, "dW", reduced=True)


@pytest.mark.parametrize("name", producer_names("static_key"))
def test_read_with_the_models_shared_static_key(name):
    t, m = load_producer(name)
    dt = DT[m["dtype"]]
    N = m["N"]
    vd = [leaf(x) for x in t["values"].unbind(0)]
    kd = [leaf(x) for x in t["keys"].unbind(0)]
    qd = leaf(t["query"])
    pd = leaf(t["static_key"])  # fp32 [R], the model's parameter
    # the model's setup as a per-source table: no static key for the embedding
    # source, the shared key cast to the key dtype (once per source) for the others
    table = torch.stack([torch.zeros_like(pd, dtype=dt)] + [pd.to(dt) for _ in range(N - 1)])
    out = ops.lrid_attention_residual_read(vd, kd, qd, m["H"], m["scale"], m["key_norm"], static_keys=table)
    out.backward(t["grad_out"].to(DEV))
    assert_close(out, t["out"], dt, "out")
    for s in range(N):
        assert_close(vd[s].grad, t["dvalues"][s], dt, f"dv{s}")
        assert_close(kd[s].grad, t["dkeys"][s], dt, f"dk{s}")
    assert_close(qd.grad, t["dquery"], dt, "dq", reduced=True)
    assert_close(pd.grad, t["dstatic_key"], dt, "dstatic_key", reduced=True)
