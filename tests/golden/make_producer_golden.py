"""Write key-producer golden vectors (tests/golden/prod_*.safetensors) from the reference's model modules.

Run in the build container only (it needs ``/root/reference``, which does not
exist on the GPU box)::

    python tests/golden/make_producer_golden.py [--reference /root/reference]

It imports the reference's ``model`` module and runs two of its key producers on
small seeded inputs, forward and backward, on the CPU:

* ``LRIDSourceKeyProjection`` (``model.py:391-428``) with ``lrid_key_from_value``:
  ``proj(norm(x))`` with ``lrid_key_value_norm`` (``:412-415, 418-419``), or
  ``proj(x)`` without it, and no key norm on this path (``:408``).  The module is
  applied once per source, as the model applies it to every source
  (``model.py:2030-2033``), so the weight gradient is autograd's sum over the
  sources.
* the shared static source key: ``LRIDStaticKey`` (``model.py:275-289``, one
  ``[rank]`` parameter) added by ``OBPM._add_static_lrid_source_key``
  (``model.py:2046-2049``) to every source key except the embedding's
  (``_lrid_source(add_static_key=True)``, ``:2062-2063``; the embedding source
  ``:2070-2078`` does not add it), followed by the reference's eager LR read
  (``attnres_ops.lrid_attention_residual_read_torch``, ``attnres_ops.py:4235``).
  The fixture holds the keys with the static key added, the read's output and
  the gradients of the raw keys, the values, the query and the fp32 static-key
  parameter.

Only data is written (safetensors + a JSON index); no reference source is
copied.  The generator is deterministic for a given torch version.
"""

from __future__ import annotations

import argparse
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))

DT = {"fp32": torch.float32, "bf16": torch.bfloat16}

# value-key projection cases: name, seed, dtype, value_norm, (N, B, T, D, R)
VKEY_CASES = [
    ("prod_vkey_fp32_norm", 701, "fp32", True, (3, 2, 5, 32, 8)),
    ("prod_vkey_bf16_norm", 702, "bf16", True, (3, 2, 5, 32, 8)),
    ("prod_vkey_bf16_nonorm", 703, "bf16", False, (4, 1, 6, 48, 16)),
    ("prod_vkey_fp32_nonorm", 704, "fp32", False, (2, 2, 3, 24, 8)),
]

# static source key cases: name, seed, key/value dtype, (N, B, T, D, R, H), key_norm
STATIC_CASES = [
    ("prod_static_bf16", 711, "bf16", (5, 2, 4, 32, 16, 2), True),
    ("prod_static_fp32", 712, "fp32", (4, 1, 6, 16, 8, 1), True),
    ("prod_static_bf16_nokn", 713, "bf16", (3, 2, 3, 16, 8, 2), False),
]


def _randn(gen, shape, dtype, std=1.0):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(dtype)


def _config(model_mod, **kw):
    base = dict(n_layer=2, n_head=2, n_embd=32, mlp_hidden_dim=32, vocab_size=37, block_size=8,
                use_attnres=True, use_lrid=True)
    base.update(kw)
    return model_mod.ModelConfig(**base)


def vkey_case(model_mod, seed, dtype, value_norm, shape):
    N, B, T, D, R = shape
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    cfg = _config(model_mod, n_embd=D, lrid_rank=R, lrid_key_from_value=True, lrid_key_value_norm=value_norm)
    mod = model_mod.LRIDSourceKeyProjection(cfg)
    assert not mod.use_key_norm and mod.use_value_norm == value_norm
    with torch.no_grad():
        mod.proj.weight.copy_(_randn(gen, (R, D), torch.float32, 0.2))
    mod.to(dtype=dt)
    xs = _randn(gen, (N, B, T, D), dt)
    gs = _randn(gen, (N, B, T, R), dt)
    x = xs.clone().requires_grad_(True)
    keys = [mod(x[s]) for s in range(N)]  # one call per source, as the model does
    loss = sum((k.float() * g.float()).sum() for k, g in zip(keys, gs))
    loss.backward()
    tensors = {"values": xs, "weight": mod.proj.weight.detach().clone(), "grad_keys": gs,
               "keys": torch.stack([k.detach() for k in keys]), "dvalues": x.grad.detach().clone(),
               "dweight": mod.proj.weight.grad.detach().clone()}
    meta = dict(kind="value_key", dtype=dtype, value_norm=value_norm, N=N, B=B, T=T, D=D, R=R, seed=seed)
    return tensors, meta


class _StaticKeyOwner:
    """The two attributes ``OBPM._add_static_lrid_source_key`` reads: its
    config and ``transformer.lrid_static_source_key``."""

    def __init__(self, cfg, static):
        self.config = cfg
        self.transformer = torch.nn.Module()
        self.transformer.lrid_static_source_key = static


def static_case(model_mod, ops_mod, seed, dtype, shape, key_norm):
    N, B, T, D, R, H = shape
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    cfg = _config(model_mod, n_embd=D, lrid_rank=R, lrid_num_heads=H, lrid_add_static_source_key=True)
    static = model_mod.LRIDStaticKey(cfg)  # fp32 parameter, cast to the key dtype in its forward
    with torch.no_grad():
        static.key.copy_(_randn(gen, (R,), torch.float32, 0.5))
    owner = _StaticKeyOwner(cfg, static)
    values = _randn(gen, (N, B, T, D), dt)
    keys = _randn(gen, (N, B, T, R), dt)
    query = _randn(gen, (H, R // H), torch.float32, 0.5)
    g = _randn(gen, (B, T, D), dt)
    scale = 1.0 / (R // H) ** 0.5
    v = values.clone().requires_grad_(True)
    k = keys.clone().requires_grad_(True)
    q = query.clone().requires_grad_(True)
    # the embedding source keeps its key; every other source gets the static key
    keyed = [k[0]] + [model_mod.OBPM._add_static_lrid_source_key(owner, k[s]) for s in range(1, N)]
    out = ops_mod.lrid_attention_residual_read_torch(list(v.unbind(0)), keyed, q, H, scale, key_norm)
    out.backward(g)
    tensors = {"values": values, "keys": keys, "query": query, "grad_out": g,
               "static_key": static.key.detach().clone(),
               "keys_with_static": torch.stack([x.detach() for x in keyed]), "out": out.detach(),
               "dvalues": v.grad.detach().clone(), "dkeys": k.grad.detach().clone(), "dquery": q.grad.detach().clone(),
               "dstatic_key": static.key.grad.detach().clone()}
    meta = dict(kind="static_key", dtype=dtype, N=N, B=B, T=T, D=D, R=R, H=H, scale=scale, key_norm=key_norm,
                seed=seed)
    return tensors, meta


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import attnres_ops as ops_mod  # the reference's op module (eager CPU functions)
    import model as model_mod  # the reference's model.py

    index = {}
    for name, seed, dtype, value_norm, shape in VKEY_CASES:
        tensors, meta = vkey_case(model_mod, seed, dtype, value_norm, shape)
        meta["torch"] = torch.__version__
        save_file({k: t.contiguous() for k, t in tensors.items()}, os.path.join(HERE, f"{name}.safetensors"))
        index[name] = meta
    for name, seed, dtype, shape, key_norm in STATIC_CASES:
        tensors, meta = static_case(model_mod, ops_mod, seed, dtype, shape, key_norm)
        meta["torch"] = torch.__version__
        save_file({k: t.contiguous() for k, t in tensors.items()}, os.path.join(HERE, f"{name}.safetensors"))
        index[name] = meta
    with open(os.path.join(HERE, "producer_index.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)
    print(f"wrote {len(index)} key-producer cases to {HERE}")


if __name__ == "__main__":
    main()
