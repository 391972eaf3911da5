"""Write the golden vectors in tests/golden/*.safetensors from the reference's eager op.

Run in the build container only (it needs ``/root/reference``, which does not
exist on the GPU box)::

    python tests/golden/make_golden.py [--reference /root/reference]

It imports the reference's ``attnres_ops`` module and calls its *eager* CPU
functions -- ``lrid_attention_residual_read_torch`` (attnres_ops.py:4235),
``attention_residual_read_torch`` (:2217), ``attention_residual_average_read``
(:2568, eager branch on CPU), ``attention_residual_phase1_from_logits``
(:3910, eager branch on CPU), ``attention_residual_phase2_torch`` and
``lrid_attention_residual_phase2_torch`` (:4142) -- on small seeded inputs,
runs autograd with a seeded upstream gradient, and stores inputs, outputs and
gradients.  These vectors pin the one thing the math checks cannot: the exact
bf16/fp16 rounding sequence of the reference's eager op.

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

DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def _randn(gen, shape, dtype, std=1.0):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(dtype)


def lr_case(ref, name, seed, dtype, B, T, D, S, R, H, scale, key_norm, bias=None, counts=None,
            dynamic=False, normalize_output=False):
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    values = _randn(gen, (S, B, T, D), dt)
    keys = _randn(gen, (S, B, T, R), dt)
    if dynamic:
        query = _randn(gen, (B, T, H, R // H), torch.float32, 0.5)
    else:
        query = _randn(gen, (H, R // H), torch.float32, 0.5)
    g = _randn(gen, (B, T, D), dt)
    tensors = {"values": values, "keys": keys, "query": query, "grad_out": g}
    v = values.clone().requires_grad_(True)
    k = keys.clone().requires_grad_(True)
    q = query.clone().requires_grad_(True)
    kwargs = {}
    b = None
    if bias is not None:
        b = torch.tensor(bias, dtype=torch.float32).requires_grad_(True)
        kwargs["source_logit_biases"] = b
        tensors["bias"] = torch.tensor(bias, dtype=torch.float32)
    if counts is not None:
        kwargs["source_counts"] = list(counts)
        tensors["counts"] = torch.tensor(counts, dtype=torch.float32)
    out = ref.lrid_attention_residual_read_torch(list(v.unbind(0)), list(k.unbind(0)), q.to(dt), H, scale,
                                                 key_norm, **kwargs)
    if normalize_output:
        out = ref._norm(out)
    out.backward(g)
    tensors.update(out=out.detach(), dvalues=v.grad, dkeys=k.grad, dquery=q.grad)
    if b is not None:
        tensors["dbias"] = b.grad
    meta = dict(kind="lr", dtype=dtype, B=B, T=T, D=D, S=S, R=R, H=H, scale=scale, key_norm=key_norm,
                dynamic=dynamic, normalize_output=normalize_output, has_bias=bias is not None,
                has_counts=counts is not None, seed=seed)
    return name, tensors, meta


def base_case(ref, name, seed, dtype, B, T, D, S, key_norm, counts=None, bias=None, normalize_output=False,
              qstd=0.5):
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    values = _randn(gen, (S, B, T, D), dt)
    query = _randn(gen, (D,), torch.float32, qstd)
    g = _randn(gen, (B, T, D), dt)
    tensors = {"values": values, "query": query, "grad_out": g}
    v = values.clone().requires_grad_(True)
    q = query.clone().requires_grad_(True)
    kwargs = {}
    b = None
    if counts is not None:
        kwargs["source_counts"] = list(counts)
        tensors["counts"] = torch.tensor(counts, dtype=torch.float32)
    if bias is not None:
        b = torch.tensor(bias, dtype=torch.float32).requires_grad_(True)
        kwargs["source_logit_biases"] = b
        tensors["bias"] = torch.tensor(bias, dtype=torch.float32)
    out = ref.attention_residual_read_torch(list(v.unbind(0)), q.to(dt), key_norm, **kwargs)
    if normalize_output:
        out = ref._norm(out)
    out.backward(g)
    tensors.update(out=out.detach(), dvalues=v.grad, dquery=q.grad)
    if b is not None:
        tensors["dbias"] = b.grad
    meta = dict(kind="base", dtype=dtype, B=B, T=T, D=D, S=S, key_norm=key_norm, normalize_output=normalize_output,
                has_bias=bias is not None, has_counts=counts is not None, seed=seed)
    return name, tensors, meta


def average_case(ref, name, seed, dtype, B, T, D, S, normalize_output):
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    values = _randn(gen, (S, B, T, D), dt)
    out = ref.attention_residual_average_read(list(values.unbind(0)), normalize_output=normalize_output)
    meta = dict(kind="average", dtype=dtype, B=B, T=T, D=D, S=S, normalize_output=normalize_output, seed=seed)
    return name, {"values": values, "out": out}, meta


def phase_case(ref, name, seed, dtype, B, T, D, S, Q):
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    values = _randn(gen, (S, B, T, D), dt)
    logits = _randn(gen, (Q, S, B, T), torch.float32)
    out, lse = ref.attention_residual_phase1_from_logits(values, logits)
    partial = _randn(gen, (B, T, D), dt)
    query = _randn(gen, (D,), dt, 0.5)
    p2 = ref.attention_residual_phase2_torch(partial, query, out[0], lse[0], True)
    pkey = _randn(gen, (B, T, 16), dt)
    lq = _randn(gen, (1, 16), dt, 0.5)
    lp2 = ref.lrid_attention_residual_phase2_torch(partial, pkey, lq, out[0], lse[0], 0.25, True)
    meta = dict(kind="phase", dtype=dtype, B=B, T=T, D=D, S=S, Q=Q, seed=seed)
    return name, {"values": values, "logits": logits, "out": out, "lse": lse, "partial": partial,
                  "query": query, "phase2_out": p2, "partial_key": pkey, "lrid_query": lq,
                  "lrid_phase2_out": lp2}, meta


def phase1_case(ref, name, seed, dtype, logits_dtype, B, T, D, S, Q, normalize_output):
    """``attention_residual_phase1_from_logits`` (eager branch) with its gradients."""
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    values = _randn(gen, (S, B, T, D), dt)
    logits = _randn(gen, (Q, S, B, T), DT[logits_dtype], 1.5)
    g = _randn(gen, (Q, B, T, D), dt)
    glse = _randn(gen, (Q, B, T), torch.float32)
    v = values.clone().requires_grad_(True)
    lg = logits.clone().requires_grad_(True)
    out, lse = ref.attention_residual_phase1_from_logits(v, lg, normalize_output=normalize_output)
    torch.autograd.backward([out, lse], [g, glse])
    meta = dict(kind="phase1", dtype=dtype, logits_dtype=logits_dtype, B=B, T=T, D=D, S=S, Q=Q,
                normalize_output=normalize_output, seed=seed)
    return name, {"values": values, "logits": logits, "grad_out": g, "grad_lse": glse, "out": out.detach(),
                  "lse": lse.detach(), "dvalues": v.grad, "dlogits": lg.grad}, meta


def phase2_case(ref, name, seed, dtype, B, T, D, variant, key_norm=True, bias=None, bias_tensor=False,
                normalize_output=False, R=16, scale=0.25):
    """Phase-2 merges with gradients.

    variant: "base" = ``attention_residual_phase2_torch`` (:4023),
    "lrid" = ``lrid_attention_residual_phase2_torch`` (:4142),
    "lrid_addcmul" = ``lrid_attention_residual_phase2`` (:4085; eager on CPU),
    "logit" = ``attention_residual_phase2_from_logit`` (:4041; eager on CPU).
    """
    gen = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    partial = _randn(gen, (B, T, D), dt)
    inter = _randn(gen, (B, T, D), dt)
    lse = _randn(gen, (B, T), torch.float32)
    g = _randn(gen, (B, T, D), dt)
    tensors = {"partial": partial, "inter": inter, "lse": lse, "grad_out": g}
    p = partial.clone().requires_grad_(True)
    it = inter.clone().requires_grad_(True)
    ls = lse.clone().requires_grad_(True)
    b = bias if bias is not None else 0.0
    bt = None
    if bias is not None and bias_tensor:
        bt = torch.tensor(float(bias), dtype=torch.float32).requires_grad_(True)
        b = bt
    if variant == "base":
        query = _randn(gen, (D,), dt, 0.5)
        q = query.clone().requires_grad_(True)
        out = ref.attention_residual_phase2_torch(p, q, it, ls, key_norm, normalize_output=normalize_output,
                                                  logit_bias=b)
        tensors["query"] = query
    elif variant in ("lrid", "lrid_addcmul"):
        pkey = _randn(gen, (B, T, R), dt)
        query = _randn(gen, (1, R), dt, 0.5)
        k = pkey.clone().requires_grad_(True)
        q = query.clone().requires_grad_(True)
        fn = ref.lrid_attention_residual_phase2_torch if variant == "lrid" else ref.lrid_attention_residual_phase2
        out = fn(p, k, q, it, ls, scale, key_norm, normalize_output=normalize_output, logit_bias=b)
        tensors.update(partial_key=pkey, query=query)
    else:
        logit = _randn(gen, (B, T), torch.float32, 2.0)
        q = logit.clone().requires_grad_(True)
        out = ref.attention_residual_phase2_from_logit(p, q, it, ls, normalize_output=normalize_output)
        tensors["logit"] = logit
    out.backward(g)
    tensors.update(out=out.detach(), dpartial=p.grad, dinter=it.grad, dlse=ls.grad)
    if variant == "logit":
        tensors["dlogit"] = q.grad
    else:
        tensors["dquery"] = q.grad
    if variant in ("lrid", "lrid_addcmul"):
        tensors["dpartial_key"] = k.grad
    if bt is not None:
        tensors["dbias"] = bt.grad.reshape(1)
    meta = dict(kind="phase2", variant=variant, dtype=dtype, B=B, T=T, D=D, R=R, scale=scale, key_norm=key_norm,
                bias=0.0 if bias is None else float(bias), bias_tensor=bt is not None,
                normalize_output=normalize_output, seed=seed)
    return name, tensors, meta


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.dont_write_bytecode = True
    sys.path.insert(0, args.reference)
    import attnres_ops as ref  # the reference module, eager CPU paths only

    torch.set_num_threads(1)
    cases = [
        # config-1 shape family (fp32, base, key_norm, q~N(0,0.02)); T cut to 32 to keep the file small
        base_case(ref, "base_c1_fp32", 101, "fp32", 2, 32, 128, 4, True, qstd=0.02),
        base_case(ref, "base_fp32_nokn", 102, "fp32", 2, 5, 64, 5, False),
        base_case(ref, "base_bf16_kn", 103, "bf16", 2, 5, 64, 5, True),
        base_case(ref, "base_bf16_nokn", 104, "bf16", 2, 3, 96, 7, False),
        base_case(ref, "base_bf16_counts", 105, "bf16", 2, 3, 64, 3, True, counts=[1, 3, 2]),
        base_case(ref, "base_fp32_bias", 106, "fp32", 1, 4, 32, 4, True, bias=[0.0, 0.7, -0.3, 1.1]),
        base_case(ref, "base_bf16_normout", 107, "bf16", 1, 4, 128, 6, True, normalize_output=True),
        base_case(ref, "base_fp16_kn", 108, "fp16", 1, 4, 64, 5, True),
        lr_case(ref, "lr_fp32_h2", 201, "fp32", 1, 8, 64, 5, 16, 2, 0.25, True),
        lr_case(ref, "lr_bf16_h2", 202, "bf16", 1, 8, 64, 5, 16, 2, 0.25, True),
        lr_case(ref, "lr_bf16_h4_nokn", 203, "bf16", 2, 4, 64, 6, 32, 4, 0.5, False),
        lr_case(ref, "lr_bf16_bias", 204, "bf16", 1, 8, 64, 5, 16, 2, 0.25, True,
                bias=[0.0, 0.693, -0.5, 1.2, 0.1]),
        lr_case(ref, "lr_bf16_counts", 205, "bf16", 1, 8, 64, 5, 16, 2, 0.25, True, counts=[1, 2, 3, 4, 2]),
        lr_case(ref, "lr_fp32_dyn", 206, "fp32", 2, 3, 64, 4, 16, 2, 0.5, True, dynamic=True),
        lr_case(ref, "lr_bf16_dyn", 207, "bf16", 2, 3, 64, 4, 16, 2, 0.5, True, dynamic=True),
        lr_case(ref, "lr_fp16_h1", 208, "fp16", 1, 6, 32, 4, 16, 1, 0.25, True),
        lr_case(ref, "lr_bf16_normout", 209, "bf16", 1, 6, 128, 5, 32, 1, 0.125, True, normalize_output=True),
        lr_case(ref, "lr_bf16_c3_slice", 210, "bf16", 1, 4, 1024, 13, 64, 4, 0.25, True),
        average_case(ref, "avg_bf16", 301, "bf16", 2, 3, 64, 5, False),
        average_case(ref, "avg_fp32_norm", 302, "fp32", 1, 4, 32, 3, True),
        phase_case(ref, "phase_fp32", 401, "fp32", 2, 3, 32, 4, 3),
        phase1_case(ref, "p1_fp32", 411, "fp32", "fp32", 2, 3, 32, 4, 3, False),
        phase1_case(ref, "p1_bf16_f32logits", 412, "bf16", "fp32", 2, 3, 64, 5, 4, False),
        phase1_case(ref, "p1_bf16_bf16logits", 413, "bf16", "bf16", 1, 4, 64, 3, 2, False),
        phase1_case(ref, "p1_bf16_normout", 414, "bf16", "fp32", 1, 4, 128, 6, 3, True),
        phase1_case(ref, "p1_fp16", 415, "fp16", "fp32", 1, 3, 64, 4, 5, False),
        phase2_case(ref, "p2_base_bf16_kn", 421, "bf16", 2, 3, 64, "base"),
        phase2_case(ref, "p2_base_bf16_nokn_bias", 422, "bf16", 1, 4, 64, "base", key_norm=False, bias=0.693),
        phase2_case(ref, "p2_base_fp32_tbias_norm", 423, "fp32", 1, 4, 32, "base", bias=0.4, bias_tensor=True,
                    normalize_output=True),
        phase2_case(ref, "p2_base_bf16_tbias", 424, "bf16", 2, 3, 64, "base", bias=1.1, bias_tensor=True),
        phase2_case(ref, "p2_lrid_bf16", 431, "bf16", 2, 3, 64, "lrid"),
        phase2_case(ref, "p2_lrid_bf16_bias_norm", 432, "bf16", 1, 4, 128, "lrid", bias=0.693, bias_tensor=True,
                    normalize_output=True, R=32, scale=0.125),
        phase2_case(ref, "p2_lrid_fp32_nokn", 433, "fp32", 1, 4, 32, "lrid", key_norm=False),
        phase2_case(ref, "p2_lridadd_bf16", 434, "bf16", 2, 3, 64, "lrid_addcmul"),
        phase2_case(ref, "p2_lridadd_bf16_bias", 435, "bf16", 1, 4, 64, "lrid_addcmul", bias=0.5),
        phase2_case(ref, "p2_logit_bf16", 441, "bf16", 2, 3, 64, "logit"),
        phase2_case(ref, "p2_logit_fp16_norm", 442, "fp16", 1, 4, 64, "logit", normalize_output=True),
    ]
    index = {}
    for name, tensors, meta in cases:
        tensors = {k: t.detach().contiguous() for k, t in tensors.items()}
        save_file(tensors, os.path.join(HERE, f"{name}.safetensors"))
        meta["torch"] = torch.__version__
        index[name] = meta
    with open(os.path.join(HERE, "index.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)
    print(f"wrote {len(index)} golden cases to {HERE}")


if __name__ == "__main__":
    main()
