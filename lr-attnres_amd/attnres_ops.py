"""Drop-in replacement of the reference's ``attnres_ops`` module, backed by HIP kernels for MI355X.

Keeps the reference's public names, argument meaning and error behaviour
(``/root/reference/attnres_ops.py:26-40``), so a model written against it --
``from attnres_ops import lrid_attention_residual_read`` -- runs unchanged when
``lr-attnres_amd`` is on ``sys.path`` instead of the reference.

Every read runs the hand-written gfx950 kernels in ``libattnres_hip.so``
through its C ABI (``include/attnres_hip.h``); there is no Triton, no eager
fallback and no dispatch switch.  Tensors that are not on a ROCm GPU, or a
missing library, raise ``RuntimeError``.  ``force_triton`` is accepted for
signature compatibility and has no effect (the HIP path is the only path).

Autograd goes through ``torch.library.custom_op`` (``attnres_hip::read`` /
``attnres_hip::read_backward``), with fake implementations for
``torch.compile``.  The forward saves the fp32 softmax weights
``[B*T, H, N]``; the backward recomputes nothing from the keys except the key
norm, and reduces cross-token gradients (static query, per-site gate, bias)
deterministically.
"""

from __future__ import annotations

import contextlib
from collections import OrderedDict
from typing import Optional

import torch
from torch import Tensor
from torch.nn import functional as F

import _attnres_hip as _hip

__all__ = [
    "attention_residual_average_read",
    "attention_residual_phase1",
    "attention_residual_phase1_from_logits",
    "attention_residual_phase2",
    "attention_residual_phase2_from_logit",
    "attention_residual_phase2_torch",
    "attention_residual_read",
    "attention_residual_read_torch",
    "is_fused_attnres_available",
    "lrid_attention_residual_phase2",
    "lrid_attention_residual_phase2_torch",
    "lrid_attention_residual_read",
    "lrid_attention_residual_read_gated",
    "lrid_attention_residual_read_torch",
]

_ALLOWED = (torch.float32, torch.bfloat16, torch.float16)


def is_fused_attnres_available() -> bool:
    """True when the HIP library loads and a ROCm GPU is visible (reference: attnres_ops.py:123-124)."""
    return _hip.available()


def _lrid_list_head_dims(values, keys, num_heads: int):
    """(value head width, key head width), or None when ``num_heads`` does not
    split both widths (reference: attnres_ops.py:4319-4330)."""
    try:
        H = int(num_heads)
    except (TypeError, ValueError):
        return None
    if H < 1:
        return None
    D = values[0].size(-1)
    R = keys[0].size(-1)
    if D % H != 0 or R % H != 0:
        return None
    return D // H, R // H


def _lrid_list_dims_within_triton_limits(values, keys, num_heads: int) -> bool:
    """The reference's head-width limits of its direct Triton LR kernel
    (value heads <= 4096, key heads <= 256; attnres_ops.py:4333-4338), kept
    with the same answers because the reference's tests import and assert it
    (tests/test_attnres_ops.py:515-520).  The HIP read here has no such limit:
    wider heads take its general kernels."""
    head_dims = _lrid_list_head_dims(values, keys, num_heads)
    if head_dims is None:
        return False
    value_head_dim, key_head_dim = head_dims
    return value_head_dim <= 4096 and key_head_dim <= 256


# ---------------------------------------------------------------- argument handling

# Logit biases given as host numbers (python floats or lists) become small
# device tensors.  They are cached by value, so repeated calls (every step of a
# training loop) neither copy host data to the device again nor launch kernels
# to build them, and a call inside HIP-graph capture (after an eager warm-up
# call with the same numbers) records no host-to-device copy.  The cached
# tensors are never written.
_HOST_BIAS_CACHE: "OrderedDict[tuple, Tensor]" = OrderedDict()
_HOST_BIAS_CACHE_SIZE = 256


def _host_bias(key, device, make) -> Tensor:
    k = (str(device), key)
    t = _HOST_BIAS_CACHE.get(k)
    if t is None:
        t = make().to(device=device, dtype=torch.float32).contiguous()
        _HOST_BIAS_CACHE[k] = t
        if len(_HOST_BIAS_CACHE) > _HOST_BIAS_CACHE_SIZE:
            _HOST_BIAS_CACHE.popitem(last=False)
    else:
        _HOST_BIAS_CACHE.move_to_end(k)
    return t


def _source_logit_bias(source_counts, source_logit_biases, n_sources: int, device) -> Optional[Tensor]:
    """fp32 [N] logit bias with the reference's rules and errors (attnres_ops.py:65-105)."""
    if source_counts is not None and source_logit_biases is not None:
        raise RuntimeError("source_counts and source_logit_biases are mutually exclusive")
    if source_logit_biases is None:
        if source_counts is None:
            return None
        if isinstance(source_counts, Tensor):
            counts = source_counts.reshape(-1).to(device=device, dtype=torch.float32)
            if counts.numel() != n_sources:
                raise RuntimeError("source_counts length must match the number of sources")
            return counts.log()
        if isinstance(source_counts, (int, float)):
            vals = (float(source_counts),) * n_sources  # (the reference checks only list entries)
        else:
            if len(source_counts) != n_sources:
                raise RuntimeError("source_counts length must match the number of sources")
            vals = tuple(float(c) for c in source_counts)
            if any(c <= 0.0 for c in vals):
                raise RuntimeError("source_counts must be positive")
        # log on the device, as the reference computes it
        return _host_bias(("log_counts", vals), device,
                          lambda: torch.tensor(vals, dtype=torch.float32).to(device).log())
    if isinstance(source_logit_biases, Tensor):
        biases = source_logit_biases.reshape(-1).to(device=device, dtype=torch.float32)
    elif isinstance(source_logit_biases, (int, float)):
        vals = (float(source_logit_biases),) * n_sources
        biases = _host_bias(("bias", vals), device, lambda: torch.tensor(vals, dtype=torch.float32))
    else:
        if len(source_logit_biases) != n_sources:
            raise RuntimeError("source_logit_biases length must match the number of sources")
        if not any(isinstance(b, Tensor) for b in source_logit_biases):
            vals = tuple(float(b) for b in source_logit_biases)
            return _host_bias(("bias", vals), device, lambda: torch.tensor(vals, dtype=torch.float32))
        items = [b.to(device=device, dtype=torch.float32).reshape(()) if isinstance(b, Tensor)
                 else torch.tensor(float(b), device=device, dtype=torch.float32) for b in source_logit_biases]
        biases = torch.stack(items)
    if biases.numel() != n_sources:
        raise RuntimeError("source_logit_biases length must match the number of sources")
    return biases.contiguous()


def _sources(values) -> list:
    if isinstance(values, Tensor):
        if values.dim() != 4:
            raise RuntimeError("stacked sources must be [S, B, T, D]")
        return list(values.unbind(0))
    return list(values)


def _check_gpu(tensors, what):
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(f"{what}: the AttnRes HIP kernels need tensors on a ROCm GPU (got {dev}); "
                           "this build has no CPU path")
    for t in tensors:
        if t.device != dev:
            raise RuntimeError(f"{what}: all tensors must be on {dev} (got {t.device})")
    return dev


def _check_sources(srcs, what):
    if len(srcs) == 0:
        raise RuntimeError(f"{what} requires at least one source")
    if len(srcs) > _hip.MAX_SOURCES:
        raise RuntimeError(f"{what} supports at most {_hip.MAX_SOURCES} sources, got {len(srcs)}")
    first = srcs[0]
    if first.dim() != 3:
        raise RuntimeError(f"{what}: sources must be [B, T, D]")
    for t in srcs:
        if t.shape != first.shape:
            raise RuntimeError(f"{what}: every source must have shape {tuple(first.shape)}, got {tuple(t.shape)}")
        if t.dtype not in _ALLOWED:
            raise RuntimeError(f"{what}: dtype {t.dtype} is not supported (fp32, bf16, fp16)")


def _promote(srcs):
    """Sources of mixed dtypes in their common (promoted) dtype, as the
    reference's eager read stacks them (``_as_stacked``, attnres_ops.py:58-61,
    used at :2224, :3940 and :4246; ``torch.stack`` promotes).  Sources already
    in that dtype are passed as they are."""
    common = srcs[0].dtype
    for t in srcs[1:]:
        common = torch.promote_types(common, t.dtype)
    return [t if t.dtype == common else t.to(common) for t in srcs]


def _norm(x: Tensor) -> Tensor:
    # identity-path output norm for a single source; same op as the reference
    return F.rms_norm(x, (x.size(-1),))


# ---------------------------------------------------------------- the custom ops

def _empty(device):
    return torch.empty((0,), device=device)


@torch.library.custom_op("attnres_hip::read", mutates_args=())
def _read_op(values: list[Tensor], keys: list[Tensor], query: Optional[Tensor], query_dyn: Optional[Tensor],
             gate: Optional[Tensor], bias: Optional[Tensor], static_keys: Optional[Tensor], heads: int,
             logit_scale: float, key_norm: bool, normalize_output: bool, mode: int, gate_act: int,
             gate_per_token: bool, save_weights: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    v0 = values[0]
    B, T, D = v0.shape
    desc = _hip.Desc(values, keys, query, query_dyn, gate, bias, heads, logit_scale, key_norm, normalize_output,
                     mode, gate_act, gate_per_token, static_keys=static_keys)
    with torch.cuda.device(v0.device):
        out, w, inv, pre = _hip.forward(desc, v0.device, v0.dtype, save_weights and mode == _hip.MODE_SOFTMAX,
                                        normalize_output, save_weights)
    return out.view(B, T, D), w, inv, pre


@_read_op.register_fake
def _read_fake(values, keys, query, query_dyn, gate, bias, static_keys, heads, logit_scale, key_norm,
               normalize_output, mode, gate_act, gate_per_token, save_weights):
    v0 = values[0]
    B, T, D = v0.shape
    n_tok = B * T
    out = v0.new_empty((B, T, D))
    w = v0.new_empty((n_tok, heads, len(values)) if save_weights and mode == 0 else (0,), dtype=torch.float32)
    keep = normalize_output and save_weights
    inv = v0.new_empty((n_tok if keep else 0,), dtype=torch.float32)
    pre = v0.new_empty((n_tok, D) if keep else (0,))
    return out, w, inv, pre


@torch.library.custom_op("attnres_hip::read_backward", mutates_args=())
def _read_backward_op(values: list[Tensor], keys: list[Tensor], query: Optional[Tensor], query_dyn: Optional[Tensor],
                      gate: Optional[Tensor], bias: Optional[Tensor], static_keys: Optional[Tensor],
                      grad_out: Tensor, prenorm: Tensor, inv_rms: Tensor, weights: Tensor, heads: int,
                      logit_scale: float, key_norm: bool, normalize_output: bool, mode: int, gate_act: int,
                      gate_per_token: bool) -> tuple[list[Tensor], list[Tensor], Tensor, Tensor, Tensor, Tensor,
                                                     Tensor]:
    v0 = values[0]
    B, T, D = v0.shape
    dev = v0.device
    desc = _hip.Desc(values, keys, query, query_dyn, gate, bias, heads, logit_scale, key_norm, normalize_output,
                     mode, gate_act, gate_per_token, static_keys=static_keys)
    lr = len(keys) > 0
    with torch.cuda.device(dev):
        dvals, dkeys, dq, dqd, dg, db, dsk = _hip.backward(
            desc, dev, v0.dtype, grad_out.contiguous(), prenorm, inv_rms, weights,
            want_dquery=query is not None and mode == _hip.MODE_SOFTMAX,
            want_dgate=gate is not None, want_dbias=bias is not None,
            query_shape=tuple(query.shape) if query is not None else (0,),
            gate_shape=tuple(gate.shape) if gate is not None else (0,), lr=lr,
            has_query_dyn=query_dyn is not None, want_dstatic=static_keys is not None)
    dvals = [t.view(B, T, D) for t in dvals]
    dkeys = [t.view(B, T, keys[0].size(-1)) for t in dkeys]
    # absent gradients are distinct empty tensors (custom-op outputs may not alias)
    return (dvals, dkeys, dq if dq is not None else _empty(dev),
            dqd.view(query_dyn.shape) if dqd is not None else _empty(dev),
            dg if dg is not None else _empty(dev), db if db is not None else _empty(dev),
            dsk.view(static_keys.shape) if dsk is not None else _empty(dev))


@_read_backward_op.register_fake
def _read_backward_fake(values, keys, query, query_dyn, gate, bias, static_keys, grad_out, prenorm, inv_rms, weights,
                        heads, logit_scale, key_norm, normalize_output, mode, gate_act, gate_per_token):
    e = lambda: values[0].new_empty((0,))  # noqa: E731
    return ([v.new_empty(v.shape) for v in values], [k.new_empty(k.shape) for k in keys],
            query.new_empty(query.shape) if query is not None else e(),
            query_dyn.new_empty(query_dyn.shape) if query_dyn is not None else e(),
            gate.new_empty(gate.shape) if gate is not None else e(),
            bias.new_empty(bias.shape) if bias is not None else e(),
            static_keys.new_empty(static_keys.shape) if static_keys is not None else e())


def _read_setup_context(ctx, inputs, output):
    (values, keys, query, query_dyn, gate, bias, static_keys, heads, logit_scale, key_norm, normalize_output, mode,
     gate_act, gate_per_token, save_weights) = inputs
    out, w, inv, pre = output
    ctx.n_values = len(values)
    ctx.n_keys = len(keys)
    ctx.has = (query is not None, query_dyn is not None, gate is not None, bias is not None, static_keys is not None)
    opt = [t for t in (query, query_dyn, gate, bias, static_keys) if t is not None]
    ctx.save_for_backward(*values, *keys, *opt, pre, w, inv)
    ctx.flags = (heads, logit_scale, key_norm, normalize_output, mode, gate_act, gate_per_token)


def _read_backward(ctx, grad_out, grad_w, grad_inv, grad_pre):
    saved = list(ctx.saved_tensors)
    values = saved[:ctx.n_values]
    keys = saved[ctx.n_values:ctx.n_values + ctx.n_keys]
    rest = saved[ctx.n_values + ctx.n_keys:]
    opt = []
    for present in ctx.has:
        opt.append(rest.pop(0) if present else None)
    query, query_dyn, gate, bias, static_keys = opt
    pre, w, inv = rest
    heads, logit_scale, key_norm, normalize_output, mode, gate_act, gate_per_token = ctx.flags
    dvals, dkeys, dq, dqd, dg, db, dsk = _read_backward_op(values, keys, query, query_dyn, gate, bias, static_keys,
                                                           grad_out, pre, inv, w, heads, logit_scale, key_norm,
                                                           normalize_output, mode, gate_act, gate_per_token)
    return (dvals, dkeys,
            dq if query is not None else None, dqd if query_dyn is not None else None,
            dg if gate is not None else None, db if bias is not None else None,
            dsk if static_keys is not None else None,
            None, None, None, None, None, None, None, None)


_read_op.register_autograd(_read_backward, setup_context=_read_setup_context)


# ---------------------------------------------------------------- eager autograd path
#
# Eager calls (no torch.compile tracing) go through torch.autograd.Function
# classes instead of the torch.library ops above: the same C ABI calls on the
# same kernels, without the custom-op layer's per-call cost (schema defaults,
# pytree flattening of the source lists, a second op for the backward).  The
# forward's C descriptor is reused by the backward, and the per-source
# gradients are views of one allocation.  While torch.compile traces, the
# library ops are used, so the compiled graph holds attnres_hip:: ops with
# their fake implementations.

def _compiling() -> bool:
    return torch.compiler.is_compiling()


def _device_ctx(dev):
    """Device guard, skipped when ``dev`` is already the current device."""
    return contextlib.nullcontext() if dev.index == torch.cuda.current_device() else torch.cuda.device(dev)


def _unflatten_opt(has, tensors):
    """Optional tensors back from a flat tuple: ``has`` marks which are present."""
    it = iter(tensors)
    return [next(it) if h else None for h in has]


class _ReadFn(torch.autograd.Function):
    """Eager autograd of the read: inputs are (meta, *values, *keys, *optional)."""

    @staticmethod
    def forward(ctx, meta, *flat):
        n_v, n_k, has, heads, logit_scale, key_norm, normalize_output, mode, gate_act, gate_per_token, save = meta
        values = flat[:n_v]
        keys = flat[n_v:n_v + n_k]
        query, query_dyn, gate, bias, static_keys = _unflatten_opt(has, flat[n_v + n_k:])
        v0 = values[0]
        B, T, D = v0.shape
        desc = _hip.Desc(values, keys, query, query_dyn, gate, bias, heads, logit_scale, key_norm, normalize_output,
                         mode, gate_act, gate_per_token, static_keys=static_keys)
        with _device_ctx(v0.device):
            out, w, inv, pre = _hip.forward(desc, v0.device, v0.dtype, save and mode == _hip.MODE_SOFTMAX,
                                            normalize_output, save)
        if save:
            ctx.desc = desc
            ctx.meta = meta
            ctx.shape = (B, T, D)
            ctx.save_for_backward(*flat, pre, w, inv)
        return out.view(B, T, D)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        n_v, n_k, has, heads, logit_scale, key_norm, normalize_output, mode, gate_act, gate_per_token, _ = ctx.meta
        saved = ctx.saved_tensors  # (checks that no input was modified in place)
        query, query_dyn, gate, bias, static_keys = _unflatten_opt(has, saved[n_v + n_k:-3])
        pre, w, inv = saved[-3:]
        B, T, D = ctx.shape
        dev = saved[0].device
        want = ctx.needs_input_grad
        with _device_ctx(dev):
            dvals, dkeys, dq, dqd, dg, db, dsk = _hip.backward(
                ctx.desc, dev, saved[0].dtype, grad_out.contiguous(), pre, inv, w,
                want_dquery=query is not None and mode == _hip.MODE_SOFTMAX,
                want_dgate=gate is not None, want_dbias=bias is not None,
                query_shape=tuple(query.shape) if query is not None else (0,),
                gate_shape=tuple(gate.shape) if gate is not None else (0,), lr=n_k > 0,
                has_query_dyn=query_dyn is not None, batched=True, lead=(B, T),
                want_dstatic=static_keys is not None)
        grads = [None, *dvals, *dkeys]
        for present, g in zip(has, (dq, dqd.view(query_dyn.shape) if dqd is not None else None, dg, db,
                                    dsk.view(static_keys.shape) if dsk is not None else None)):
            if present:
                grads.append(g)
        # inputs that do not need a gradient get None (the kernels write all of them in one pass)
        return tuple(g if (g is None or want[i]) else None for i, g in enumerate(grads))


def _run(values, keys, query, query_dyn, gate, bias, heads, logit_scale, key_norm, normalize_output, mode,
         gate_act=_hip.GATE_NONE, gate_per_token=False, static_keys=None):
    opt = (query, query_dyn, gate, bias, static_keys)
    save = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (*values, *keys, *opt))
    if _compiling():
        out, _, _, _ = _read_op(values, keys, query, query_dyn, gate, bias, static_keys, int(heads),
                                float(logit_scale), bool(key_norm), bool(normalize_output), int(mode), int(gate_act),
                                bool(gate_per_token), bool(save))
        return out
    meta = (len(values), len(keys), tuple(t is not None for t in opt), int(heads), float(logit_scale),
            bool(key_norm), bool(normalize_output), int(mode), int(gate_act), bool(gate_per_token), bool(save))
    return _ReadFn.apply(meta, *values, *keys, *[t for t in opt if t is not None])


# ---------------------------------------------------------------- public API: base read

def attention_residual_read(values, query: Tensor, key_norm: bool, force_triton: bool = False,
                            normalize_output: bool = False, source_counts=None, source_logit_biases=None) -> Tensor:
    """Base AttnRes read (reference: attnres_ops.py:2503-2565).

    values: list of N [B,T,D] tensors or a stacked [N,B,T,D] tensor; query [D].
    Keys are ``rms_norm(values)`` when ``key_norm``.  A single source is
    returned as is (rms-normed when ``normalize_output``).
    """
    srcs = _sources(values)
    _check_sources(srcs, "attention_residual_read")
    if len(srcs) == 1:
        return _norm(srcs[0]) if normalize_output else srcs[0]
    dev = _check_gpu(srcs + [query], "attention_residual_read")
    # the reference casts the query to the first source's dtype (attnres_ops.py:2516),
    # and its eager read to the stacked sources' dtype (:2184)
    query = query.to(srcs[0].dtype)
    srcs = _promote(srcs)
    dtype = srcs[0].dtype
    D = srcs[0].size(-1)
    query = query.to(dtype)
    if query.numel() != D:
        raise RuntimeError(f"attention_residual_read: query must have {D} elements, got {query.numel()}")
    bias = _source_logit_bias(source_counts, source_logit_biases, len(srcs), dev)
    srcs = [_hip.as_rows(t) for t in srcs]
    return _run(srcs, [], query.reshape(D).contiguous(), None, None, bias, 1, 1.0, key_norm, normalize_output,
                _hip.MODE_SOFTMAX)


def attention_residual_read_torch(values, query: Tensor, key_norm: bool, source_counts=None,
                                  source_logit_biases=None) -> Tensor:
    """Name kept for import compatibility (reference: attnres_ops.py:2217-2225).

    In this build it runs the same HIP kernel as ``attention_residual_read``;
    the eager restatement used to check the kernels lives in ``oracle/``.
    """
    return attention_residual_read(values, query, key_norm, source_counts=source_counts,
                                   source_logit_biases=source_logit_biases)


def attention_residual_average_read(values, normalize_output: bool = False, force_triton: bool = False) -> Tensor:
    """Uniform mean over the sources (reference: attnres_ops.py:2568-2617), with a backward."""
    srcs = _sources(values)
    _check_sources(srcs, "attention_residual_average_read")
    if len(srcs) == 1:
        return _norm(srcs[0]) if normalize_output else srcs[0]
    _check_gpu(srcs, "attention_residual_average_read")
    srcs = [_hip.as_rows(t) for t in _promote(srcs)]
    return _run(srcs, [], None, None, None, None, 1, 1.0, False, normalize_output, _hip.MODE_AVERAGE)


# ---------------------------------------------------------------- public API: LR read

def _lr_common(values, keys, num_heads, what):
    """Values and keys as lists of [B, T, W] tensors, each list in its common
    (promoted) dtype.  The first key's own dtype is returned too: the
    reference casts the query to it (attnres_ops.py:4866-4870)."""
    vs = _sources(values)
    ks = _sources(keys)
    if len(vs) != len(ks):
        raise RuntimeError(f"{what}: got {len(vs)} value sources and {len(ks)} key sources")
    _check_sources(vs, what)
    _check_sources(ks, what)
    H = int(num_heads)
    B, T, D = vs[0].shape
    R = ks[0].size(-1)
    if ks[0].shape[:2] != (B, T):
        raise RuntimeError(f"{what}: keys must be [B, T, R] with the values' B, T")
    if H < 1 or D % H or R % H:
        raise RuntimeError(f"{what}: num_heads={H} must divide n_embd={D} and rank={R}")
    return _promote(vs), _promote(ks), H, D, R, ks[0].dtype


def _static_keys(static_keys, n: int, R: int, dtype, what: str) -> Tensor:
    """A static key per source as one [N, R] tensor in the key dtype: the
    model's ``key + static_key.to(key.dtype)`` (model.py:2046-2049, :286-288)."""
    sk = torch.stack(list(static_keys)) if isinstance(static_keys, (list, tuple)) else static_keys
    if sk.numel() != n * R:
        raise RuntimeError(f"{what}: static_keys must be [{n}, {R}] (one rank-{R} key per source), "
                           f"got {tuple(sk.shape)}")
    return sk.to(dtype).reshape(n, R).contiguous()


def lrid_attention_residual_read(values, keys, query: Tensor, num_heads: int, logit_scale: float, key_norm: bool,
                                 force_triton: bool = False, normalize_output: bool = False, source_counts=None,
                                 source_logit_biases=None, static_keys=None) -> Tensor:
    """LR AttnRes read (reference: attnres_ops.py:4852-5003).

    values: N x [B,T,D] (list or stacked); keys: N x [B,T,R]; query [H, R/H]
    (static, per read site) or [B,T,H,R/H] (input dependent).  The query is
    cast to the key dtype first, as in the reference.  The optional output
    rms-norm is fused for any number of heads.  Extra (not in the reference's
    op): ``static_keys`` [N, R] (or N tensors [R]) adds source s's static key to
    every key of source s inside the kernel, as the model adds it eagerly
    before the read (model.py:2046-2049); its gradient is the token sum of the
    key gradient.  The model's one shared ``[R]`` parameter (LRIDStaticKey,
    model.py:275-289), which it adds to every source but the embedding
    (model.py:2062-2063, 2070-2078), is the table with a zero row 0 and the
    parameter cast to the key dtype in every other row; autograd then sums the
    rows' gradients back into the parameter.
    """
    vs, ks, H, D, R, k0_dtype = _lr_common(values, keys, num_heads, "lrid_attention_residual_read")
    query = query.to(k0_dtype)
    if len(vs) == 1:
        return _norm(vs[0]) if normalize_output else vs[0]
    sk = None if static_keys is None else _static_keys(static_keys, len(vs), R, ks[0].dtype,
                                                        "lrid_attention_residual_read")
    dev = _check_gpu(vs + ks + [query] + ([sk] if sk is not None else []), "lrid_attention_residual_read")
    # Keys of another dtype than the values stay in their dtype: the eager read
    # norms them in fp32 and rounds them to the value dtype (attnres_ops.py:4179-4180),
    # so the logits are a value-dtype contraction with key_norm and a key-dtype
    # one without it; the query is cast to that dtype (:4182).
    query = query.to(vs[0].dtype if key_norm else ks[0].dtype)
    B, T, _ = vs[0].shape
    bias = _source_logit_bias(source_counts, source_logit_biases, len(vs), dev)
    vs = [_hip.as_rows(t) for t in vs]
    ks = [_hip.as_rows(t) for t in ks]
    if query.dim() == 4:
        if tuple(query.shape) != (B, T, H, R // H):
            raise RuntimeError(f"lrid_attention_residual_read: per-token query must be {(B, T, H, R // H)}, "
                               f"got {tuple(query.shape)}")
        qd = _hip.as_rows(query.reshape(B, T, R))
        return _run(vs, ks, None, qd, None, bias, H, logit_scale, key_norm, normalize_output, _hip.MODE_SOFTMAX,
                    static_keys=sk)
    if query.numel() != R:
        raise RuntimeError(f"lrid_attention_residual_read: static query must have {R} elements "
                           f"([{H}, {R // H}]), got {tuple(query.shape)}")
    return _run(vs, ks, query.reshape(H, R // H).contiguous(), None, None, bias, H, logit_scale, key_norm,
                normalize_output, _hip.MODE_SOFTMAX, static_keys=sk)


def lrid_attention_residual_read_gated(values, keys, static_query: Optional[Tensor], dynamic_query: Tensor,
                                       gate: Optional[Tensor], num_heads: int, logit_scale: float, key_norm: bool,
                                       gate_activation: str = "sigmoid", normalize_output: bool = False,
                                       source_counts=None, source_logit_biases=None, static_keys=None) -> Tensor:
    """LR read with the query composed inside the kernel: ``q = q_static + act(gate) * q_dyn``.

    ``gate_activation="linear"`` with a per-site ``gate[H]`` is the model's
    input-dependent query (model.py:2102-2113); ``"sigmoid"`` with a per-token
    ``gate[B,T,H]`` is benchmark config 4.  ``dynamic_query`` is [B,T,R] or
    [B,T,H,R/H]; ``static_query`` is [H,R/H] or None.  Gradients flow to all
    three (the per-site gate and static query are reduced over tokens
    deterministically).  Not present in the reference, which composes the query
    eagerly and then reads with an input-dependent query.  ``static_keys`` as
    in ``lrid_attention_residual_read`` (config 4's [N, 128] static source key).
    """
    vs, ks, H, D, R, _ = _lr_common(values, keys, num_heads, "lrid_attention_residual_read_gated")
    dtype = vs[0].dtype
    B, T, _ = vs[0].shape
    dev = _check_gpu(vs + ks + [dynamic_query], "lrid_attention_residual_read_gated")
    ks = [k.to(dtype) for k in ks]
    if dynamic_query.numel() != B * T * R:
        raise RuntimeError(f"dynamic_query must hold [B, T, {R}] elements")
    qd = _hip.as_rows(dynamic_query.to(dtype).reshape(B, T, R))
    qs = None
    if static_query is not None:
        if static_query.numel() != R:
            raise RuntimeError(f"static_query must have {R} elements")
        qs = static_query.to(dtype).reshape(H, R // H).contiguous()
    act = {"linear": _hip.GATE_LINEAR, "sigmoid": _hip.GATE_SIGMOID}.get(gate_activation)
    if act is None:
        raise RuntimeError(f"unknown gate_activation {gate_activation!r}")
    g = None
    per_token = False
    if gate is not None:
        g = gate.to(dtype)
        if g.numel() == H:
            g = g.reshape(H).contiguous()
        elif g.numel() == B * T * H:
            g = g.reshape(B, T, H).contiguous()
            per_token = True
        else:
            raise RuntimeError(f"gate must be [{H}] (per site) or [B, T, {H}] (per token)")
    if len(vs) == 1:
        return _norm(vs[0]) if normalize_output else vs[0]
    bias = _source_logit_bias(source_counts, source_logit_biases, len(vs), dev)
    sk = None if static_keys is None else _static_keys(static_keys, len(vs), R, dtype,
                                                        "lrid_attention_residual_read_gated")
    if sk is not None:
        _check_gpu([sk], "lrid_attention_residual_read_gated")
    vs = [_hip.as_rows(t) for t in vs]
    ks = [_hip.as_rows(t) for t in ks]
    return _run(vs, ks, qs, qd, g, bias, H, logit_scale, key_norm, normalize_output, _hip.MODE_SOFTMAX,
                act if g is not None else _hip.GATE_NONE, per_token, static_keys=sk)


def lrid_attention_residual_read_torch(values, keys, query: Tensor, num_heads: int, logit_scale: float,
                                       key_norm: bool, source_counts=None, source_logit_biases=None) -> Tensor:
    """Name kept for import compatibility (reference: attnres_ops.py:4235-4256); runs the HIP kernel."""
    return lrid_attention_residual_read(values, keys, query, num_heads, logit_scale, key_norm,
                                        source_counts=source_counts, source_logit_biases=source_logit_biases)


# ---------------------------------------------------------------- cached-logit phases

def _rows2d(t: Tensor) -> Tensor:
    """[B, T, W] -> [B*T, W] row view (copied only when tokens are not uniformly strided)."""
    t = _hip.as_rows(t)
    return t.view(t.size(0) * t.size(1), t.size(2))


@torch.library.custom_op("attnres_hip::phase1", mutates_args=())
def _phase1_op(values: list[Tensor], logits: Tensor, normalize_output: bool,
               save: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    desc = _hip.Phase1(values, logits, normalize_output)
    v0 = values[0]
    with torch.cuda.device(v0.device):
        out, lse, pre, inv = _hip.phase1_forward(desc, v0.device, v0.dtype, save)
    return out, lse, pre, inv


@_phase1_op.register_fake
def _phase1_fake(values, logits, normalize_output, save):
    v0 = values[0]
    Q, n, D = logits.size(0), v0.size(0), v0.size(1)
    keep = normalize_output and save
    return (v0.new_empty((Q, n, D)), v0.new_empty((Q, n), dtype=torch.float32),
            v0.new_empty((Q, n, D) if keep else (0,)), v0.new_empty((Q, n) if keep else (0,), dtype=torch.float32))


@torch.library.custom_op("attnres_hip::phase1_backward", mutates_args=())
def _phase1_backward_op(values: list[Tensor], logits: Tensor, grad_out: Tensor, grad_lse: Optional[Tensor],
                        prenorm: Tensor, inv_rms: Tensor, normalize_output: bool) -> tuple[list[Tensor], Tensor]:
    desc = _hip.Phase1(values, logits, normalize_output)
    v0 = values[0]
    with torch.cuda.device(v0.device):
        dvals, dlog = _hip.phase1_backward(desc, v0.device, v0.dtype, logits.dtype, grad_out, grad_lse, prenorm,
                                           inv_rms)
    return dvals, dlog


@_phase1_backward_op.register_fake
def _phase1_backward_fake(values, logits, grad_out, grad_lse, prenorm, inv_rms, normalize_output):
    return [v.new_empty((v.size(0), v.size(1))) for v in values], logits.new_empty(logits.shape)


def _phase1_setup_context(ctx, inputs, output):
    values, logits, normalize_output, save = inputs
    out, lse, pre, inv = output
    ctx.n_values = len(values)
    ctx.normalize_output = normalize_output
    ctx.save_for_backward(*values, logits, pre, inv)


def _phase1_backward(ctx, grad_out, grad_lse, grad_pre, grad_inv):
    saved = list(ctx.saved_tensors)
    values = saved[:ctx.n_values]
    logits, pre, inv = saved[ctx.n_values:]
    v0 = values[0]
    if grad_out is None:
        grad_out = v0.new_zeros((logits.size(0), v0.size(0), v0.size(1)))
    grad_lse = grad_lse.float().contiguous() if grad_lse is not None else None
    dvals, dlog = _phase1_backward_op(values, logits, grad_out.contiguous(), grad_lse, pre, inv,
                                      ctx.normalize_output)
    return dvals, dlog, None, None


_phase1_op.register_autograd(_phase1_backward, setup_context=_phase1_setup_context)


class _Phase1Fn(torch.autograd.Function):
    """Eager autograd of phase 1: inputs (meta, logits [Q,S,n], *value rows)."""

    @staticmethod
    def forward(ctx, meta, logits, *values):
        normalize_output, save = meta
        ctx.set_materialize_grads(False)
        v0 = values[0]
        desc = _hip.Phase1(values, logits, normalize_output)
        with _device_ctx(v0.device):
            out, lse, pre, inv = _hip.phase1_forward(desc, v0.device, v0.dtype, save)
        if save:
            ctx.desc = desc
            ctx.save_for_backward(logits, *values, pre, inv)
        return out, lse

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out, grad_lse):
        saved = ctx.saved_tensors
        logits, values, (pre, inv) = saved[0], saved[1:-2], saved[-2:]
        v0 = values[0]
        if grad_out is None and grad_lse is None:
            return (None, None, *([None] * len(values)))
        if grad_out is None:
            grad_out = v0.new_zeros((logits.size(0), v0.size(0), v0.size(1)))
        grad_lse = grad_lse.float().contiguous() if grad_lse is not None else None
        with _device_ctx(v0.device):
            dvals, dlog = _hip.phase1_backward(ctx.desc, v0.device, v0.dtype, logits.dtype, grad_out.contiguous(),
                                               grad_lse, pre, inv, batched=True)
        want = ctx.needs_input_grad
        return (None, dlog if want[1] else None, *[d if want[2 + i] else None for i, d in enumerate(dvals)])


def attention_residual_phase1_from_logits(values, logits: Tensor, force_triton: bool = False,
                                          normalize_output: bool = False):
    """Cached-logit read of completed sources for Q read sites (reference: attnres_ops.py:3910-3961).

    values: S x [B,T,D] (list or stacked [S,B,T,D]); logits [Q,S,B,T] (any
    float dtype; softmax in fp32).  Returns (out [Q,B,T,D] in the value dtype,
    lse [Q,B,T] fp32).  Up to 64 sources and 16 read sites, D <= 4096.
    """
    srcs = _sources(values)
    if len(srcs) == 0:
        raise RuntimeError("Cached-logit AttnRes phase1 requires at least one source")
    _check_sources(srcs, "attention_residual_phase1_from_logits")
    srcs = _promote(srcs)  # the eager read stacks the sources (attnres_ops.py:3940)
    B, T, D = srcs[0].shape
    S = len(srcs)
    if logits.dim() != 4 or logits.size(1) != S or tuple(logits.shape[2:]) != (B, T):
        raise RuntimeError(f"attention_residual_phase1_from_logits: logits must be [Q, {S}, {B}, {T}], "
                           f"got {tuple(logits.shape)}")
    Q = logits.size(0)
    if Q < 1 or Q > _hip.PHASE1_MAX_QUERIES:
        raise RuntimeError(f"attention_residual_phase1_from_logits: 1 <= Q <= {_hip.PHASE1_MAX_QUERIES}, got {Q}")
    if D > _hip.PHASE_MAX_DIM:
        raise RuntimeError(f"attention_residual_phase1_from_logits: D={D} exceeds {_hip.PHASE_MAX_DIM}")
    if logits.dtype not in _ALLOWED:
        raise RuntimeError(f"attention_residual_phase1_from_logits: logits dtype {logits.dtype} is not supported")
    _check_gpu(srcs + [logits], "attention_residual_phase1_from_logits")
    rows = [_rows2d(t) for t in srcs]
    lg = logits.contiguous().view(Q, S, B * T)
    save = torch.is_grad_enabled() and (logits.requires_grad or any(t.requires_grad for t in srcs))
    if _compiling():
        out, lse, _, _ = _phase1_op(rows, lg, bool(normalize_output), bool(save))
    else:
        out, lse = _Phase1Fn.apply((bool(normalize_output), bool(save)), lg, *rows)
    return out.view(Q, B, T, D), lse.view(Q, B, T)


class _Phase1SourcesFn(torch.autograd.Function):
    """Phase 1 of one block phase with per-source logits and per-site outputs:
    inputs (n_src, *source logits [Q, n], *value rows [n, D]); outputs the Q
    site outputs [n, D] and the Q lse rows [n].  The backward takes each
    site's gradients where the consumers left them and gives each source its
    own logit gradient, so nothing is stacked or sliced on either side."""

    @staticmethod
    def forward(ctx, n_src, *tensors):
        logits, values = tensors[:n_src], tensors[n_src:]
        v0 = values[0]
        ctx.set_materialize_grads(False)
        desc = _hip.Phase1Sources(values, logits, False)
        with _device_ctx(v0.device):
            out, lse, _, _ = _hip.phase1_forward(desc, v0.device, v0.dtype, False)
        ctx.desc = desc
        ctx.n_src = n_src
        ctx.ldt = logits[0].dtype
        ctx.save_for_backward(*logits, *values)
        return (*out.unbind(0), *lse.unbind(0))

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grads):
        Q = ctx.desc.n_q
        values = ctx.saved_tensors[ctx.n_src:]
        v0 = values[0]
        g_out = [g.contiguous() if g is not None else v0.new_zeros(v0.shape) for g in grads[:Q]]
        g_lse = [g.float().contiguous() if g is not None else None for g in grads[Q:]]
        with _device_ctx(v0.device):
            dvals, dlog = _hip.phase1_backward_sites(ctx.desc, v0.device, v0.dtype, ctx.ldt, g_out, g_lse, None,
                                                     None)
        want = ctx.needs_input_grad
        n = ctx.n_src
        return (None, *[d if want[1 + i] else None for i, d in enumerate(dlog)],
                *[d if want[1 + n + i] else None for i, d in enumerate(dvals)])


def lrid_block_phase1(values, source_logits):
    """Phase 1 of one block phase of the block LR decoder, from per-source logits.

    values: S x [B,T,D]; source_logits: S x [Q,B,T], source s's logits for
    the phase's Q sites (promoted to one dtype, as a stack of them is).  Returns (Q outputs [B,T,D], Q lse [B,T]
    fp32) -- what the reference's decoder gets from stacking the sources'
    logit pieces and calling phase 1 (``model.py:1931-1933``,
    ``attnres_ops.py:3910-3961``), with the stack and its backward's slices
    left out.
    """
    srcs = _promote(_sources(values))
    S = len(srcs)
    if S == 0 or len(source_logits) != S:
        raise RuntimeError(f"lrid_block_phase1: {len(source_logits)} logit tensors for {S} sources")
    _check_sources(srcs, "lrid_block_phase1")
    B, T, D = srcs[0].shape
    Q = source_logits[0].size(0)
    # one logits dtype, promoted as the reference's stack of the pieces promotes
    # (a source without a count prior keeps 16-bit logits, the others are fp32)
    ldt = source_logits[0].dtype
    for lg in source_logits[1:]:
        ldt = torch.promote_types(ldt, lg.dtype)
    source_logits = [lg.to(ldt) for lg in source_logits]
    for lg in source_logits:
        if tuple(lg.shape) != (Q, B, T) or lg.dtype != ldt:
            raise RuntimeError(f"lrid_block_phase1: logits must all be [{Q}, {B}, {T}] in {ldt}, got "
                               f"{tuple(lg.shape)} {lg.dtype}")
    if Q < 1 or Q > _hip.PHASE1_MAX_QUERIES:
        raise RuntimeError(f"lrid_block_phase1: 1 <= Q <= {_hip.PHASE1_MAX_QUERIES}, got {Q}")
    if D > _hip.PHASE_MAX_DIM:
        raise RuntimeError(f"lrid_block_phase1: D={D} exceeds {_hip.PHASE_MAX_DIM}")
    _check_gpu(srcs + list(source_logits), "lrid_block_phase1")
    rows = [_rows2d(t) for t in srcs]
    lgs = [lg.contiguous().view(Q, B * T) for lg in source_logits]
    res = _Phase1SourcesFn.apply(S, *lgs, *rows)
    return tuple(o.view(B, T, D) for o in res[:Q]), tuple(l.view(B, T) for l in res[Q:])


class _SiteLogitsFn(torch.autograd.Function):
    """One source's site logits: inputs (meta, key rows [n, R], queries [2L, R]);
    outputs the phase pieces [Q_b, n] of the [Q', n] logits."""

    @staticmethod
    def forward(ctx, meta, key, queries):
        first, sizes, scale, bias, key_norm, ldt = meta
        ctx.set_materialize_grads(False)
        desc = _hip.SiteLogits(key, queries[first:], key_norm, scale, ldt, bias)
        with _device_ctx(key.device):
            out = _hip.site_logits_forward(desc, key.device)
        ctx.desc = desc
        ctx.first = first
        ctx.sizes = sizes
        ctx.save_for_backward(key, queries)
        return tuple(out.split(list(sizes), dim=0))

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grads):
        key, queries = ctx.saved_tensors
        n = key.size(0)
        rows = []
        for g, sz in zip(grads, ctx.sizes):
            g = g.contiguous() if g is not None else key.new_zeros((sz, n), dtype=ctx.desc.logits_dtype)
            rows.extend(g.view(sz, n).unbind(0))
        with _device_ctx(key.device):
            dkey, du, khat = _hip.site_logits_backward(ctx.desc, key.device, rows)
            dq = None
            if ctx.needs_input_grad[2]:
                # the queries' gradient is the linear's weight gradient du^T khat (one GEMM)
                dq = torch.zeros_like(queries)
                torch.mm(du, khat, out=dq[ctx.first:])
        return None, dkey if ctx.needs_input_grad[1] else None, dq


def lrid_site_logits(key: Tensor, queries: Tensor, first: int, sizes, logit_scale: float,
                     logit_bias: float = 0.0, key_norm: bool = True):
    """A completed LR source's logits for every read site that will read it,
    as the pieces the block phases read (block decoder; reference:
    ``make_source_logits``, ``model.py:1843-1865``).

    key [B,T,R] (R <= 128); queries [2L, R] in the key dtype, row i-1 for site
    i; ``first``: row of the first site (its 1-based index minus one); sizes:
    site counts of the phases (summing to ``2L - first``).  Logits are
    ``rnd(rnd(<khat, q>) * logit_scale)`` in the key dtype, ``khat`` the
    fp32 rms-norm of the key rounded to its dtype; a nonzero ``logit_bias``
    (the count prior) is added in fp32 and makes the logits fp32, as the
    reference's eager chain does.  Returns the pieces [Q_b, B, T].
    """
    if key.dim() != 3 or queries.dim() != 2 or queries.size(1) != key.size(2):
        raise RuntimeError(f"lrid_site_logits: key [B,T,R] and queries [L,R], got {tuple(key.shape)} and "
                           f"{tuple(queries.shape)}")
    B, T, R = key.shape
    sizes = tuple(int(x) for x in sizes)
    if first < 0 or sum(sizes) != queries.size(0) - first or min(sizes) < 1:
        raise RuntimeError(f"lrid_site_logits: phase sizes {sizes} must cover query rows {first}..{queries.size(0) - 1}")
    if R > _hip.SITE_LOGITS_MAX_RANK:
        raise RuntimeError(f"lrid_site_logits: rank {R} exceeds {_hip.SITE_LOGITS_MAX_RANK}")
    if queries.dtype != key.dtype or key.dtype not in _ALLOWED:
        raise RuntimeError(f"lrid_site_logits: queries ({queries.dtype}) must be in the key dtype ({key.dtype})")
    _check_gpu([key, queries], "lrid_site_logits")
    ldt = torch.float32 if float(logit_bias) != 0.0 else key.dtype
    rows = _rows2d(key)
    q = queries.contiguous()
    meta = (int(first), sizes, float(logit_scale), float(logit_bias), bool(key_norm), ldt)
    parts = _SiteLogitsFn.apply(meta, rows, q)
    return tuple(p.view(p.size(0), B, T) for p in parts)


class _KeyedLogitsFn(torch.autograd.Function):
    """Eager autograd of the query-bank logits: inputs (key_norm, queries [Q,D], *value rows)."""

    @staticmethod
    def forward(ctx, key_norm, queries, *values):
        ctx.set_materialize_grads(False)
        v0 = values[0]
        desc = _hip.KeyedLogits(values, queries, key_norm)
        with _device_ctx(v0.device):
            logits, inv = _hip.keyed_logits_forward(desc, v0.device, v0.dtype, True)
        ctx.desc = desc
        ctx.save_for_backward(queries, inv, *values)
        return logits

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dlogits):
        saved = ctx.saved_tensors
        queries, inv, values = saved[0], saved[1], saved[2:]
        if dlogits is None:
            return (None, None, *([None] * len(values)))
        v0 = values[0]
        want = ctx.needs_input_grad
        with _device_ctx(v0.device):
            dvals, dq = _hip.keyed_logits_backward(ctx.desc, v0.device, v0.dtype, dlogits.contiguous(), inv,
                                                   bool(want[1]))
        return (None, dq, *[d if want[2 + i] else None for i, d in enumerate(dvals)])


def attention_residual_phase1(values, queries: Tensor, key_norm: bool, force_triton: bool = False):
    """Phase 1 with logits from a query bank (reference: attnres_ops.py:3862-3907; eager form
    ``_attnres_phase1_read_torch`` :2620-2627).

    values: S x [B,T,D] (list or stacked [S,B,T,D]); queries [Q,D], cast to the
    value dtype as the reference does.  The logits ``<queries[q], rms_norm(v_s)>``
    (value dtype) come from the keyed-logits kernels; the read over them is
    ``attention_residual_phase1_from_logits``.  Returns (out [Q,B,T,D], lse [Q,B,T]).
    """
    srcs = _sources(values)
    if len(srcs) == 0:
        raise RuntimeError("Two-phase AttnRes phase1 requires at least one source")
    _check_sources(srcs, "attention_residual_phase1")
    srcs = _promote(srcs)
    B, T, D = srcs[0].shape
    if queries.dim() != 2 or queries.size(1) != D:
        raise RuntimeError(f"attention_residual_phase1: queries must be [Q, {D}], got {tuple(queries.shape)}")
    Q = queries.size(0)
    if Q < 1 or Q > _hip.PHASE1_MAX_QUERIES:
        raise RuntimeError(f"attention_residual_phase1: 1 <= Q <= {_hip.PHASE1_MAX_QUERIES}, got {Q}")
    if D > _hip.PHASE_MAX_DIM:
        raise RuntimeError(f"attention_residual_phase1: D={D} exceeds {_hip.PHASE_MAX_DIM}")
    _check_gpu(srcs + [queries], "attention_residual_phase1")
    q = queries.to(srcs[0].dtype).contiguous()
    rows = [_rows2d(t) for t in srcs]
    logits = _KeyedLogitsFn.apply(bool(key_norm), q, *rows)
    return attention_residual_phase1_from_logits(srcs, logits.view(Q, len(srcs), B, T))


@torch.library.custom_op("attnres_hip::phase2", mutates_args=())
def _phase2_op(partial_value: Tensor, partial_key: Optional[Tensor], query: Optional[Tensor],
               partial_logit: Optional[Tensor], inter: Tensor, lse: Tensor, bias_t: Optional[Tensor],
               scale_t: Optional[Tensor], merge: int, key_norm: bool, normalize_output: bool, logit_scale: float,
               bias_value: float, scale_value: float, scale_key: bool) -> Tensor:
    desc = _hip.Phase2(partial_value, partial_key, query, partial_logit, inter, lse, merge, key_norm,
                       normalize_output, logit_scale, bias_value, bias_t, scale_value, scale_t, scale_key)
    with torch.cuda.device(partial_value.device):
        return _hip.phase2_forward(desc, partial_value.device, partial_value.dtype)


@_phase2_op.register_fake
def _phase2_fake(partial_value, partial_key, query, partial_logit, inter, lse, bias_t, scale_t, merge, key_norm,
                 normalize_output, logit_scale, bias_value, scale_value, scale_key):
    return partial_value.new_empty(partial_value.shape)


@torch.library.custom_op("attnres_hip::phase2_backward", mutates_args=())
def _phase2_backward_op(partial_value: Tensor, partial_key: Optional[Tensor], query: Optional[Tensor],
                        partial_logit: Optional[Tensor], inter: Tensor, lse: Tensor, bias_t: Optional[Tensor],
                        scale_t: Optional[Tensor], grad_out: Tensor, merge: int, key_norm: bool,
                        normalize_output: bool, logit_scale: float, bias_value: float, scale_value: float,
                        scale_key: bool, want_dbias: bool, want_dscale: bool) -> list[Tensor]:
    desc = _hip.Phase2(partial_value, partial_key, query, partial_logit, inter, lse, merge, key_norm,
                       normalize_output, logit_scale, bias_value, bias_t, scale_value, scale_t, scale_key)
    dev = partial_value.device
    with torch.cuda.device(dev):
        dp, dpk, dq, di, dl, dlg, db, ds = _hip.phase2_backward(
            desc, dev, partial_value.dtype, grad_out,
            want_dquery=query is not None and partial_logit is None,
            query_shape=tuple(query.shape) if query is not None else (0,),
            logit_dtype=partial_logit.dtype if partial_logit is not None else None,
            want_dbias=want_dbias, want_dscale=want_dscale)
    e = lambda: torch.empty((0,), device=dev)  # noqa: E731
    return [dp, dpk if dpk is not None else e(), dq if dq is not None else e(), di, dl,
            dlg if dlg is not None else e(), db if db is not None else e(), ds if ds is not None else e()]


@_phase2_backward_op.register_fake
def _phase2_backward_fake(partial_value, partial_key, query, partial_logit, inter, lse, bias_t, scale_t, grad_out,
                          merge, key_norm, normalize_output, logit_scale, bias_value, scale_value, scale_key,
                          want_dbias, want_dscale):
    e = lambda: partial_value.new_empty((0,))  # noqa: E731
    n = partial_value.size(0)
    return [partial_value.new_empty(partial_value.shape),
            partial_key.new_empty(partial_key.shape) if partial_key is not None else e(),
            query.new_empty(query.shape) if query is not None and partial_logit is None else e(),
            inter.new_empty(inter.shape), partial_value.new_empty((n,), dtype=torch.float32),
            partial_logit.new_empty(partial_logit.shape) if partial_logit is not None else e(),
            partial_value.new_empty((1,), dtype=torch.float32) if want_dbias else e(),
            partial_value.new_empty((1,), dtype=torch.float32) if want_dscale else e()]


def _phase2_setup_context(ctx, inputs, output):
    (partial_value, partial_key, query, partial_logit, inter, lse, bias_t, scale_t, merge, key_norm,
     normalize_output, logit_scale, bias_value, scale_value, scale_key) = inputs
    ctx.has = tuple(t is not None for t in (partial_key, query, partial_logit, bias_t, scale_t))
    opt = [t for t in (partial_key, query, partial_logit, bias_t, scale_t) if t is not None]
    ctx.save_for_backward(partial_value, inter, lse, *opt)
    ctx.flags = (merge, key_norm, normalize_output, logit_scale, bias_value, scale_value, scale_key)


def _phase2_backward(ctx, grad_out):
    saved = list(ctx.saved_tensors)
    partial_value, inter, lse = saved[:3]
    rest = saved[3:]
    partial_key, query, partial_logit, bias_t, scale_t = [rest.pop(0) if h else None for h in ctx.has]
    merge, key_norm, normalize_output, logit_scale, bias_value, scale_value, scale_key = ctx.flags
    want_dbias = bias_t is not None and ctx.needs_input_grad[6]
    want_dscale = scale_t is not None and ctx.needs_input_grad[7]
    dp, dpk, dq, di, dl, dlg, db, ds = _phase2_backward_op(
        partial_value, partial_key, query, partial_logit, inter, lse, bias_t, scale_t, grad_out.contiguous(), merge,
        key_norm, normalize_output, logit_scale, bias_value, scale_value, scale_key, want_dbias, want_dscale)
    return (dp, dpk if partial_key is not None else None,
            dq if query is not None and partial_logit is None else None,
            dlg if partial_logit is not None else None, di, dl,
            db.reshape(bias_t.shape) if want_dbias else None,
            ds.reshape(scale_t.shape) if want_dscale else None,
            None, None, None, None, None, None, None)


_phase2_op.register_autograd(_phase2_backward, setup_context=_phase2_setup_context)


class _Phase2Fn(torch.autograd.Function):
    """Eager autograd of the phase-2 merge: inputs (meta, partial rows, inter rows, lse, *optional)."""

    @staticmethod
    def forward(ctx, meta, partial_value, inter, lse, *opt_flat):
        has, merge, key_norm, normalize_output, logit_scale, bias_value, scale_value, scale_key, qrow = meta
        partial_key, query, partial_logit, bias_t, scale_t = _unflatten_opt(has, opt_flat)
        # query_row: `query` is a bank and the merge reads one of its rows (a view)
        qd = query[qrow] if qrow is not None else query
        desc = _hip.Phase2(partial_value, partial_key, qd, partial_logit, inter, lse, merge, key_norm,
                           normalize_output, logit_scale, bias_value, bias_t, scale_value, scale_t, scale_key)
        dev = partial_value.device
        with _device_ctx(dev):
            out = _hip.phase2_forward(desc, dev, partial_value.dtype)
        ctx.desc = desc
        ctx.meta = meta
        ctx.save_for_backward(partial_value, inter, lse, *opt_flat)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        has = ctx.meta[0]
        saved = ctx.saved_tensors
        partial_value = saved[0]
        partial_key, query, partial_logit, bias_t, scale_t = _unflatten_opt(has, saved[3:])
        want = ctx.needs_input_grad
        # needs_input_grad index of each present optional input (after meta, partial, inter, lse)
        pos = {}
        k = 4
        for name, h in zip(("pk", "q", "pl", "b", "s"), has):
            if h:
                pos[name] = k
                k += 1
        want_dbias = bias_t is not None and want[pos["b"]]
        want_dscale = scale_t is not None and want[pos["s"]]
        dev = partial_value.device
        with _device_ctx(dev):
            dp, dpk, dq, di, dl, dlg, db, ds = _hip.phase2_backward(
                ctx.desc, dev, partial_value.dtype, grad_out.contiguous(),
                want_dquery=query is not None and partial_logit is None and want[pos["q"]],
                query_shape=tuple(query.shape) if query is not None else (0,),
                logit_dtype=partial_logit.dtype if partial_logit is not None else None,
                want_dbias=want_dbias, want_dscale=want_dscale, query_row=ctx.meta[-1])
        grads = [None, dp if want[1] else None, di if want[2] else None, dl if want[3] else None]
        for name, g in (("pk", dpk), ("q", dq), ("pl", dlg), ("b", db), ("s", ds)):
            if name in pos:
                t = pos[name]
                if name == "b" and g is not None:
                    g = g.reshape(bias_t.shape)
                if name == "s" and g is not None:
                    g = g.reshape(scale_t.shape)
                grads.append(g if want[t] else None)
        return tuple(grads)


def _scalar_arg(x, device, what):
    """(float value, fp32 [1] tensor or None) for a float-or-tensor argument."""
    if x is None:
        return 0.0, None
    if isinstance(x, Tensor):
        if x.numel() != 1:
            raise RuntimeError(f"{what} must be a scalar")
        return 0.0, x.to(device=device, dtype=torch.float32).reshape(1)
    return float(x), None


def _phase2(partial_value, partial_key, query, partial_logit, interblock_output, interblock_lse, merge, key_norm,
            normalize_output, logit_scale, logit_bias, partial_scale, scale_key, what, query_row=None):
    if partial_value.dim() != 3:
        raise RuntimeError(f"{what}: partial_value must be [B, T, D]")
    B, T, D = partial_value.shape
    dtype = partial_value.dtype
    if dtype not in _ALLOWED:
        raise RuntimeError(f"{what}: dtype {dtype} is not supported (fp32, bf16, fp16)")
    if D > _hip.PHASE_MAX_DIM:
        raise RuntimeError(f"{what}: D={D} exceeds {_hip.PHASE_MAX_DIM}")
    if tuple(interblock_output.shape) != (B, T, D):
        raise RuntimeError(f"{what}: interblock_output must be {(B, T, D)}, got {tuple(interblock_output.shape)}")
    if interblock_lse.numel() != B * T:
        raise RuntimeError(f"{what}: interblock_lse must be [B, T]")
    dev = _check_gpu([partial_value, interblock_output, interblock_lse], what)
    bias_value, bias_t = _scalar_arg(logit_bias, dev, "logit_bias")
    if partial_scale is None:
        scale_value, scale_t = 1.0, None
    else:
        scale_value, scale_t = _scalar_arg(partial_scale, dev, "partial_scale")
    pv = _rows2d(partial_value)
    it = _rows2d(interblock_output.to(dtype))
    lse = interblock_lse.float().reshape(B * T).contiguous()
    pk = q = pl = None
    if partial_logit is not None:
        if partial_logit.numel() != B * T:
            raise RuntimeError(f"{what}: partial_logit must be [B, T]")
        pl = partial_logit.reshape(B * T).contiguous()
    elif partial_key is not None:
        pk = _rows2d(partial_key.reshape(B, T, partial_key.size(-1)).to(dtype))
        if query_row is not None:
            # a bank [rows, width] and the row this merge reads
            if query.dim() != 2 or query.size(1) != pk.size(1):
                raise RuntimeError(f"{what}: a query bank must be [rows, {pk.size(1)}], got {tuple(query.shape)}")
            if not 0 <= int(query_row) < query.size(0):
                raise RuntimeError(f"{what}: query_row={query_row} outside [0, {query.size(0)})")
            q = query.to(dtype).contiguous()
            if _compiling():  # the custom op takes one row: select it
                q, query_row = q[int(query_row)], None
        else:
            q = query.reshape(-1).to(dtype).contiguous()
            if q.numel() != pk.size(1):
                raise RuntimeError(f"{what}: query must have {pk.size(1)} elements, got {q.numel()}")
    else:
        q = query.reshape(-1).to(dtype).contiguous()
        if q.numel() != D:
            raise RuntimeError(f"{what}: query must have {D} elements, got {q.numel()}")
    if _compiling():
        out = _phase2_op(pv, pk, q, pl, it, lse, bias_t, scale_t, int(merge), bool(key_norm), bool(normalize_output),
                         float(logit_scale), bias_value, scale_value, bool(scale_key))
    else:
        opt = (pk, q, pl, bias_t, scale_t)
        meta = (tuple(t is not None for t in opt), int(merge), bool(key_norm), bool(normalize_output),
                float(logit_scale), bias_value, scale_value, bool(scale_key),
                None if query_row is None else int(query_row))
        out = _Phase2Fn.apply(meta, pv, it, lse, *[t for t in opt if t is not None])
    return out.view(B, T, D)


def attention_residual_phase2(partial_value: Tensor, query: Tensor, interblock_output: Tensor,
                              interblock_lse: Tensor, key_norm: bool, force_triton: bool = False,
                              normalize_output: bool = False, logit_bias=0.0, partial_scale=None) -> Tensor:
    """Merge of the live partial block into a phase-1 read (reference: attnres_ops.py:3964-4019).

    ``prob = sigmoid(<key(partial), query> + logit_bias - lse)``, ``out =
    inter + (partial - inter) * prob``; ``key = rms_norm(partial)`` when
    ``key_norm``.  ``partial_scale`` (float or scalar tensor, not in the
    reference) multiplies the partial value first, which folds the block
    summary ``partial_block * count**-alpha`` (model.py:990-1001) into the
    kernel.
    """
    return _phase2(partial_value, None, query, None, interblock_output, interblock_lse, _hip.MERGE_ADDCMUL, key_norm,
                   normalize_output, 1.0, logit_bias, partial_scale, False, "attention_residual_phase2")


def attention_residual_phase2_torch(partial_value: Tensor, query: Tensor, interblock_output: Tensor,
                                    interblock_lse: Tensor, key_norm: bool, normalize_output: bool = False,
                                    logit_bias=0.0, partial_scale=None) -> Tensor:
    """Name kept for import compatibility (reference: attnres_ops.py:4022-4040); runs the HIP kernel."""
    return attention_residual_phase2(partial_value, query, interblock_output, interblock_lse, key_norm,
                                     normalize_output=normalize_output, logit_bias=logit_bias,
                                     partial_scale=partial_scale)


def attention_residual_phase2_from_logit(partial_value: Tensor, partial_logit: Tensor, interblock_output: Tensor,
                                         interblock_lse: Tensor, force_triton: bool = False,
                                         normalize_output: bool = False, partial_scale=None) -> Tensor:
    """Merge with a precomputed partial logit (reference: attnres_ops.py:4043-4072)."""
    return _phase2(partial_value, None, None, partial_logit, interblock_output, interblock_lse, _hip.MERGE_ADDCMUL,
                   False, normalize_output, 1.0, None, partial_scale, False, "attention_residual_phase2_from_logit")


def lrid_attention_residual_phase2(partial_value: Tensor, partial_key: Tensor, query: Tensor,
                                   interblock_output: Tensor, interblock_lse: Tensor, logit_scale: float,
                                   key_norm: bool, force_triton: bool = False, normalize_output: bool = False,
                                   logit_bias=0.0, partial_scale=None, scale_key: bool = False,
                                   query_row: Optional[int] = None) -> Tensor:
    """LR merge, ``addcmul`` form (reference: attnres_ops.py:4075-4139; single head).

    ``partial_scale`` multiplies the partial value (and, with ``scale_key``,
    the partial key) first: the LR block source of model.py:1003-1018.
    ``query_row`` (an addition to the reference's signature): ``query`` is a
    [rows, rank] bank and the merge reads row ``query_row``; the backward
    hands the bank its gradient directly (the row's, zeros elsewhere), the
    tensor ``query[query_row]``'s select would produce, without the select's
    fill and copy launches.
    """
    return _phase2(partial_value, partial_key, query, None, interblock_output, interblock_lse, _hip.MERGE_ADDCMUL,
                   key_norm, normalize_output, logit_scale, logit_bias, partial_scale, scale_key,
                   "lrid_attention_residual_phase2", query_row)


def lrid_attention_residual_phase2_torch(partial_value: Tensor, partial_key: Tensor, query: Tensor,
                                         interblock_output: Tensor, interblock_lse: Tensor, logit_scale: float,
                                         key_norm: bool, normalize_output: bool = False, logit_bias=0.0,
                                         partial_scale=None, scale_key: bool = False,
                                         query_row: Optional[int] = None) -> Tensor:
    """LR merge, ``torch.lerp`` form (reference: attnres_ops.py:4142-4160), on the HIP kernel
    (``query_row`` as in lrid_attention_residual_phase2)."""
    return _phase2(partial_value, partial_key, query, None, interblock_output, interblock_lse, _hip.MERGE_LERP,
                   key_norm, normalize_output, logit_scale, logit_bias, partial_scale, scale_key,
                   "lrid_attention_residual_phase2_torch", query_row)


# ------------------------------------------------------------------ key-producer epilogue

@torch.library.custom_op("attnres_hip::keyed_split", mutates_args=())
def _keyed_split_op(y: Tensor, dim: int, rank: int, heads: int, key_norm: bool) -> tuple[Tensor, Tensor, Tensor]:
    return _hip.keyed_split_forward(y, dim, rank, heads, key_norm)


@_keyed_split_op.register_fake
def _keyed_split_fake(y, dim, rank, heads, key_norm):
    n = y.size(0)
    return (y.new_empty((n, dim)), y.new_empty((n, rank)),
            y.new_empty((n, heads) if key_norm else (0,), dtype=torch.float32))


@torch.library.custom_op("attnres_hip::keyed_split_backward", mutates_args=())
def _keyed_split_backward_op(y: Optional[Tensor], grad_out: Optional[Tensor], grad_key: Optional[Tensor],
                             inv: Tensor, n_tok: int, proj_cols: int, dim: int, rank: int, heads: int,
                             key_norm: bool) -> Tensor:
    like = grad_out if grad_out is not None else grad_key
    return _hip.keyed_split_backward(y, n_tok, proj_cols, dim, rank, heads, key_norm, grad_out, grad_key, inv,
                                     like.dtype, like.device)


@_keyed_split_backward_op.register_fake
def _keyed_split_backward_fake(y, grad_out, grad_key, inv, n_tok, proj_cols, dim, rank, heads, key_norm):
    like = grad_out if grad_out is not None else grad_key
    return like.new_empty((n_tok, proj_cols))


def _keyed_split_setup_context(ctx, inputs, output):
    y, dim, rank, heads, key_norm = inputs
    ctx.args = (y.size(0), y.size(1), dim, rank, heads, key_norm)
    # the raw key (inside y) is read only by the key-norm backward
    ctx.save_for_backward(y if key_norm else None, output[2])


def _keyed_split_backward(ctx, grad_out, grad_key, grad_inv):
    y, inv = ctx.saved_tensors
    go = grad_out.contiguous() if grad_out is not None else None
    gk = grad_key.contiguous() if grad_key is not None else None
    if go is None and gk is None:
        return None, None, None, None, None
    return _keyed_split_backward_op(y, go, gk, inv, *ctx.args), None, None, None, None


_keyed_split_op.register_autograd(_keyed_split_backward, setup_context=_keyed_split_setup_context)


class _KeySplitFn(torch.autograd.Function):
    """Eager autograd of the key-producer epilogue: inputs (meta, y [n, P])."""

    @staticmethod
    def forward(ctx, meta, y):
        dim, rank, heads, key_norm = meta
        ctx.set_materialize_grads(False)
        with _device_ctx(y.device):
            out, key, inv = _hip.keyed_split_forward(y, dim, rank, heads, key_norm)
        ctx.args = (y.size(0), y.size(1), dim, rank, heads, key_norm)
        # the raw key (inside y) is read only by the key-norm backward
        ctx.save_for_backward(y if key_norm else None, inv)
        return out, key

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out, grad_key):
        y, inv = ctx.saved_tensors
        if grad_out is None and grad_key is None:
            return None, None
        go = grad_out.contiguous() if grad_out is not None else None
        gk = grad_key.contiguous() if grad_key is not None else None
        like = go if go is not None else gk
        with _device_ctx(like.device):
            gy = _hip.keyed_split_backward(y, *ctx.args, go, gk, inv, like.dtype, like.device)
        return None, gy


def lrid_fused_projection_split(projected: Tensor, output_dim: int, rank: int, num_heads: int = 1,
                                key_norm: bool = True):
    """Sublayer output and LR key from a fused ``[out | key | pad]`` projection.

    Not in the reference's op module: the reference does this in
    ``LRIDFusedProjection.forward`` (model.py:363-388) as
    ``out = projected[..., :D].contiguous()``, ``key = projected[..., D:D+rank]``
    and, with key norm, ``_norm_lrid_key(key, num_heads)`` (model.py:34-37).
    Here one HIP pass writes both (the key rms-normed per depth head in fp32,
    torch's default eps) and the backward writes the projection's gradient
    ``[d_out | norm backward of d_key | 0]`` in one pass, instead of two
    zero-filled slice gradients and their sum.  ``projected`` is ``[..., >= D +
    rank]`` on the GPU; returns ``(out [..., D], key [..., rank])``.
    """
    if projected.size(-1) < output_dim + rank:
        raise RuntimeError(f"lrid_fused_projection_split: projection has {projected.size(-1)} columns, "
                           f"needs at least {output_dim + rank}")
    _check_gpu([projected], "lrid_fused_projection_split")
    lead = projected.shape[:-1]
    y = projected.reshape(-1, projected.size(-1))
    if y.stride(-1) != 1:
        y = y.contiguous()
    if _compiling():
        out, key, _ = _keyed_split_op(y, int(output_dim), int(rank), int(num_heads), bool(key_norm))
    else:
        out, key = _KeySplitFn.apply((int(output_dim), int(rank), int(num_heads), bool(key_norm)), y)
    return out.view(*lead, output_dim), key.view(*lead, rank)


# ------------------------------------------------------------------ value-derived keys

class _ValueKeyFn(torch.autograd.Function):
    """Eager autograd of the value-derived keys: inputs (meta, W [R, D], *values);
    outputs N keys [B, T, R]."""

    @staticmethod
    def forward(ctx, meta, weight, *values):
        value_norm, = meta
        v0 = values[0]
        B, T, D = v0.shape
        n = len(values)
        R = weight.size(0)
        ctx.set_materialize_grads(False)
        if value_norm:
            d = _hip.ValueKey(values)
            with _device_ctx(v0.device):
                x, inv = _hip.value_norm_forward(d, v0.device, v0.dtype)
            ctx.desc, ctx.inv = d, inv
        else:
            x = torch.stack([v.reshape(B * T, D) for v in values]).reshape(n * B * T, D)
            ctx.desc = None
        # one library GEMM over every source's rows: [N * n_tok, D] x [D, R]
        keys = torch.mm(x, weight.t())
        ctx.save_for_backward(weight, x, *values)
        ctx.shape = (n, B, T, D, R)
        return tuple(keys.view(n, B, T, R).unbind(0))

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grad_keys):
        weight, x, *values = ctx.saved_tensors
        n, B, T, D, R = ctx.shape
        if all(g is None for g in grad_keys):
            return (None, None) + (None,) * n
        gk = torch.stack([g.reshape(B * T, R) if g is not None else x.new_zeros((B * T, R)) for g in grad_keys])
        gk = gk.reshape(n * B * T, R)
        want = ctx.needs_input_grad  # (meta, weight, *values)
        dw = torch.mm(gk.t(), x) if want[1] else None
        dvals = [None] * n
        if any(want[2:]):
            gx = torch.mm(gk, weight)
            if ctx.desc is not None:
                with _device_ctx(x.device):
                    dvals = _hip.value_norm_backward(ctx.desc, x.device, x.dtype, gx, ctx.inv, (B, T))
            else:
                dvals = list(gx.view(n, B, T, D).unbind(0))
        return (None, dw) + tuple(dv if want[2 + i] else None for i, dv in enumerate(dvals))


def lrid_value_key_projection(values, weight: Tensor, value_norm: bool = True):
    """LR keys projected from the sources' values: ``rms_norm(v_s) @ W^T``.

    Not in the reference's op module: the reference's
    ``LRIDSourceKeyProjection.forward`` (model.py:420-428, with
    ``lrid_key_from_value`` and ``lrid_key_value_norm``) does this per source as
    ``self.proj(norm(x))`` -- config 4's key producer.  Here one HIP pass
    rms-norms every source (fp32, one rounding to the dtype) into one block, a
    single library GEMM projects all of them, and the backward runs the GEMMs
    for the weight and input gradients and one HIP pass of the rms-norm
    backward.  ``values``: N x [B, T, D] (or [N, B, T, D]); ``weight`` [R, D]
    (``nn.Linear(D, R).weight``).  Returns N keys [B, T, R] in the values' dtype.
    """
    vs = _sources(values)
    _check_sources(vs, "lrid_value_key_projection")
    _check_gpu(vs + [weight], "lrid_value_key_projection")
    vs = _promote(vs)
    D = vs[0].size(-1)
    if weight.dim() != 2 or weight.size(1) != D:
        raise RuntimeError(f"lrid_value_key_projection: weight must be [rank, {D}], got {tuple(weight.shape)}")
    vs = [_hip.as_rows(t) for t in vs]
    w = weight.to(vs[0].dtype)
    return list(_ValueKeyFn.apply((bool(value_norm),), w, *vs))


# ------------------------------------------------------------------ block-summary accumulation

class _BlockAccumFn(torch.autograd.Function):
    """Eager autograd of the fused block accumulation: inputs (meta, y [n, P],
    partial value rows [n, D] | None, partial key rows [n, R] | None, learned
    scale fp32 [1] | None); outputs (value [n, D], key [n, R])."""

    @staticmethod
    def forward(ctx, meta, y, pv, pk, scale_t):
        dim, rank, heads, key_norm, complete, value_norm, scale_key, scale_value = meta
        ctx.set_materialize_grads(False)
        d = _hip.block_accum_desc(y, dim, rank, heads, key_norm, pv, pk, complete, value_norm, scale_key,
                                  scale_value, scale_t)
        with _device_ctx(y.device):
            value, key, kinv, vinv = _hip.block_accum_forward(d, y.device, y.dtype, dim, rank, heads, key_norm,
                                                              complete and value_norm)
        ctx.meta = meta
        ctx.desc = d
        ctx.save_for_backward(y, pv, pk, scale_t, kinv, vinv)
        return value, key

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, g_value, g_key):
        y, pv, pk, scale_t, kinv, vinv = ctx.saved_tensors
        dim, rank, heads, key_norm, complete, value_norm, scale_key, scale_value = ctx.meta
        if g_value is None and g_key is None:
            return None, None, None, None, None
        want = ctx.needs_input_grad  # (meta, y, pv, pk, scale)
        if g_value is not None and g_value.stride(-1) != 1:
            g_value = g_value.contiguous()
        gk = g_key.contiguous() if g_key is not None else None
        key_scaled = complete and scale_key and not value_norm
        with _device_ctx(y.device):
            gy, dpk, ds = _hip.block_accum_backward(ctx.desc, y.device, y.dtype, g_value, gk, kinv, vinv,
                                                    want_dpk=key_scaled and pk is not None and want[3] and gk is not None,
                                                    want_dscale=scale_t is not None and want[4])
        # the grown partial value's gradient is also the partial value's: columns [0, D) of gy
        # (or the incoming gradient itself when nothing scales or norms it)
        d_pv = None
        if pv is not None and want[2] and g_value is not None:
            d_pv = gy[:, :dim] if complete else g_value
        d_pk = None
        if pk is not None and want[3] and gk is not None:
            d_pk = dpk if key_scaled else gk
        d_s = ds.reshape(scale_t.shape) if ds is not None else None
        return None, gy if want[1] else None, d_pv, d_pk, d_s


def lrid_block_accumulate(projected: Tensor, partial_value: Optional[Tensor], partial_key: Optional[Tensor],
                          output_dim: int, rank: int, num_heads: int = 1, key_norm: bool = True,
                          complete: bool = False, partial_scale=1.0, value_norm: bool = False,
                          scale_key: bool = False):
    """A sublayer's fused projection added to the live partial block in one pass.

    Not in the reference's op module: the reference model splits the projection
    (``LRIDFusedProjection.forward``, model.py:363-388, as
    ``lrid_fused_projection_split``), then adds the output and key to the
    partial block eagerly (model.py:2377-2389, 2451-2463) and, at a block end,
    forms the block source with ``_attnres_block_summary`` /
    ``_lrid_block_source`` (model.py:990-1028).  Here::

        partial_value' = partial_value + projected[..., :D]
        partial_key'   = partial_key + key(projected)    (per-head rms-norm when key_norm)

    and with ``complete`` the block source instead:
    ``value = partial_value' * partial_scale`` (float or learned scalar tensor;
    ``rms_norm(partial_value')`` with ``value_norm``) and ``key = partial_key'``
    (``* partial_scale`` with ``scale_key``, the model's rule for keys that are
    not rms-normed).  ``partial_value`` / ``partial_key`` are None for the first
    sublayer of a block.  Every add and product rounds to the dtype as the
    eager ops do.  Returns ``(value [..., D], key [..., rank])``.
    """
    P = projected.size(-1)
    if P < output_dim + rank:
        raise RuntimeError(f"lrid_block_accumulate: projection has {P} columns, needs at least {output_dim + rank}")
    if projected.dtype not in _ALLOWED:
        raise RuntimeError(f"lrid_block_accumulate: dtype {projected.dtype} is not supported (fp32, bf16, fp16)")
    if not complete and (value_norm or scale_key or isinstance(partial_scale, Tensor) or float(partial_scale) != 1.0):
        raise RuntimeError("lrid_block_accumulate: partial_scale / value_norm / scale_key apply to complete=True only")
    if value_norm and scale_key:
        raise RuntimeError("lrid_block_accumulate: value_norm leaves the key unscaled")
    lead = projected.shape[:-1]
    n = projected.numel() // P
    tensors = [projected] + [t for t in (partial_value, partial_key) if t is not None]
    dev = _check_gpu(tensors, "lrid_block_accumulate")
    y = projected.reshape(n, P)
    if y.stride(-1) != 1:
        y = y.contiguous()

    def rows(t, width, what):
        if t is None:
            return None
        if t.dtype != projected.dtype or t.numel() != n * width:
            raise RuntimeError(f"lrid_block_accumulate: {what} must be {tuple(lead) + (width,)} in {projected.dtype}")
        return t.reshape(n, width).contiguous()

    pv = rows(partial_value, output_dim, "partial_value")
    pk = rows(partial_key, rank, "partial_key")
    scale_value, scale_t = (1.0, None) if not complete or value_norm else _scalar_arg(partial_scale, dev, "partial_scale")
    meta = (int(output_dim), int(rank), int(num_heads), bool(key_norm), bool(complete), bool(value_norm),
            bool(scale_key), scale_value)
    value, key = _BlockAccumFn.apply(meta, y, pv, pk, scale_t)
    return value.view(*lead, output_dim), key.view(*lead, rank)


class _AccumReadFn(torch.autograd.Function):
    """Eager autograd of the block accumulation fused with the merge that reads
    the grown block: inputs (meta, y [n, P], partial value rows [n, D] | None,
    partial key rows [n, R] | None, query bank [rows, R], inter rows [n, D],
    lse fp32 [n], logit bias fp32 [1] | None, value scale fp32 [1] | None);
    outputs (value [n, D], key [n, R], out [n, D])."""

    @staticmethod
    def forward(ctx, meta, y, pv, pk, query, inter, lse, bias_t, scale_t):
        (dim, rank, heads, key_norm, merge, merge_key_norm, normalize_output, logit_scale, bias_value, scale_value,
         scale_key, qrow) = meta
        ctx.set_materialize_grads(False)
        n, dev, dtype = y.size(0), y.device, y.dtype
        acc = _hip.block_accum_desc(y, dim, rank, heads, key_norm, pv, pk, False, False, False, 1.0, None)
        value = torch.empty((n, dim), device=dev, dtype=dtype)
        key = torch.empty((n, rank), device=dev, dtype=dtype)
        kinv = torch.empty((n, heads) if key_norm else (0,), device=dev, dtype=torch.float32)
        out = torch.empty((n, dim), device=dev, dtype=dtype)
        read = _hip.Phase2(value, key, query[qrow], None, inter, lse, merge, merge_key_norm, normalize_output,
                           logit_scale, bias_value, bias_t, scale_value, scale_t, scale_key)
        d = _hip.accum_read_desc(acc, read)
        with _device_ctx(dev):
            _hip.accum_read_forward(d, value, key, kinv, out, dev)
        ctx.meta = meta
        # the descriptor is plain bytes; the tensors its pointers name (y, the old
        # and grown blocks, the merge's inputs) live on as saved tensors -- the
        # outputs only there, so that ctx holds no reference cycle through them
        ctx.desc = d
        ctx.save_for_backward(y, pv, pk, query, inter, lse, bias_t, scale_t, kinv, value, key)
        return value, key, out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, g_value, g_key, g_out):
        if g_value is None and g_key is None and g_out is None:
            return (None,) * 9
        y, pv, pk, query, inter, lse, bias_t, scale_t, kinv, value, key = ctx.saved_tensors
        dim, qrow = ctx.meta[0], ctx.meta[-1]
        want = ctx.needs_input_grad  # (meta, y, pv, pk, query, inter, lse, bias, scale)
        d = ctx.desc
        g_out = torch.zeros_like(value) if g_out is None else g_out.contiguous()
        if g_value is not None and (g_value.stride(-1) != 1 or g_value.stride(0) < dim):
            g_value = g_value.contiguous()
        gk = g_key.contiguous() if g_key is not None else None
        dev = y.device
        with _device_ctx(dev):
            gy, dpk, dq, di, dl, db, ds = _hip.accum_read_backward(
                d, dev, y.dtype, g_out, g_value, gk, kinv if kinv.numel() else None, want_dquery=want[4],
                query_shape=tuple(query.shape), query_row=qrow, want_dbias=bias_t is not None and want[7],
                want_dscale=scale_t is not None and want[8], want_dpk_old=pk is not None and want[3])
        # the grown value's total gradient is also the old partial value's: columns [0, D) of gy
        return (None, gy if want[1] else None, gy[:, :dim] if pv is not None and want[2] else None,
                dpk if pk is not None and want[3] else None, dq if want[4] else None, di if want[5] else None,
                dl if want[6] else None, db.reshape(bias_t.shape) if db is not None else None,
                ds.reshape(scale_t.shape) if ds is not None else None)


def _accum_read_fits(y: Tensor, inter: Tensor, D: int, R: int, heads: int) -> bool:
    """Shapes the fused accumulate-and-read kernels take: 16-bit rows one wave
    covers exactly (D = 256, 512, 768, 1024), rank <= 256, 16-byte aligned rows."""
    if y.dtype not in (torch.bfloat16, torch.float16) or D not in (256, 512, 768, 1024):
        return False
    if not 1 <= R <= 256 or R % heads != 0:
        return False
    return all(t.data_ptr() % 16 == 0 and (t.stride(0) * t.element_size()) % 16 == 0 for t in (y, inter))


def lrid_block_accumulate_read(projected: Tensor, partial_value: Optional[Tensor], partial_key: Optional[Tensor],
                               query: Tensor, interblock_output: Tensor, interblock_lse: Tensor, output_dim: int,
                               rank: int, logit_scale: float, num_heads: int = 1, key_norm: bool = True,
                               merge_key_norm: Optional[bool] = None, lerp: bool = False,
                               normalize_output: bool = False, logit_bias=0.0, partial_scale=None,
                               scale_key: bool = False, query_row: Optional[int] = None):
    """A sublayer's block accumulation and the read at the next site, in one pass.

    Not in the reference's op module: its model grows the live partial block
    after the projection split (model.py:363-388, 2377-2389) and the next read
    site merges it with ``lrid_attention_residual_phase2[_torch]``
    (attnres_ops.py:4075-4160).  Same results, bit for bit, as::

        value, key = lrid_block_accumulate(projected, partial_value, partial_key, output_dim, rank,
                                           num_heads, key_norm)
        out = lrid_attention_residual_phase2[_torch](value, key, query, interblock_output, interblock_lse,
                                                     logit_scale, merge_key_norm, ...)

    (``_torch``, the ``lerp`` merge, with ``lerp``), and the gradients of all
    three outputs as autograd sums them there; the cross-token sums (the
    query's, a learned bias's or scale's gradient) group their fp32 partials
    by the fused backward's own grid, which above about 3000 tokens has fewer
    workgroups than the merge's, so there they agree to rounding, not bit for
    bit.  ``merge_key_norm`` defaults to ``key_norm``.  Returns ``(value, key, out)``: the grown block and the read.
    Shapes the fused kernels do not take run the two calls.
    """
    mkn = key_norm if merge_key_norm is None else bool(merge_key_norm)
    D, R = int(output_dim), int(rank)
    if interblock_output.dim() != 3 or interblock_output.size(-1) != D:
        raise RuntimeError(f"lrid_block_accumulate_read: interblock_output must be [B, T, {D}]")
    B, T = interblock_output.shape[:2]
    P = projected.size(-1)
    y = projected.reshape(B * T, P) if projected.numel() == B * T * P else None
    inter = _rows2d(interblock_output) if interblock_output.dtype == projected.dtype else None
    fused = (y is not None and inter is not None and y.stride(-1) == 1 and B * T > 0 and not _compiling()
             and P >= D + R and _accum_read_fits(y, inter, D, R, int(num_heads)))
    if not fused:
        value, key = lrid_block_accumulate(projected, partial_value, partial_key, D, R, num_heads, key_norm)
        value, key = value.reshape(B, T, D), key.reshape(B, T, R)
        phase2 = lrid_attention_residual_phase2_torch if lerp else lrid_attention_residual_phase2
        out = phase2(value, key, query, interblock_output, interblock_lse, logit_scale, mkn,
                     normalize_output=normalize_output, logit_bias=logit_bias, partial_scale=partial_scale,
                     scale_key=scale_key, query_row=query_row)
        return value, key, out
    what = "lrid_block_accumulate_read"
    dev = _check_gpu([t for t in (projected, partial_value, partial_key, query, interblock_output, interblock_lse)
                      if t is not None], what)
    if interblock_lse.numel() != B * T:
        raise RuntimeError(f"{what}: interblock_lse must be [B, T]")

    def rows(t, width, name):
        if t is None:
            return None
        if t.dtype != projected.dtype or t.numel() != B * T * width:
            raise RuntimeError(f"{what}: {name} must be {(B, T, width)} in {projected.dtype}")
        return t.reshape(B * T, width).contiguous()

    pv = rows(partial_value, D, "partial_value")
    pk = rows(partial_key, R, "partial_key")
    if query_row is None:
        if query.numel() != R:
            raise RuntimeError(f"{what}: query must have {R} elements, got {query.numel()}")
        bank, qrow = query.reshape(1, R).to(projected.dtype).contiguous(), 0
    else:
        if query.dim() != 2 or query.size(1) != R or not 0 <= int(query_row) < query.size(0):
            raise RuntimeError(f"{what}: a query bank must be [rows, {R}] with query_row in range")
        bank, qrow = query.to(projected.dtype).contiguous(), int(query_row)
    bias_value, bias_t = _scalar_arg(logit_bias, dev, "logit_bias")
    scale_value, scale_t = (1.0, None) if partial_scale is None else _scalar_arg(partial_scale, dev, "partial_scale")
    lse = interblock_lse.float().reshape(B * T).contiguous()
    meta = (D, R, int(num_heads), bool(key_norm), _hip.MERGE_LERP if lerp else _hip.MERGE_ADDCMUL, mkn,
            bool(normalize_output), float(logit_scale), bias_value, scale_value, bool(scale_key), qrow)
    value, key, out = _AccumReadFn.apply(meta, y, pv, pk, bank, inter, lse, bias_t, scale_t)
    return value.view(B, T, D), key.view(B, T, R), out.view(B, T, D)
