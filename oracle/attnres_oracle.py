"""Eager PyTorch restatement of the reference AttnRes read (TEST INFRASTRUCTURE).

This module is the parity oracle for the HIP kernels in ``lr-attnres_amd``.
It is imported only by ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg; the product never imports it.

It restates the reference's *eager* op (``/root/reference/attnres_ops.py``)
step by step, keeping the same sequence of dtype casts, because that sequence
decides the bf16/fp16 rounding points the HIP kernels mirror:

* rms-norm with ``eps=None`` is ``F.rms_norm``'s default, which for a bf16 or
  fp16 input is the float32 epsilon (``attnres_ops.py:49-52``).
* LR keys are normed in fp32 and rounded to the value dtype
  (``attnres_ops.py:4179-4180``); base keys are ``rms_norm(values)`` in the
  value dtype (``attnres_ops.py:2183``).
* logits are a contraction in the value dtype (fp32 accumulate, one
  rounding), then ``* logit_scale`` (rounded again), then ``+ bias`` which
  promotes to fp32 (``attnres_ops.py:4183-4189``).
* softmax runs in fp32 and the weights are rounded to the value dtype before
  the mix (``attnres_ops.py:4190``); the mix is a contraction in the value
  dtype (``attnres_ops.py:4191``).

Contractions use ``torch.einsum`` exactly where the reference does, so the
autograd graph (and therefore the rounding of every gradient) is the
reference's own.

Pinning (see tests/test_oracle_pinning.py and tests/test_oracle_golden.py):

========================================  ======================================
function                                  pinned by
========================================  ======================================
attention_residual_read_torch             fp64 brute force (oracle/fp64.py),
                                          closed forms, invariants, gradcheck,
                                          golden fixtures from the reference
lrid_attention_residual_read_torch        same
attention_residual_read_ref               same + single-source identity
lrid_attention_residual_read_ref          same + single-source identity
attention_residual_average_read_ref       closed form (mean) and fp64
gated_query_ref                           closed form (zero gate -> static)
block_* helpers                           the reference tests' known answers
lrid_fused_projection_split_ref           the reference model itself: whole-model
                                          golden vectors (tests/golden/model_*)
lrid_value_key_projection_ref             golden vectors written by the reference's
                                          LRIDSourceKeyProjection (lrid_key_from_value,
                                          value norm on and off; fp32 and bf16; keys,
                                          value and weight gradients), bit for bit
                                          (tests/test_oracle_producers.py)
static_key_add_ref,                       golden vectors written by the reference's
shared_static_key_table_ref               LRIDStaticKey + OBPM._add_static_lrid_source_key
                                          followed by its eager LR read (keys with the
                                          static key, output, value / key / query
                                          gradients and the fp32 parameter's gradient)
                                          (tests/test_oracle_producers.py)
lrid_block_accumulate_ref                 composition of the pinned split and
                                          block_* helpers; the decoder built on
                                          it reproduces the reference-model
                                          golden vectors
lrid_site_logits_ref,                     the decoder built on them reproduces the
lrid_block_phase1_ref                     reference-model golden vectors bit for bit
                                          (tests/test_decoder_host.py): they are the
                                          decoder's former inline eager chain
phase1_from_logits_ref / phase2_*_ref     phase1+phase2 == full read identity
                                          (tests/test_attnres_ops.py:582-610),
                                          golden fixtures with gradients,
                                          fp64 gradcheck
attention_residual_phase1_ref             one query == the base read (pinned
                                          above), fp64 brute force of out / lse
========================================  ======================================
"""

from __future__ import annotations

import math

import torch
from torch import Tensor
from torch.nn import functional as F


# --------------------------------------------------------------------------
# small helpers
# --------------------------------------------------------------------------

def norm(x: Tensor) -> Tensor:
    """rms-norm over the last dim with torch's default eps.

    Follows ``attnres_ops.py:49-52`` / ``model.py:26-31`` (``eps=None``).
    """
    return F.rms_norm(x, (x.size(-1),))


def stack_sources(values) -> Tensor:
    """``attnres_ops.py:58-61``: a list of [B,T,D] becomes [S,B,T,D]."""
    if isinstance(values, Tensor):
        return values
    return torch.stack(list(values), dim=0)


def source_logit_bias(source_counts, source_logit_biases, n_sources: int, device) -> Tensor | None:
    """Per-source fp32 logit bias, ``attnres_ops.py:65-105``.

    ``source_counts`` gives ``log(count)``; ``source_logit_biases`` is used as
    is; they are mutually exclusive.  Scalars broadcast to every source.
    """
    if source_counts is not None and source_logit_biases is not None:
        raise RuntimeError("source_counts and source_logit_biases are mutually exclusive")
    if source_logit_biases is None:
        if source_counts is None:
            return None
        if isinstance(source_counts, Tensor):
            counts = source_counts.reshape(-1).to(device=device, dtype=torch.float32)
        elif isinstance(source_counts, (int, float)):
            counts = torch.full((n_sources,), float(source_counts), device=device, dtype=torch.float32)
        else:
            if len(source_counts) != n_sources:
                raise RuntimeError("source_counts length must match the number of sources")
            vals = [float(c) for c in source_counts]
            if any(c <= 0.0 for c in vals):
                raise RuntimeError("source_counts must be positive")
            counts = torch.tensor(vals, device=device, dtype=torch.float32)
        if counts.numel() != n_sources:
            raise RuntimeError("source_counts length must match the number of sources")
        return counts.log()
    if isinstance(source_logit_biases, Tensor):
        biases = source_logit_biases.reshape(-1).to(device=device, dtype=torch.float32)
    elif isinstance(source_logit_biases, (int, float)):
        biases = torch.full((n_sources,), float(source_logit_biases), device=device, dtype=torch.float32)
    else:
        if len(source_logit_biases) != n_sources:
            raise RuntimeError("source_logit_biases length must match the number of sources")
        items = []
        for b in source_logit_biases:
            if isinstance(b, Tensor):
                items.append(b.to(device=device, dtype=torch.float32).reshape(()))
            else:
                items.append(torch.tensor(float(b), device=device, dtype=torch.float32))
        biases = torch.stack(items)
    if biases.numel() != n_sources:
        raise RuntimeError("source_logit_biases length must match the number of sources")
    return biases


# --------------------------------------------------------------------------
# base AttnRes (keys = rms_norm(values) or values), attnres_ops.py:2176-2225
# --------------------------------------------------------------------------

def attention_residual_read_torch(values, query: Tensor, key_norm: bool,
                                  source_counts=None, source_logit_biases=None) -> Tensor:
    """Stacked eager base read, ``attnres_ops.py:2176-2190`` via ``:2217-2225``.

    values [S,B,T,D] (or list of [B,T,D]); query [D].  Returns [B,T,D] in the
    value dtype.
    """
    v = stack_sources(values)
    k = norm(v) if key_norm else v
    q = query.to(k.dtype)
    logits = torch.einsum("d,sbtd->sbt", q, k)
    bias = source_logit_bias(source_counts, source_logit_biases, v.size(0), logits.device)
    if bias is not None:
        logits = logits + bias.view(-1, 1, 1)
    w = F.softmax(logits.float(), dim=0).to(v.dtype)
    return torch.einsum("sbt,sbtd->btd", w, v)


def attention_residual_read_ref(values, query: Tensor, key_norm: bool, normalize_output: bool = False,
                                source_counts=None, source_logit_biases=None) -> Tensor:
    """What the reference's ``attention_residual_read`` returns, in eager form.

    ``attnres_ops.py:2503-2565``: a single source is returned as is (then
    optionally normed); the query is cast to the value dtype; an optional
    rms-norm of the output follows the read.
    """
    srcs = list(values) if not isinstance(values, Tensor) else list(values.unbind(0))
    if len(srcs) == 1:
        return norm(srcs[0]) if normalize_output else srcs[0]
    q = query.to(srcs[0].dtype)
    out = attention_residual_read_torch(srcs, q, key_norm, source_counts, source_logit_biases)
    return norm(out) if normalize_output else out


def attention_residual_average_read_ref(values, normalize_output: bool = False) -> Tensor:
    """Uniform mean over sources, ``attnres_ops.py:2568-2617`` (eager branch)."""
    srcs = list(values) if not isinstance(values, Tensor) else list(values.unbind(0))
    if len(srcs) == 1:
        out = srcs[0]
    else:
        out = torch.stack(srcs, dim=0).mean(dim=0)
    return norm(out) if normalize_output else out


# --------------------------------------------------------------------------
# LR AttnRes (low-rank keys, multi-head), attnres_ops.py:4163-4256
# --------------------------------------------------------------------------

def lrid_attention_residual_read_torch(values, keys, query: Tensor, num_heads: int, logit_scale: float,
                                       key_norm: bool, source_counts=None, source_logit_biases=None) -> Tensor:
    """Stacked eager LR read, ``attnres_ops.py:4163-4192`` via ``:4235-4256``.

    values [S,B,T,D], keys [S,B,T,R], query [H,R/H] (static) or
    [B,T,H,R/H] (per token).  Returns [B,T,D].
    """
    v = stack_sources(values)
    k = stack_sources(keys)
    H = int(num_heads)
    S, B, T, D = v.shape
    rh = k.size(-1) // H
    dh = D // H
    k = k.reshape(S, B, T, H, rh)
    v = v.reshape(S, B, T, H, dh)
    if key_norm:
        k = norm(k.float()).to(v.dtype)
    q = query.to(k.dtype)
    if q.dim() == 4:
        logits = torch.einsum("sbthr,bthr->sbth", k, q) * logit_scale
    else:
        logits = torch.einsum("sbthr,hr->sbth", k, q) * logit_scale
    bias = source_logit_bias(source_counts, source_logit_biases, S, logits.device)
    if bias is not None:
        logits = logits + bias.view(-1, 1, 1, 1)
    w = F.softmax(logits.float(), dim=0).to(v.dtype)
    out = torch.einsum("sbth,sbthd->bthd", w, v)
    return out.reshape(B, T, H * dh)


def lrid_attention_residual_read_ref(values, keys, query: Tensor, num_heads: int, logit_scale: float,
                                     key_norm: bool, normalize_output: bool = False,
                                     source_counts=None, source_logit_biases=None) -> Tensor:
    """What the reference's ``lrid_attention_residual_read`` returns, eagerly.

    ``attnres_ops.py:4852-5003``: the query is cast to the key dtype first
    (``:4870``); a single source is returned as is; the optional output norm
    is a full-width rms-norm after the read (``:4971-5003``).
    """
    vs = list(values) if not isinstance(values, Tensor) else list(values.unbind(0))
    ks = list(keys) if not isinstance(keys, Tensor) else list(keys.unbind(0))
    q = query.to(ks[0].dtype)
    if len(vs) == 1:
        return norm(vs[0]) if normalize_output else vs[0]
    out = lrid_attention_residual_read_torch(vs, ks, q, num_heads, logit_scale, key_norm,
                                             source_counts, source_logit_biases)
    return norm(out) if normalize_output else out


def gated_query_ref(static_query: Tensor | None, dynamic_query: Tensor | None, gate: Tensor | None,
                    num_heads: int, activation: str = "linear") -> Tensor:
    """Input-dependent query composition.

    ``activation="linear"`` is the model's rule, ``model.py:2102-2113``:
    ``q = q_static + gate[H] * q_dyn[B,T,H,R/H]`` (no sigmoid, one gate per
    read site and head).  ``activation="sigmoid"`` is the benchmark config-4
    rule ``q = q_static + sigmoid(gate[B,T,H]) * q_dyn``.  The result is
    [B,T,H,R/H] (or the static query when there is no dynamic part).
    """
    if dynamic_query is None:
        return static_query
    B, T = dynamic_query.shape[:2]
    H = int(num_heads)
    qd = dynamic_query.reshape(B, T, H, -1)
    if gate is None:
        g = torch.ones((), dtype=qd.dtype, device=qd.device)
    else:
        g = gate
        if activation == "sigmoid":
            g = torch.sigmoid(g)
        elif activation != "linear":
            raise ValueError(f"unknown gate activation {activation!r}")
        g = g.reshape(B, T, H, 1) if g.dim() >= 2 else g.reshape(1, 1, H, 1)
    q = g * qd
    if static_query is not None:
        q = static_query.reshape(1, 1, H, -1) + q
    return q


# --------------------------------------------------------------------------
# block summaries (model.py), the "fused accumulation" semantics
# --------------------------------------------------------------------------

def make_block_ends(n_layer: int, num_blocks: int) -> frozenset:
    """``model.py:828-836``: block ends over the 2*n_layer sublayers."""
    total = 2 * n_layer
    nb = min(num_blocks, total)
    return frozenset(math.ceil(total * i / nb) for i in range(1, nb + 1))


def block_count_scale(count: int, alpha) -> float | Tensor:
    """``model.py:955-959``: ``count ** -alpha`` (alpha may be a tensor)."""
    if isinstance(alpha, Tensor):
        return torch.exp(-alpha * alpha.new_tensor(float(count)).log())
    return float(count) ** (-float(alpha))


def _as_value_dtype(s, value: Tensor):
    """A scale tensor as the reference multiplies by it on the GPU: in the value
    dtype.  The learned scale is cast explicitly (``model.py:983-985``); a
    learned alpha leaves ``count ** -alpha`` a 0-dim fp32 device tensor, and
    multiplying a 16-bit tensor by one casts it to that dtype first (the CPU
    kernel would keep it in fp32 -- this oracle runs on the CPU, so it casts
    explicitly).  A python number stays in fp32."""
    return s.to(value.dtype) if isinstance(s, Tensor) else s


def block_summary(partial_sum: Tensor, count: int, alpha=1.0, value_norm: bool = False,
                  scale=None) -> Tensor:
    """Block source value, ``model.py:990-1001``.

    ``value_norm`` replaces the scaling by an rms-norm; an explicit ``scale``
    (learned per-summary scale) overrides ``count ** -alpha``.
    """
    if value_norm:
        return norm(partial_sum)
    s = block_count_scale(count, alpha) if scale is None else scale
    return partial_sum * _as_value_dtype(s, partial_sum)


def lrid_block_source(partial_sum: Tensor, partial_key: Tensor, count: int, alpha=1.0,
                      key_norm: bool = True, value_norm: bool = False, scale=None):
    """LR block source (value, key), ``model.py:1003-1018``.

    The key is scaled like the value only when keys are not rms-normed
    (a norm would cancel the scale anyway).
    """
    if value_norm:
        return norm(partial_sum), partial_key
    s = _as_value_dtype(block_count_scale(count, alpha) if scale is None else scale, partial_sum)
    value = partial_sum * s
    key = partial_key
    if key is not None and not key_norm:
        key = key * (s.to(key.dtype) if isinstance(s, Tensor) else s)
    return value, key


def block_count_logit_bias(count: int, beta) -> float | Tensor:
    """``model.py:1045-1069``: ``beta * log(count)``; zero for a count of 1."""
    if count == 1:
        return 0.0
    if isinstance(beta, Tensor):
        return beta * beta.new_tensor(math.log(float(count)))
    beta = float(beta)
    return 0.0 if beta == 0.0 else beta * math.log(float(count))


# --------------------------------------------------------------------------
# cached-logit phase1 / phase2 (next-tier rows), attnres_ops.py:3956-4160
# --------------------------------------------------------------------------

def phase1_from_logits_ref(values, logits: Tensor, normalize_output: bool = False):
    """Eager cached-logit read, ``attnres_ops.py:3956-3961``.

    values [S,B,T,D]; logits [Q,S,B,T].  Returns (out [Q,B,T,D], lse [Q,B,T]).
    """
    v = stack_sources(values)
    w = F.softmax(logits.float(), dim=1).to(v.dtype)
    out = torch.einsum("qsbt,sbtd->qbtd", w, v)
    if normalize_output:
        out = norm(out)
    return out, torch.logsumexp(logits.float(), dim=1)


def lrid_site_logits_ref(key: Tensor, queries: Tensor, first: int, sizes, logit_scale: float,
                         logit_bias: float = 0.0, key_norm: bool = True):
    """One completed LR source's logits for the read sites that will read it,
    split into the phases that read them -- ``make_source_logits``
    (``model.py:1843-1865``): key rms-normed in fp32 and rounded to its dtype,
    ``F.linear`` with the queries of sites ``first + 1 ..`` (rows ``first ..``
    of ``queries``), permuted to [Q', B, T], ``* logit_scale`` and, when the
    count prior gives a nonzero bias, ``+ bias`` in fp32.

    key [B, T, R]; queries [2L, R] (the key dtype).  Returns ``sizes``-long
    pieces of the [Q', B, T] logits along the sites (views).
    """
    k = key
    if key_norm:
        k = norm(k.float()).to(key.dtype)
    logits = F.linear(k, queries[first:].to(k.dtype)).permute(2, 0, 1).contiguous()
    logits = logits * logit_scale
    if logit_bias != 0.0:
        logits = logits + torch.full((logits.size(0),), logit_bias, dtype=torch.float32,
                                     device=logits.device).view(-1, 1, 1)
    return logits.split(list(sizes), dim=0)


def lrid_block_phase1_ref(values, source_logits):
    """Phase 1 of one block phase from the per-source logits of its sites: the
    decoder's stack of the sources' logit pieces along S (``model.py:1931-1933``)
    followed by phase 1 (``attnres_ops.py:3956-3961``).  values S x [B,T,D];
    source_logits S x [Q,B,T].  Returns per-site (out [B,T,D] ..., lse [B,T] ...)."""
    logits = torch.stack(list(source_logits), dim=1).contiguous()
    out, lse = phase1_from_logits_ref(values, logits)
    return out.unbind(0), lse.unbind(0)


def attention_residual_phase1_ref(values, queries: Tensor, key_norm: bool):
    """Phase 1 from a query bank, ``_attnres_phase1_read_torch`` (``attnres_ops.py:2620-2627``,
    reached from ``attention_residual_phase1`` :3862-3907, which casts the
    queries to the value dtype first).

    values [S,B,T,D]; queries [Q,D].  Returns (out [Q,B,T,D], lse [Q,B,T]).
    """
    v = stack_sources(values)
    keys = norm(v) if key_norm else v
    logits = torch.einsum("qd,sbtd->qsbt", queries.to(keys.dtype), keys)
    lse = torch.logsumexp(logits.float(), dim=1)
    w = F.softmax(logits.float(), dim=1).to(v.dtype)
    return torch.einsum("qsbt,sbtd->qbtd", w, v), lse


def attention_residual_phase2_ref(partial_value: Tensor, query: Tensor, interblock_output: Tensor,
                                  interblock_lse: Tensor, key_norm: bool, logit_bias=0.0,
                                  normalize_output: bool = False) -> Tensor:
    """Two-way merge of the live partial block, ``attnres_ops.py:2628-2642``."""
    key = norm(partial_value) if key_norm else partial_value
    logit = torch.sum(key * query.to(key.dtype), dim=-1).float()
    if isinstance(logit_bias, Tensor):
        logit = logit + logit_bias.to(device=logit.device, dtype=torch.float32)
    elif float(logit_bias) != 0.0:
        logit = logit + float(logit_bias)
    prob = torch.sigmoid(logit - interblock_lse.float()).to(partial_value.dtype)
    out = torch.addcmul(interblock_output, partial_value - interblock_output, prob.unsqueeze(-1))
    return norm(out) if normalize_output else out


def lrid_attention_residual_phase2_ref(partial_value: Tensor, partial_key: Tensor, query: Tensor,
                                       interblock_output: Tensor, interblock_lse: Tensor,
                                       logit_scale: float, key_norm: bool, normalize_output: bool = False,
                                       logit_bias=0.0, merge: str = "lerp") -> Tensor:
    """LR two-way merge (single head).

    ``merge="lerp"`` is ``lrid_attention_residual_phase2_torch``
    (``attnres_ops.py:4142-4160``); ``merge="addcmul"`` is the eager path of
    ``lrid_attention_residual_phase2`` (``:4085-4139``), which hands the logit
    to ``attention_residual_phase2_from_logit`` (``:4041-4068``).
    """
    q = query.reshape(-1).to(partial_key.dtype)
    pk = partial_key.reshape(partial_key.size(0), partial_key.size(1), -1)
    key = norm(pk.float()).to(partial_value.dtype) if key_norm else pk
    logit = torch.sum(key * q.to(key.dtype).view(1, 1, -1), dim=-1) * float(logit_scale)
    logit = logit.float()
    if isinstance(logit_bias, Tensor):
        logit = logit + logit_bias.to(device=logit.device, dtype=torch.float32)
    elif float(logit_bias) != 0.0:
        logit = logit + float(logit_bias)
    if merge == "addcmul":
        return phase2_from_logit_ref(partial_value, logit, interblock_output, interblock_lse,
                                     normalize_output=normalize_output)
    prob = torch.sigmoid(logit - interblock_lse.float()).to(partial_value.dtype)
    out = torch.lerp(interblock_output, partial_value, prob.unsqueeze(-1))
    return norm(out) if normalize_output else out


def phase2_from_logit_ref(partial_value: Tensor, partial_logit: Tensor, interblock_output: Tensor,
                          interblock_lse: Tensor, normalize_output: bool = False) -> Tensor:
    """Merge with a given partial logit, ``attnres_ops.py:4041-4068`` (eager branch)."""
    prob = torch.sigmoid(partial_logit.float() - interblock_lse.float()).to(partial_value.dtype)
    out = torch.addcmul(interblock_output, partial_value - interblock_output, prob.unsqueeze(-1))
    return norm(out) if normalize_output else out


def lrid_fused_projection_split_ref(projected: Tensor, output_dim: int, rank: int, num_heads: int = 1,
                                    key_norm: bool = True):
    """Sublayer output and LR key of a fused projection, ``model.py:374-378``
    with the per-head key norm ``_norm_lrid_key`` (``model.py:34-37``)."""
    out = projected[..., :output_dim].contiguous()
    key = projected[..., output_dim:output_dim + rank]
    if key_norm:
        shape = key.shape
        key = norm(key.reshape(*shape[:-1], num_heads, shape[-1] // num_heads)).reshape(shape)
    return out, key


def lrid_value_key_projection_ref(values, weight: Tensor, value_norm: bool = True):
    """Keys projected from the values: ``LRIDSourceKeyProjection.forward``
    (model.py:420-428) with ``lrid_key_from_value`` -- ``norm(x)`` when
    ``lrid_key_value_norm``, then the rank-R ``nn.Linear`` without bias (no key
    norm on this path: ``use_key_norm`` is off with ``lrid_key_from_value``,
    :418)."""
    return [F.linear(norm(v) if value_norm else v, weight.to(v.dtype)) for v in values]


def static_key_add_ref(keys, static_keys):
    """Keys with each source's static key added: ``key + static.to(key.dtype)``
    broadcast over (B, T) (``_add_static_lrid_source_key`` model.py:2046-2049,
    ``LRIDStaticKey.forward`` :286-288)."""
    return [k + static_keys[i].to(k.dtype) for i, k in enumerate(keys)]


def shared_static_key_table_ref(static_key: Tensor, n_src: int, dtype) -> Tensor:
    """The reference model's static source key as a per-source ``[n_src, R]``
    table: one shared ``[R]`` parameter (``LRIDStaticKey``, model.py:275-289)
    added to every source key except the embedding's (``_lrid_source`` with
    ``add_static_key=True``, model.py:2062-2063; the embedding source, :2070-2078,
    does not add it).  Row 0 is zero and every other row is the parameter cast
    to the key dtype, one cast per source as the model casts it once per call
    (:286-288), so autograd sums the per-source gradients into the parameter in
    its own dtype as the model's graph does."""
    zero = torch.zeros_like(static_key, dtype=dtype)
    return torch.stack([zero] + [static_key.to(dtype) for _ in range(n_src - 1)])


def lrid_block_accumulate_ref(projected: Tensor, partial_value, partial_key, output_dim: int, rank: int,
                              num_heads: int = 1, key_norm: bool = True, complete: bool = False,
                              partial_scale=1.0, value_norm: bool = False, scale_key: bool = False):
    """The eager sequence the fused block accumulation replaces: the fused
    projection split (``model.py:374-378``), the partial-block adds
    (``model.py:2377-2389, 2451-2463``) and, with ``complete``, the block source
    (``_lrid_block_source``, ``model.py:1003-1018``: the value scaled, or
    rms-normed with value_norm, and a scale tensor cast to the key dtype
    before it scales the key)."""
    out, key = lrid_fused_projection_split_ref(projected, output_dim, rank, num_heads, key_norm)
    value = out if partial_value is None else partial_value + out
    k = key if partial_key is None else partial_key + key
    if not complete:
        return value, k
    if value_norm:
        return norm(value), k
    s = _as_value_dtype(partial_scale, value)
    value = value * s
    if scale_key:
        k = k * (s.to(k.dtype) if isinstance(s, Tensor) else s)
    return value, k


def softmax_weights_ref(values_or_keys, query: Tensor, num_heads: int, logit_scale: float, key_norm: bool,
                        base: bool, source_counts=None, source_logit_biases=None) -> Tensor:
    """fp32 softmax weights [S,B,T,H] of a read (what the kernels save).

    For the base read pass the values (H must be 1) and ``base=True``.
    """
    if base:
        v = stack_sources(values_or_keys)
        k = norm(v) if key_norm else v
        logits = torch.einsum("d,sbtd->sbt", query.to(k.dtype), k).unsqueeze(-1)
    else:
        k = stack_sources(values_or_keys)
        S, B, T, R = k.shape
        H = int(num_heads)
        k = k.reshape(S, B, T, H, R // H)
        if key_norm:
            k = norm(k.float()).to(k.dtype)
        q = query.to(k.dtype)
        if q.dim() == 4:
            logits = torch.einsum("sbthr,bthr->sbth", k, q) * logit_scale
        else:
            logits = torch.einsum("sbthr,hr->sbth", k, q) * logit_scale
    bias = source_logit_bias(source_counts, source_logit_biases, logits.size(0), logits.device)
    if bias is not None:
        logits = logits + bias.view(-1, 1, 1, 1)
    return F.softmax(logits.float(), dim=0)


__all__ = [
    "norm",
    "stack_sources",
    "source_logit_bias",
    "attention_residual_read_torch",
    "attention_residual_read_ref",
    "attention_residual_average_read_ref",
    "lrid_attention_residual_read_torch",
    "lrid_attention_residual_read_ref",
    "gated_query_ref",
    "make_block_ends",
    "block_count_scale",
    "block_summary",
    "lrid_block_source",
    "block_count_logit_bias",
    "phase1_from_logits_ref",
    "lrid_block_accumulate_ref",
    "static_key_add_ref",
    "shared_static_key_table_ref",
    "lrid_value_key_projection_ref",
    "attention_residual_phase1_ref",
    "attention_residual_phase2_ref",
    "lrid_attention_residual_phase2_ref",
    "softmax_weights_ref",
]
