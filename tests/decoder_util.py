"""Helpers for the whole-model decoder tests: oracle-backed read functions and golden-case loading."""

from __future__ import annotations

import json
import os

import torch
from safetensors.torch import load_file
from torch.nn import functional as F

import attnres_decoder as AD
from oracle import attnres_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _phase2(pv, pk, q, inter, lse, scale, key_norm, normalize_output, logit_bias, partial_scale, scale_key, merge):
    if partial_scale is not None:
        pv = pv * partial_scale
        if scale_key:
            pk = pk * partial_scale
    return O.lrid_attention_residual_phase2_ref(pv, pk, q, inter, lse, scale, key_norm, normalize_output,
                                                logit_bias, merge=merge)


class OracleOps:
    """The read functions the decoder calls, answered by the eager oracle (CPU tensors)."""

    @staticmethod
    def attention_residual_phase1_from_logits(values, logits, force_triton=False, normalize_output=False):
        return O.phase1_from_logits_ref(values, logits, normalize_output)

    @staticmethod
    def lrid_site_logits(key, queries, first, sizes, logit_scale, logit_bias=0.0, key_norm=True):
        return O.lrid_site_logits_ref(key, queries, first, sizes, logit_scale, logit_bias, key_norm)

    @staticmethod
    def lrid_block_phase1(values, source_logits):
        return O.lrid_block_phase1_ref(values, source_logits)

    @staticmethod
    def lrid_attention_residual_phase2_torch(pv, pk, q, inter, lse, scale, key_norm, normalize_output=False,
                                             logit_bias=0.0, partial_scale=None, scale_key=False, query_row=None):
        if query_row is not None:  # the reference reads the site's row of the bank
            q = q[query_row]
        return _phase2(pv, pk, q, inter, lse, scale, key_norm, normalize_output, logit_bias, partial_scale,
                       scale_key, "lerp")

    @staticmethod
    def lrid_fused_projection_split(projected, output_dim, rank, num_heads=1, key_norm=True):
        return O.lrid_fused_projection_split_ref(projected, output_dim, rank, num_heads, key_norm)

    @staticmethod
    def lrid_block_accumulate(projected, partial_value, partial_key, output_dim, rank, num_heads=1, key_norm=True,
                              complete=False, partial_scale=1.0, value_norm=False, scale_key=False):
        return O.lrid_block_accumulate_ref(projected, partial_value, partial_key, output_dim, rank, num_heads,
                                           key_norm, complete, partial_scale, value_norm, scale_key)

    @staticmethod
    def lrid_block_accumulate_read(projected, partial_value, partial_key, query, inter, lse, output_dim, rank,
                                   logit_scale, num_heads=1, key_norm=True, merge_key_norm=None, lerp=False,
                                   normalize_output=False, logit_bias=0.0, partial_scale=None, scale_key=False,
                                   query_row=None):
        """The composition the fused op stands for: the accumulation, then the next site's merge."""
        value, key = O.lrid_block_accumulate_ref(projected, partial_value, partial_key, output_dim, rank, num_heads,
                                                 key_norm)
        q = query[query_row] if query_row is not None else query
        mkn = key_norm if merge_key_norm is None else merge_key_norm
        out = _phase2(value, key, q, inter, lse, logit_scale, mkn, normalize_output, logit_bias, partial_scale,
                      scale_key, "lerp" if lerp else "addcmul")
        return value, key, out

    @staticmethod
    def lrid_attention_residual_phase2(pv, pk, q, inter, lse, scale, key_norm, force_triton=False,
                                       normalize_output=False, logit_bias=0.0, partial_scale=None, scale_key=False,
                                       query_row=None):
        if query_row is not None:  # the reference reads the site's row of the bank
            q = q[query_row]
        return _phase2(pv, pk, q, inter, lse, scale, key_norm, normalize_output, logit_bias, partial_scale,
                       scale_key, "addcmul")


def model_index():
    with open(os.path.join(GOLDEN, "model_index.json")) as f:
        return json.load(f)


def load_model_case(name):
    meta = model_index()[name]
    return load_file(os.path.join(GOLDEN, f"{name}.safetensors")), meta


def decoder_config(meta_config, **overrides):
    fields = set(AD.DecoderConfig.__dataclass_fields__)
    cfg = {k: v for k, v in meta_config.items() if k in fields}
    cfg.update(overrides)
    return AD.DecoderConfig(**cfg)


def build_from_case(tensors, meta, ops, device="cpu", **overrides):
    model = AD.Decoder(decoder_config(meta["config"], **overrides), ops=ops)
    if meta["dtype"] == "bf16":
        model.to(torch.bfloat16)
    state = {k[len("state."):]: v for k, v in tensors.items() if k.startswith("state.")}
    model.load_state_dict(state, strict=True)
    return model.to(device)


def lm_step(model, idx, targets):
    """Forward to the hidden state, LM cross-entropy (fp32 logits), backward."""
    hidden = model(idx, return_hidden=True)
    logits = model.lm_head(hidden)
    loss = F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.view(-1))
    loss.backward()
    return hidden.detach(), loss.detach()
