"""Decoder that runs the block LR-AttnRes training schedule on the HIP read kernels.

This is the whole-model harness around the fused read: a pre-norm decoder
(rotary attention through SDPA, SwiGLU MLP) whose residual stream is replaced
by block LR-AttnRes, following the reference model's fused training path
(``model.py:1808-2000``, selected by ``model.py:2013-2028``) for one depth
head:

* every sublayer's output projection emits ``D + rank`` columns; the last
  ``rank`` are its LR key, rms-normed (``model.py:316-388``);
* the embedding's key comes from its own projection (``model.py:391-428``,
  ``:2070-2078``);
* sublayer outputs and keys are summed into the live partial block; at each
  block end the summary ``partial * count**-alpha`` becomes a completed source
  (``model.py:1003-1028``, ``:1944-1955``) and its logits against every later
  read site's query are computed once (``model.py:1844-1873``), with the
  count prior ``beta * log(count)`` added (``model.py:1288-1300``);
* read sites between two block ends form one phase: one
  ``attention_residual_phase1_from_logits`` call reads the completed sources
  for all of them (``model.py:1888-1914``), and each site merges the live
  partial block in with ``lrid_attention_residual_phase2[_torch]``
  (``model.py:1919-1942``, ``:1616-1643``).

What differs from the reference's module: only this path is built (one depth
head, static queries, projection keys; no KV cache, no base AttnRes, no
split-sublayer mode), and the live partial block is handed to phase 2 raw
with ``partial_scale = count**-alpha`` instead of being multiplied out first
(``fold_block_summary``; the result is bit-identical, the kernel applies the
same rounding), and with pre-norm sublayers each sublayer's fused projection
goes straight into ``lrid_block_accumulate``, which splits it, norms the key,
adds both to the partial block and, at a block end, forms the block source in
one pass (``fuse_block_accumulation``; bit-identical too); a sublayer that does
not end a block also merges the grown block into the next site's read in that
pass (``lrid_block_accumulate_read``, ``fuse_accumulate_read``; bit-identical,
gradients included).  Module and parameter names match the reference's, so a
reference state dict for this configuration loads with ``load_state_dict``.

The read functions are looked up on ``ops`` (default: the HIP-backed
``attnres_ops`` module); any object with the same function names can stand in
for it.  With ``use_attnres=False`` the model is the reference's plain
pre-norm baseline (``model.py:626-733``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor, nn
from torch.nn import functional as F

try:
    from torch.nn.attention import SDPBackend, sdpa_kernel
except ImportError:  # pragma: no cover - torch >= 2.3 has it
    SDPBackend = None
    sdpa_kernel = None


def norm(x: Tensor) -> Tensor:
    """rms-norm over the last dim with torch's default eps (``model.py:28-31``)."""
    return F.rms_norm(x, (x.size(-1),))


def _norm_heads(x: Tensor, heads: int) -> Tensor:
    """Per-head rms-norm of a key (``model.py:34-37``)."""
    if heads == 1:
        return norm(x)
    shape = x.shape
    return norm(x.reshape(*shape[:-1], heads, shape[-1] // heads)).reshape(shape)


@dataclass
class DecoderConfig:
    """The reference's ``ModelConfig`` fields that this decoder reads (``model.py:52-208``).

    Defaults are the reference's; the whole-model benchmark sets its own
    shape (12 layers, d=768, 6 blocks, rank 64, ...).
    """

    block_size: int = 1024
    vocab_size: int = 100277
    n_layer: int = 12
    n_head: int = 12
    n_embd: int = 768
    mlp_hidden_dim: Optional[int] = None
    mlp_ratio: float = 4.0
    weight_tying: bool = False
    rope_theta: float = 500000.0
    norm_pos: str = "before"
    qk_norm: bool = True
    init_std: float = 0.02
    use_attnres: bool = True
    attnres_num_blocks: int = 8
    attnres_block_average: bool = True
    attnres_block_average_mode: str = "count"
    attnres_block_count_prior: bool = True
    attnres_key_norm: bool = True
    attn_res_query_norm: bool = False
    attn_res_query_init: str = "zero"
    attnres_training_torch_phase2: bool = True
    attnres_fuse_read_norm: bool = True
    lrid_rank: int = 64
    lrid_projection_rank: Optional[int] = None
    lrid_num_heads: int = 1
    lrid_use_logit_scale: bool = True
    lrid_logit_scale: Optional[float] = None
    fold_block_summary: bool = True
    fuse_block_accumulation: bool = True
    fuse_accumulate_read: bool = True

    def __post_init__(self):
        if self.norm_pos not in {"before", "after", "both"}:
            raise ValueError("norm_pos must be one of: before, after, both")
        if self.attnres_block_average_mode not in {"count", "sqrt"}:
            raise ValueError("attnres_block_average_mode must be one of: count, sqrt")
        if self.attn_res_query_init not in {"zero", "normal"}:
            raise ValueError("attn_res_query_init must be one of: zero, normal")
        if self.n_embd % self.n_head != 0:
            raise ValueError("n_embd must be divisible by n_head")
        if self.lrid_rank < 1:
            raise ValueError("lrid_rank must be >= 1")
        if self.lrid_projection_rank is None:
            self.lrid_projection_rank = self.lrid_rank
        if self.lrid_projection_rank < self.lrid_rank:
            raise ValueError("lrid_projection_rank must be >= lrid_rank")
        if self.use_attnres and self.lrid_num_heads != 1:
            raise NotImplementedError("the block LR training schedule runs one depth head (lrid_num_heads=1), "
                                      "as the reference's fused training path requires (model.py:2013-2028)")
        if self.attnres_num_blocks < 1:
            raise ValueError("attnres_num_blocks must be >= 1")
        if not self.lrid_use_logit_scale:
            self.lrid_logit_scale = 1.0
        elif self.lrid_logit_scale is None:
            self.lrid_logit_scale = 1.0 / math.sqrt(self.lrid_rank // self.lrid_num_heads)
        elif self.lrid_logit_scale <= 0.0:
            raise ValueError("lrid_logit_scale must be positive")

    @property
    def hidden_dim(self) -> int:
        return self.mlp_hidden_dim if self.mlp_hidden_dim is not None else int(self.n_embd * self.mlp_ratio)

    @property
    def block_alpha(self) -> float:
        """Summary exponent: ``count`` averaging -> 1, ``sqrt`` -> 0.5, none -> 0 (``model.py:869-874``)."""
        if not self.attnres_block_average:
            return 0.0
        return 0.5 if self.attnres_block_average_mode == "sqrt" else 1.0

    @property
    def block_beta(self) -> float:
        """Count-prior weight (``model.py:876-877``)."""
        return 1.0 if self.attnres_block_count_prior else 0.0


def block_ends(n_layer: int, num_blocks: int) -> frozenset:
    """Sublayer indices that close a block: ``ceil(2L * i / n)`` for ``i = 1..n`` (``model.py:828-836``)."""
    total = 2 * n_layer
    n = min(num_blocks, total)
    return frozenset(math.ceil(total * i / n) for i in range(1, n + 1))


class RotaryEmbedding(nn.Module):
    """Rotary position embedding on interleaved (even, odd) pairs (``model.py:291-313``).

    ``sin``/``cos`` are persistent buffers (they follow ``.to(dtype)``, so a
    bf16 model rotates with bf16 tables, as the reference's does).
    """

    def __init__(self, config: DecoderConfig):
        super().__init__()
        dim = config.n_embd // config.n_head
        inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, dim, 2) / dim))
        angle = torch.outer(torch.arange(config.block_size), inv_freq)
        self.register_buffer("sin", angle.sin()[None, None])
        self.register_buffer("cos", angle.cos()[None, None])

    def rotate(self, x: Tensor) -> Tensor:
        T = x.size(-2)
        sin = self.sin[:, :, :T]
        cos = self.cos[:, :, :T]
        even, odd = x[..., 0::2], x[..., 1::2]
        return torch.stack([cos * even - sin * odd, sin * even + cos * odd], dim=-1).flatten(-2)


class KeyedOutputProjection(nn.Module):
    """Output projection that also emits the sublayer's LR key (``model.py:316-388``, key-only form).

    One GEMM produces ``D + projection_rank`` columns; the first ``rank`` of
    the extra columns are the key, rms-normed per depth head when key norm is
    on.  The split is ``ops.lrid_fused_projection_split`` (one HIP pass each
    way, in place of slicing, copying and norming in separate kernels).
    """

    def __init__(self, config: DecoderConfig, input_dim: int, output_dim: int, ops):
        super().__init__()
        self.output_dim = output_dim
        self.rank = config.lrid_rank
        self.heads = config.lrid_num_heads
        self.key_norm = config.attnres_key_norm
        self.ops = ops
        self.proj = nn.Linear(input_dim, output_dim + config.lrid_projection_rank, bias=False)
        # set by the decoder when it folds the projection into the partial block itself
        self.emit_projection = False

    def forward(self, x: Tensor):
        """``(output, key)``, or ``(projection, None)`` with ``emit_projection``."""
        if self.emit_projection:
            return self.proj(x), None
        return self.ops.lrid_fused_projection_split(self.proj(x), self.output_dim, self.rank, self.heads,
                                                    self.key_norm)


class SourceKeyProjection(nn.Module):
    """Key of the embedding source: ``rms_norm(x @ W)`` (``model.py:391-423``, projection form)."""

    def __init__(self, config: DecoderConfig):
        super().__init__()
        self.heads = config.lrid_num_heads
        self.key_norm = config.attnres_key_norm
        self.proj = nn.Linear(config.n_embd, config.lrid_rank, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        key = self.proj(x)
        return _norm_heads(key, self.heads) if self.key_norm else key


def _attend(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Causal SDPA.  For 16-bit inputs on the GPU only the fused flash /
    memory-efficient kernels are allowed: the math path forms 16-bit batched
    products on transposed operands, which this build does not run."""
    if q.is_cuda and q.dtype != torch.float32 and sdpa_kernel is not None:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, is_causal=True)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


class MultiHeadAttention(nn.Module):
    """Causal self-attention with qk-norm and rotary positions (``model.py:430-569``)."""

    def __init__(self, config: DecoderConfig, ops=None):
        super().__init__()
        self.n_head = config.n_head
        self.n_embd = config.n_embd
        self.head_dim = config.n_embd // config.n_head
        self.qk_norm = config.qk_norm
        self.keyed = config.use_attnres
        self.rope = RotaryEmbedding(config)
        self.c_attn = nn.Linear(config.n_embd, 3 * config.n_embd, bias=False)
        if self.keyed:
            self.c_proj = KeyedOutputProjection(config, config.n_embd, config.n_embd, ops)
        else:
            self.c_proj = nn.Linear(config.n_embd, config.n_embd, bias=False)

    def forward(self, x: Tensor):
        B, T, C = x.shape
        q, k, v = self.c_attn(x).split(C, dim=2)
        q = q.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        k = k.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        v = v.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        if self.qk_norm:
            q = norm(q)
            k = norm(k)
        q = self.rope.rotate(q)
        k = self.rope.rotate(k)
        y = _attend(q, k, v).transpose(1, 2).contiguous().view(B, T, C)
        if self.keyed:
            return self.c_proj(y)
        return self.c_proj(y), None


class MLP(nn.Module):
    """SwiGLU MLP: ``fc2(silu(gate) * up)`` with ``[up, gate] = fc1(x)`` (``model.py:572-589``)."""

    def __init__(self, config: DecoderConfig, ops=None):
        super().__init__()
        hidden = config.hidden_dim
        self.keyed = config.use_attnres
        self.fc1 = nn.Linear(config.n_embd, 2 * hidden, bias=False)
        if self.keyed:
            self.fc2 = KeyedOutputProjection(config, hidden, config.n_embd, ops)
        else:
            self.fc2 = nn.Linear(hidden, config.n_embd, bias=False)

    def forward(self, x: Tensor):
        up, gate = self.fc1(x).chunk(2, dim=-1)
        h = F.silu(gate) * up
        if self.keyed:
            return self.fc2(h)
        return self.fc2(h), None


class Block(nn.Module):
    """One decoder layer: an attention sublayer and an MLP sublayer (``model.py:626-732``).

    ``attention``/``mlp`` return ``(output, lr_key)``; the caller owns the
    residual stream (plain addition for the baseline, AttnRes reads otherwise).
    """

    def __init__(self, config: DecoderConfig, ops=None):
        super().__init__()
        self.norm_pos = config.norm_pos
        self.attn = MultiHeadAttention(config, ops)
        self.mlp = MLP(config, ops)

    def _sublayer(self, fn, x: Tensor, x_is_normalized: bool):
        if self.norm_pos in {"before", "both"} and not x_is_normalized:
            x = norm(x)
        out, key = fn(x)
        if self.norm_pos in {"after", "both"}:
            out = norm(out)
        return out, key

    def attention(self, x: Tensor, x_is_normalized: bool = False):
        return self._sublayer(self.attn, x, x_is_normalized)

    def feed_forward(self, x: Tensor, x_is_normalized: bool = False):
        return self._sublayer(self.mlp, x, x_is_normalized)


def _default_ops():
    import attnres_ops
    return attnres_ops


class Decoder(nn.Module):
    """Decoder LM with block LR-AttnRes residuals (or the plain pre-norm baseline).

    ``forward(idx, return_hidden=False)`` returns the final normed hidden
    state ``[B,T,D]`` or the LM logits ``[B,T,vocab]``.
    """

    def __init__(self, config: DecoderConfig, ops=None):
        super().__init__()
        self.config = config
        self.ops = ops if ops is not None else (_default_ops() if config.use_attnres else None)
        self.block_ends = block_ends(config.n_layer, config.attnres_num_blocks) if config.use_attnres else None
        modules = dict(
            wte=nn.Embedding(config.vocab_size, config.n_embd),
            layers=nn.ModuleList([Block(config, self.ops) for _ in range(config.n_layer)]),
        )
        if config.use_attnres:
            modules["lrid_embedding_key"] = SourceKeyProjection(config)
            head_dim = config.lrid_rank // config.lrid_num_heads
            modules["lrid_queries"] = nn.ParameterList(
                [nn.Parameter(torch.empty(config.lrid_num_heads, head_dim)) for _ in range(2 * config.n_layer)])
        self.transformer = nn.ModuleDict(modules)
        if self._fused_accumulation():
            for layer in self.transformer.layers:
                layer.attn.c_proj.emit_projection = True
                layer.mlp.fc2.emit_projection = True
        if not config.weight_tying:
            self.lm_head = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self.reset_parameters()

    # -- parameters ---------------------------------------------------------

    def reset_parameters(self):
        """Normal(0, init_std) for every projection and the embedding; queries
        zero or normal per ``attn_res_query_init`` (``model.py:2161-2196``)."""
        std = self.config.init_std
        for module in self.modules():
            if isinstance(module, (nn.Linear, nn.Embedding)):
                nn.init.normal_(module.weight, mean=0.0, std=std)
        if self.config.use_attnres:
            for query in self.transformer.lrid_queries:
                if self.config.attn_res_query_init == "zero":
                    nn.init.zeros_(query)
                else:
                    nn.init.normal_(query, mean=0.0, std=std)

    def get_num_params(self) -> int:
        return sum(p.numel() for p in self.parameters())

    # -- forward ------------------------------------------------------------

    def forward(self, idx: Tensor, return_hidden: bool = False) -> Tensor:
        _, T = idx.shape
        if T > self.config.block_size:
            raise ValueError(f"token length {T} exceeds block_size {self.config.block_size}")
        x = self.transformer.wte(idx)
        if self.config.use_attnres:
            x = self._forward_block_lrid(x)
        else:
            x = self._forward_baseline(x)
        if return_hidden:
            return x
        if self.config.weight_tying:
            return F.linear(x, self.transformer.wte.weight, None)
        return self.lm_head(x)

    def _forward_baseline(self, x: Tensor) -> Tensor:
        """Plain residual stream ``x += sublayer(x)`` and a final norm (``model.py:704-733``, ``:2642-2643``)."""
        for block in self.transformer.layers:
            out, _ = block.attention(x)
            x = x + out
            out, _ = block.feed_forward(x)
            x = x + out
        return norm(x)

    def _fused_read_norm(self) -> bool:
        """Reads return the normed input of the next sublayer (``model.py:2238-2244``)."""
        c = self.config
        return c.norm_pos == "before" and c.attnres_fuse_read_norm and c.lrid_num_heads == 1

    def _fused_accumulation(self) -> bool:
        """Sublayers hand over their projection and ``lrid_block_accumulate`` grows the
        partial block from it; only for pre-norm sublayers (a post-norm acts on the
        output before it is added)."""
        c = self.config
        return c.use_attnres and c.fuse_block_accumulation and c.norm_pos == "before"

    def _block_scale(self, count: int) -> float:
        """``count ** -alpha`` (``model.py:955-959``, ``:979-988``)."""
        return float(count) ** (-self.config.block_alpha)

    def _count_bias(self, count: int) -> float:
        """``beta * log(count)``, zero for a count of 1 (``model.py:1045-1069``)."""
        beta = self.config.block_beta
        if count == 1 or beta == 0.0:
            return 0.0
        return beta * math.log(float(count))

    def _forward_block_lrid(self, x: Tensor) -> Tensor:
        c = self.config
        ops = self.ops
        n_sites = 2 * c.n_layer
        ends = sorted(self.block_ends)
        rank = c.lrid_rank
        fused_norm = self._fused_read_norm()
        phase2 = (ops.lrid_attention_residual_phase2_torch if c.attnres_training_torch_phase2
                  else ops.lrid_attention_residual_phase2)
        queries = torch.stack([q.reshape(rank) for q in self.transformer.lrid_queries], dim=0)
        if c.attn_res_query_norm:
            queries = norm(queries.float()).to(x.dtype)
        else:
            queries = queries.to(x.dtype)
        queries = queries.contiguous()       # [2L, rank]; row i-1 is read site i's query

        def next_end(site: int) -> int:
            for e in ends:
                if e > site:
                    return e
            return site + 1

        def site_logits(value: Tensor, key: Tensor, first_read: int, count: int) -> dict:
            """Logits of one completed source against read sites ``first_read..2L`` (``model.py:1838-1873``),
            as ``{phase start: [Q_phase, B, T]}`` for the block phases that will read them."""
            spans, s = [], first_read
            while s <= n_sites:
                spans.append((s, next_end(s)))
                s = spans[-1][1]
            k = key.reshape(key.size(0), key.size(1), rank)
            parts = ops.lrid_site_logits(k, queries, first_read - 1, [e - b for b, e in spans], c.lrid_logit_scale,
                                         self._count_bias(count), c.attnres_key_norm)
            return {b: t for (b, _), t in zip(spans, parts)}

        emb_key = self.transformer.lrid_embedding_key(x)
        done_values = [x]
        done_logits = [site_logits(x, emb_key, 1, 1)]
        partial = partial_key = None
        count = 0
        phase = None                          # (first, end, outputs, lses)

        def ensure_phase(site: int):
            nonlocal phase
            if phase is not None and phase[0] <= site < phase[1]:
                return
            end = next_end(site)
            if len(done_values) == 1:
                # One completed source: its logit is its own lse and the read is the source itself.
                # The expand/unbind views keep the reference's gradient summation order for it.
                lse = done_logits[0][site].float()
                outs = done_values[0].unsqueeze(0).expand(lse.size(0), -1, -1, -1).unbind(0)
                phase = (site, end, outs, lse.unbind(0))
                return
            outs, lses = ops.lrid_block_phase1(done_values, [lg[site] for lg in done_logits])
            phase = (site, end, outs, lses)

        def summary(value: Tensor, key: Tensor, n: int):
            """Completed LR block source (``model.py:1003-1018``)."""
            scale = self._block_scale(n)
            value = value * scale
            if not c.attnres_key_norm:
                key = key * scale
            return value, key

        def read(site: int) -> Tensor:
            if site == 0:
                out = done_values[0]
                return norm(out) if fused_norm else out
            ensure_phase(site)
            i = site - phase[0]
            inter, lse = phase[2][i], phase[3][i]
            if partial is None:
                return norm(inter) if fused_norm else inter
            # site i reads row i - 1 of the query bank; the merge takes the bank and
            # the row, so the bank's gradient comes back without a select's fill and copy
            pkey = partial_key.reshape(partial_key.size(0), partial_key.size(1), rank)
            if c.fold_block_summary:
                return phase2(partial, pkey, queries, inter, lse, c.lrid_logit_scale, c.attnres_key_norm,
                              normalize_output=fused_norm, logit_bias=self._count_bias(count),
                              partial_scale=self._block_scale(count), scale_key=not c.attnres_key_norm,
                              query_row=site - 1)
            value, key = summary(partial, pkey, count)
            return phase2(value, key, queries, inter, lse, c.lrid_logit_scale, c.attnres_key_norm,
                          normalize_output=fused_norm, logit_bias=self._count_bias(count), query_row=site - 1)

        def add(out: Tensor, key: Optional[Tensor], site_after: int) -> Optional[Tensor]:
            """Grows the partial block by a sublayer's output; returns the read at
            ``site_after`` when the accumulation produced it as well."""
            nonlocal partial, partial_key, count, phase
            complete = site_after in self.block_ends
            if key is None and not complete and c.fuse_accumulate_read and c.fold_block_summary:
                # the grown block and the next site's merge of it in one pass (model.py:2377-2389
                # then :1919-1942): the read() below, on the block this call grows
                ensure_phase(site_after)
                i = site_after - phase[0]
                n = count + 1
                partial, partial_key, h = ops.lrid_block_accumulate_read(
                    out, partial, partial_key, queries, phase[2][i], phase[3][i], c.n_embd, rank,
                    c.lrid_logit_scale, c.lrid_num_heads, c.attnres_key_norm,
                    lerp=c.attnres_training_torch_phase2, normalize_output=fused_norm,
                    logit_bias=self._count_bias(n), partial_scale=self._block_scale(n),
                    scale_key=not c.attnres_key_norm, query_row=site_after - 1)
                count = n
                return h
            if key is None:
                # ``out`` is the sublayer's fused projection: split, key norm, partial-block add
                # and, at a block end, the block source in one pass (model.py:2377-2389, 1003-1018)
                value, key = ops.lrid_block_accumulate(
                    out, partial, partial_key, c.n_embd, rank, c.lrid_num_heads, c.attnres_key_norm,
                    complete=complete, partial_scale=self._block_scale(count + 1) if complete else 1.0,
                    scale_key=complete and not c.attnres_key_norm)
                if not complete:
                    partial, partial_key, count = value, key, count + 1
                    return None
                count += 1
            else:
                if partial is None:
                    partial, partial_key, count = out, key, 1
                else:
                    partial, partial_key, count = partial + out, partial_key + key, count + 1
                if not complete:
                    return None
                value, key = summary(partial, partial_key, count)
            done_values.append(value)
            done_logits.append(site_logits(value, key, site_after, count))
            partial = partial_key = None
            count = 0
            phase = None
            return None

        h = read(0)
        for layer_idx, block in enumerate(self.transformer.layers):
            out, key = block.attention(h, x_is_normalized=fused_norm)
            site = 2 * layer_idx + 1
            h = add(out, key, site)
            if h is None:
                h = read(site)
            out, key = block.feed_forward(h, x_is_normalized=fused_norm)
            h = add(out, key, site + 1)
            if h is None:
                h = read(site + 1)
        return h if fused_norm else norm(h)
