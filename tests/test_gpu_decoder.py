"""GPU tests of the whole-model decoder with its AttnRes reads on the HIP kernels.

* the reference model's golden cases (tests/golden/model_*.safetensors) run on
  the GPU with the HIP reads: hidden state, loss and every parameter gradient
  match the reference model's CPU values within a model-level bound (the
  GEMMs and SDPA run on the GPU too, so this is not bit-exact);
* every read the decoder makes at the whole-model shape (12 layers, d=768,
  6 blocks, rank 64, T=1024) is checked against the oracle on the same
  model-produced inputs, at the kernel bound of gpu_util.assert_close;
* the decoder with HIP reads on the GPU agrees with the same decoder with
  oracle reads on the CPU, forward and backward, on a mid-size bf16 model;
* one full-size training step (B=16, T=1024, vocab 100277) runs with finite
  loss and gradients, as the whole-model benchmark does.
"""

import math

import pytest
import torch

import _attnres_hip as H
import attnres_decoder as AD
import attnres_ops as ops
from oracle import attnres_oracle as O
from decoder_util import OracleOps, build_from_case, lm_step, load_model_case, model_index
from gpu_util import DEV, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


def _rel_l2(a, e):
    a = a.detach().float().cpu()
    e = e.detach().float().cpu()
    return float((a - e).norm() / e.norm().clamp_min(1e-30))


def _model_bound(dtype):
    # Whole-model comparison GPU vs CPU: relative L2 error of each tensor.
    return 1e-4 if dtype == "fp32" else 3e-2


LR_CASES = [n for n, m in sorted(model_index().items()) if m["config"].get("use_attnres")]


@pytest.mark.parametrize("name", LR_CASES)
def test_decoder_golden_on_gpu(name):
    t, meta = load_model_case(name)
    model = build_from_case(t, meta, None, device=DEV)
    hidden, loss = lm_step(model, t["idx"].to(DEV), t["targets"].to(DEV))
    bound = _model_bound(meta["dtype"])
    assert _rel_l2(hidden, t["hidden"]) <= bound
    assert abs(float(loss) - float(t["loss"][0])) <= bound * abs(float(t["loss"][0]))
    for pname, p in model.named_parameters():
        assert p.grad is not None, pname
        assert _rel_l2(p.grad, t[f"grad.{pname}"]) <= bound, pname


class CheckingOps:
    """HIP reads, each checked against the oracle on CPU copies of its inputs (forward only)."""

    def __init__(self):
        self.calls = []

    def attention_residual_phase1_from_logits(self, values, logits, force_triton=False, normalize_output=False):
        out, lse = ops.attention_residual_phase1_from_logits(values, logits, normalize_output=normalize_output)
        e_out, e_lse = O.phase1_from_logits_ref([v.cpu() for v in values], logits.cpu(), normalize_output)
        assert_close(out, e_out, values[0].dtype, "phase1 out")
        assert_close(lse, e_lse, values[0].dtype, "phase1 lse")
        self.calls.append(("phase1", len(values), logits.size(0)))
        return out, lse

    def lrid_block_phase1(self, values, source_logits):
        outs, lses = ops.lrid_block_phase1(values, source_logits)
        e_outs, e_lses = O.lrid_block_phase1_ref([v.cpu() for v in values], [lg.cpu() for lg in source_logits])
        for a, e in zip(outs, e_outs):
            assert_close(a, e, values[0].dtype, "phase1 out")
        for a, e in zip(lses, e_lses):
            assert_close(a, e, values[0].dtype, "phase1 lse")
        self.calls.append(("phase1", len(values), len(outs)))
        return outs, lses

    def lrid_site_logits(self, key, queries, first, sizes, logit_scale, logit_bias=0.0, key_norm=True):
        parts = ops.lrid_site_logits(key, queries, first, sizes, logit_scale, logit_bias, key_norm)
        e_parts = O.lrid_site_logits_ref(key.cpu(), queries.cpu(), first, sizes, logit_scale, logit_bias, key_norm)
        for a, e in zip(parts, e_parts):
            assert a.dtype == e.dtype
            assert_close(a, e, key.dtype, "site logits")
        self.calls.append(("site_logits", first, tuple(sizes)))
        return parts

    def lrid_fused_projection_split(self, projected, output_dim, rank, num_heads=1, key_norm=True):
        out, key = ops.lrid_fused_projection_split(projected, output_dim, rank, num_heads, key_norm)
        e_out, e_key = O.lrid_fused_projection_split_ref(projected.cpu(), output_dim, rank, num_heads, key_norm)
        assert torch.equal(out.cpu(), e_out)
        assert_close(key, e_key, projected.dtype, "key")
        self.calls.append(("split",))
        return out, key

    def lrid_block_accumulate(self, projected, partial_value, partial_key, output_dim, rank, num_heads=1,
                              key_norm=True, complete=False, partial_scale=1.0, value_norm=False, scale_key=False):
        value, key = ops.lrid_block_accumulate(projected, partial_value, partial_key, output_dim, rank, num_heads,
                                               key_norm, complete, partial_scale, value_norm, scale_key)
        cpu = lambda t: t.cpu() if t is not None else None  # noqa: E731
        e_value, e_key = O.lrid_block_accumulate_ref(cpu(projected), cpu(partial_value), cpu(partial_key), output_dim,
                                                     rank, num_heads, key_norm, complete, partial_scale, value_norm,
                                                     scale_key)
        assert torch.equal(value.cpu(), e_value)
        assert_close(key, e_key, projected.dtype, "accumulated key")
        self.calls.append(("accumulate", complete))
        return value, key

    def lrid_block_accumulate_read(self, projected, partial_value, partial_key, query, inter, lse, output_dim, rank,
                                   logit_scale, num_heads=1, key_norm=True, merge_key_norm=None, lerp=False,
                                   normalize_output=False, logit_bias=0.0, partial_scale=None, scale_key=False,
                                   query_row=None):
        kw = dict(merge_key_norm=merge_key_norm, lerp=lerp, normalize_output=normalize_output,
                  logit_bias=logit_bias, partial_scale=partial_scale, scale_key=scale_key, query_row=query_row)
        value, key, out = ops.lrid_block_accumulate_read(projected, partial_value, partial_key, query, inter, lse,
                                                         output_dim, rank, logit_scale, num_heads, key_norm, **kw)
        cpu = lambda t: t.cpu() if t is not None else None  # noqa: E731
        e_value, e_key, e_out = OracleOps.lrid_block_accumulate_read(
            cpu(projected), cpu(partial_value), cpu(partial_key), cpu(query), cpu(inter), cpu(lse), output_dim, rank,
            logit_scale, num_heads, key_norm, **kw)
        assert torch.equal(value.cpu(), e_value)
        assert_close(key, e_key, projected.dtype, "accumulated key")
        assert_close(out, e_out, projected.dtype, "fused read")
        self.calls.append(("accumulate", False))
        self.calls.append(("phase2", "lerp" if lerp else "addcmul", partial_scale))
        return value, key, out

    def _phase2(self, fn, merge, pv, pk, q, inter, lse, scale, key_norm, normalize_output, logit_bias,
                partial_scale, scale_key, query_row=None):
        out = fn(pv, pk, q, inter, lse, scale, key_norm, normalize_output=normalize_output, logit_bias=logit_bias,
                 partial_scale=partial_scale, scale_key=scale_key, query_row=query_row)
        if query_row is not None:
            q = q[query_row]
        epv, epk = pv.cpu(), pk.cpu()
        if partial_scale is not None:
            epv = epv * partial_scale
            if scale_key:
                epk = epk * partial_scale
        e = O.lrid_attention_residual_phase2_ref(epv, epk, q.cpu(), inter.cpu(), lse.cpu(), scale, key_norm,
                                                 normalize_output, logit_bias, merge=merge)
        assert_close(out, e, pv.dtype, f"phase2 ({merge})")
        self.calls.append(("phase2", merge, partial_scale))
        return out

    def lrid_attention_residual_phase2_torch(self, pv, pk, q, inter, lse, scale, key_norm, normalize_output=False,
                                             logit_bias=0.0, partial_scale=None, scale_key=False, query_row=None):
        return self._phase2(ops.lrid_attention_residual_phase2_torch, "lerp", pv, pk, q, inter, lse, scale,
                            key_norm, normalize_output, logit_bias, partial_scale, scale_key, query_row)

    def lrid_attention_residual_phase2(self, pv, pk, q, inter, lse, scale, key_norm, force_triton=False,
                                       normalize_output=False, logit_bias=0.0, partial_scale=None, scale_key=False,
                                       query_row=None):
        return self._phase2(ops.lrid_attention_residual_phase2, "addcmul", pv, pk, q, inter, lse, scale, key_norm,
                            normalize_output, logit_bias, partial_scale, scale_key, query_row)


def _config5(**kw):
    base = dict(n_layer=12, n_head=12, n_embd=768, vocab_size=100277, block_size=1024, attnres_num_blocks=6,
                lrid_rank=64, attn_res_query_init="normal")
    base.update(kw)
    return AD.DecoderConfig(**base)


@pytest.mark.parametrize("torch_phase2,fuse_read", [(True, False), (False, False), (True, True), (False, True)])
def test_config5_every_read_matches_oracle(torch_phase2, fuse_read):
    torch.manual_seed(5)
    checker = CheckingOps()
    with torch.device(DEV):
        model = AD.Decoder(_config5(vocab_size=4096, attnres_training_torch_phase2=torch_phase2,
                                    fuse_accumulate_read=fuse_read), ops=checker)
    model.to(torch.bfloat16)
    idx = torch.randint(0, 4096, (2, 1024), device=DEV)
    with torch.no_grad():
        hidden = model(idx, return_hidden=True)
    assert torch.isfinite(hidden.float()).all()
    n1 = sum(1 for c in checker.calls if c[0] == "phase1")
    n2 = sum(1 for c in checker.calls if c[0] == "phase2")
    # 24 read sites + the final read over 6 blocks of 4: phase 1 at sites 4, 8, ..., 24; phase 2 at the
    # three in-block sites of each block (site 1..3 read the embedding alone in phase 1).
    assert n1 == 6
    assert n2 == 18
    # the embedding and the 6 block sources each get their logits once, split into the phases after them
    assert sum(1 for c in checker.calls if c[0] == "site_logits") == 7
    # every sublayer grows the partial block in one fused pass; 6 of them end a block
    assert sum(1 for c in checker.calls if c[0] == "accumulate") == 24
    assert sum(1 for c in checker.calls if c == ("accumulate", True)) == 6


@pytest.mark.parametrize("fuse_read", [True, False])
def test_fused_block_accumulation_is_bit_identical_to_the_split_path(fuse_read):
    """The decoder with sublayer projections folded by lrid_block_accumulate
    (with fuse_read, by lrid_block_accumulate_read together with the next
    site's merge) against the same weights with the split + eager adds: hidden
    state, loss and every gradient bit for bit (the kernels round as the eager
    ops do)."""
    cfg = dict(n_layer=4, n_head=4, n_embd=256, mlp_hidden_dim=512, vocab_size=1000, block_size=256,
               attnres_num_blocks=3, lrid_rank=32, attn_res_query_init="normal")
    torch.manual_seed(13)
    with torch.device(DEV):
        fused = AD.Decoder(AD.DecoderConfig(**cfg, fuse_block_accumulation=True,
                                            fuse_accumulate_read=fuse_read)).to(torch.bfloat16)
        split = AD.Decoder(AD.DecoderConfig(**cfg, fuse_block_accumulation=False)).to(torch.bfloat16)
    split.load_state_dict(fused.state_dict())
    g = torch.Generator().manual_seed(14)
    idx = torch.randint(0, 1000, (2, 256), generator=g).to(DEV)
    tgt = torch.randint(0, 1000, (2, 256), generator=g).to(DEV)
    h_f, l_f = lm_step(fused, idx, tgt)
    h_s, l_s = lm_step(split, idx, tgt)
    assert torch.equal(h_f, h_s)
    assert torch.equal(l_f, l_s)
    # a second split step tells which gradients the GPU itself reproduces bit for bit
    # (the attention backward may sum in a varying order); those must match exactly
    first = {n: p.grad.clone() for n, p in split.named_parameters()}
    split.zero_grad(set_to_none=True)
    lm_step(split, idx, tgt)
    split_params = dict(split.named_parameters())
    n_exact = 0
    for pname, p in fused.named_parameters():
        again = split_params[pname].grad
        if torch.equal(first[pname], again):
            assert torch.equal(p.grad, again), pname
            n_exact += 1
        else:
            assert _rel_l2(p.grad, again) <= 1e-2, pname
    # at least the last MLP projection and the read queries sit after every attention backward
    assert n_exact >= 1


def test_decoder_hip_vs_oracle_cpu_mid_size():
    cfg = dict(n_layer=4, n_head=4, n_embd=256, mlp_hidden_dim=512, vocab_size=1000, block_size=256,
               attnres_num_blocks=3, lrid_rank=32, attn_res_query_init="normal")
    torch.manual_seed(11)
    ref = AD.Decoder(AD.DecoderConfig(**cfg), ops=OracleOps).to(torch.bfloat16)
    hip = AD.Decoder(AD.DecoderConfig(**cfg)).to(torch.bfloat16)
    hip.load_state_dict(ref.state_dict())
    hip.to(DEV)
    g = torch.Generator().manual_seed(12)
    idx = torch.randint(0, 1000, (2, 256), generator=g)
    tgt = torch.randint(0, 1000, (2, 256), generator=g)
    h_ref, l_ref = lm_step(ref, idx, tgt)
    h_hip, l_hip = lm_step(hip, idx.to(DEV), tgt.to(DEV))
    assert _rel_l2(h_hip, h_ref) <= 3e-2
    assert abs(float(l_hip) - float(l_ref)) <= 1e-2 * abs(float(l_ref))
    ref_params = dict(ref.named_parameters())
    for pname, p in hip.named_parameters():
        assert _rel_l2(p.grad, ref_params[pname].grad) <= 5e-2, pname


def test_config5_full_training_step():
    torch.manual_seed(7)
    with torch.device(DEV):
        model = AD.Decoder(_config5())
    model.to(torch.bfloat16)
    idx = torch.randint(0, 100277, (16, 1024), device=DEV)
    tgt = torch.randint(0, 100277, (16, 1024), device=DEV)
    hidden, loss = lm_step(model, idx, tgt)
    assert hidden.shape == (16, 1024, 768)
    assert math.isfinite(float(loss))
    # random init: the loss is near log(vocab)
    assert abs(float(loss) - math.log(100277)) < 1.0
    for pname, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), pname
    assert float(model.transformer.lrid_queries[5].grad.float().abs().sum()) > 0.0
