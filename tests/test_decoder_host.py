"""CPU tests of the whole-model decoder (no GPU): its schedule against the reference model.

The decoder runs with the oracle's read functions (``OracleOps``) and must
reproduce, bit for bit, the hidden state, loss and every parameter gradient
that the reference's ``OBPM`` produced for the same weights and tokens
(tests/golden/model_*.safetensors, written by make_model_golden.py from
``model.py:1808-2000`` and the baseline ``model.py:626-733``).  This pins the
block ends, the per-source logit cache, the count prior, the summary scaling,
the read norms and the phase boundaries -- everything around the kernels.
"""

import pytest
import torch

import attnres_decoder as AD
from decoder_util import OracleOps, build_from_case, lm_step, load_model_case, model_index

CASES = sorted(model_index())


@pytest.mark.parametrize("fold,fuse,fuse_read", [(True, True, True), (True, True, False), (True, False, False),
                                                (False, False, False)])
@pytest.mark.parametrize("name", CASES)
def test_decoder_matches_reference_model(name, fold, fuse, fuse_read):
    """Also pins the oracle's block accumulation (``fuse``: split, partial-block
    adds and block source composed in ``lrid_block_accumulate_ref``) and the
    schedule of the fused accumulate-and-read (``fuse_read``: the read at the
    site after a sublayer that does not end a block comes from that call)."""
    t, meta = load_model_case(name)
    model = build_from_case(t, meta, OracleOps, fold_block_summary=fold, fuse_block_accumulation=fuse,
                            fuse_accumulate_read=fuse_read)
    hidden, loss = lm_step(model, t["idx"], t["targets"])
    assert torch.equal(hidden, t["hidden"])
    assert torch.equal(loss.reshape(1), t["loss"])
    for pname, p in model.named_parameters():
        assert torch.equal(p.grad, t[f"grad.{pname}"]), pname


def test_state_dict_names_match_reference():
    for name in CASES:
        t, meta = load_model_case(name)
        model = AD.Decoder(AD.DecoderConfig(**{k: v for k, v in meta["config"].items()
                                                if k in AD.DecoderConfig.__dataclass_fields__}), ops=OracleOps)
        ref_keys = {k[len("state."):] for k in t if k.startswith("state.")}
        assert set(model.state_dict()) == ref_keys


def test_block_ends_known_answers():
    # model.py:828-836: ceil(2L * i / n)
    assert AD.block_ends(12, 6) == frozenset({4, 8, 12, 16, 20, 24})
    assert AD.block_ends(3, 2) == frozenset({3, 6})
    assert AD.block_ends(3, 4) == frozenset({2, 3, 5, 6})
    assert AD.block_ends(2, 10) == frozenset({1, 2, 3, 4})


def test_config_checks():
    with pytest.raises(NotImplementedError):
        AD.DecoderConfig(lrid_num_heads=2, lrid_rank=64)
    with pytest.raises(ValueError):
        AD.DecoderConfig(lrid_projection_rank=8, lrid_rank=16)
    with pytest.raises(ValueError):
        AD.DecoderConfig(norm_pos="middle")
    c = AD.DecoderConfig(lrid_rank=64)
    assert c.lrid_logit_scale == pytest.approx(0.125)
    assert c.hidden_dim == 4 * 768
    assert AD.DecoderConfig(use_attnres=False, lrid_num_heads=3).lrid_num_heads == 3


def test_config5_shapes_on_meta_device():
    # The whole-model configuration: 12 layers, d=768, 12 heads, MLP 4d, vocab 100277, 6 blocks, rank 64.
    cfg = AD.DecoderConfig(n_layer=12, n_head=12, n_embd=768, vocab_size=100277, block_size=1024,
                           attnres_num_blocks=6, lrid_rank=64)
    with torch.device("meta"):
        model = AD.Decoder(cfg)
    n = model.get_num_params()
    # embedding + lm head + 12 * (qkv + keyed out proj + fc1 + keyed fc2) + embedding key + 24 queries
    d, h, r, v = 768, 3072, 64, 100277
    expect = 2 * v * d + 12 * (3 * d * d + (d + r) * d + 2 * h * d + (d + r) * h) + r * d + 24 * r
    assert n == expect
