"""Write whole-model golden vectors (tests/golden/model_*.safetensors) from the reference's model.

Run in the build container only (it needs ``/root/reference``, which does not
exist on the GPU box)::

    python tests/golden/make_model_golden.py [--reference /root/reference]

It imports the reference's ``model`` module (``ModelConfig``, ``OBPM``), builds
small seeded models on the CPU and runs one forward + backward of each:

* block LR-AttnRes on the fused training path (``model.py:1808-2000``), whose
  phase functions take their eager CPU branches (``attnres_ops.py:3956-3961``,
  ``:4142-4160``, ``:4085-4139``);
* the plain pre-norm baseline (``use_attnres=False``).

Each case stores the model's state dict (parameters and rotary tables), the
token ids and targets, the final hidden state, the LM cross-entropy loss and
the gradient of every parameter.  These pin the decoder's schedule (block
ends, logit caching, count prior, summary scaling, read norms) to the
reference model itself; no reference source is copied.
"""

from __future__ import annotations

import argparse
import json
import os
import sys

import torch
from safetensors.torch import save_file
from torch.nn import functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

SMALL = dict(n_layer=3, n_head=2, n_embd=24, mlp_hidden_dim=32, vocab_size=37, block_size=12)

CASES = [
    # name, seed, dtype, batch, extra config
    ("model_lrid_fp32", 501, "fp32", 2,
     dict(use_attnres=True, use_lrid=True, use_fused_attnres=True, attnres_num_blocks=2, lrid_rank=8,
          norm_pos="before", attn_res_query_init="normal")),
    ("model_lrid_bf16", 502, "bf16", 2,
     dict(use_attnres=True, use_lrid=True, use_fused_attnres=True, attnres_num_blocks=2, lrid_rank=8,
          norm_pos="before", attn_res_query_init="normal")),
    ("model_lrid_fp32_variant", 503, "fp32", 2,
     dict(use_attnres=True, use_lrid=True, use_fused_attnres=True, attnres_num_blocks=3, lrid_rank=8,
          norm_pos="after", attnres_key_norm=False, attnres_training_torch_phase2=False,
          attnres_block_average_mode="sqrt", attnres_block_count_prior=False, attn_res_query_init="normal")),
    ("model_lrid_bf16_blocks3", 504, "bf16", 1,
     dict(use_attnres=True, use_lrid=True, use_fused_attnres=True, attnres_num_blocks=3, lrid_rank=8,
          norm_pos="before", attn_res_query_init="normal")),
    ("model_baseline_fp32", 505, "fp32", 2, dict(use_attnres=False, norm_pos="before")),
]

DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def run_case(model_mod, name, seed, dtype, batch, extra):
    cfg = dict(SMALL)
    cfg.update(extra)
    torch.manual_seed(seed)
    model = model_mod.OBPM(model_mod.ModelConfig(**cfg)).train()
    if dtype != "fp32":
        model.to(dtype=DT[dtype])
    if cfg.get("use_lrid"):
        assert model._use_block_lrid_attnres_fused_training_path(None, False)
    gen = torch.Generator().manual_seed(seed + 1000)
    idx = torch.randint(0, cfg["vocab_size"], (batch, cfg["block_size"]), generator=gen)
    targets = torch.randint(0, cfg["vocab_size"], (batch, cfg["block_size"]), generator=gen)
    hidden = model(idx, return_hidden=True)
    logits = model.lm_head(hidden)
    loss = F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.view(-1))
    loss.backward()
    tensors = {f"state.{k}": v.detach().clone() for k, v in model.state_dict().items()}
    tensors.update({"idx": idx, "targets": targets, "hidden": hidden.detach(), "loss": loss.detach().reshape(1)})
    for pname, p in model.named_parameters():
        if p.grad is not None:
            tensors[f"grad.{pname}"] = p.grad.detach().clone()
    meta = dict(kind="model", dtype=dtype, batch=batch, seed=seed, config=cfg, torch=torch.__version__)
    return tensors, meta


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import model as model_mod  # the reference's model.py; its phase functions run their eager CPU branches

    index = {}
    for name, seed, dtype, batch, extra in CASES:
        tensors, meta = run_case(model_mod, name, seed, dtype, batch, extra)
        save_file({k: t.contiguous() for k, t in tensors.items()}, os.path.join(HERE, f"{name}.safetensors"))
        index[name] = meta
    with open(os.path.join(HERE, "model_index.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)
    print(f"wrote {len(index)} whole-model cases to {HERE}")


if __name__ == "__main__":
    main()
