"""Whole-model benchmark: block LR-AttnRes decoder vs the plain pre-norm decoder (reference: bench_attnres.py).

Times one training step (or forward) of the decoder in ``attnres_decoder``
with its AttnRes reads on the HIP kernels, beside the same decoder with a
plain residual stream, and reports what the reference's script reports
(``bench_attnres.py:150-318``): latency per step and the overhead of AttnRes
over the baseline, plus end-to-end tokens/s and the share of the step spent
in this library's kernels (from ``torch.profiler``'s device-time totals).

Defaults are the whole-model configuration: 12 layers, d=768, 12 heads,
MLP 4d, vocab 100277, block LR-AttnRes with rank 64 over 6 blocks (7 sources
at the last read), B=16, T=1024, bf16 weights and activations (the model is
cast with ``.to(bf16)``, as ``bench_attnres.py:180-181`` does), SDPA token
attention, LM cross-entropy loss and an SGD update, random init and uniform
random token ids.  Eager by default (no ``torch.compile``); ``--graph true``
replays everything after the embedding lookup from HIP graphs, the
counterpart of the reference's CUDA-graph runs (``FUSED_ATTNRES.md:317-345``).

    python lr-attnres_amd/bench_attnres.py [--batch_sizes 16] [--phase train] [--loss lm] ...

Output: a header line, one CSV row per case and one JSON summary line.
"""

from __future__ import annotations

import argparse
import faulthandler
import gc
import json
import os
import sys

import torch
from torch.nn import functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import attnres_decoder as AD  # noqa: E402

# Every kernel of libattnres_hip.so lives in the C++ namespace ``attnres``.
ATTNRES_KERNEL_PREFIX = "attnres::"


def _bool(value):
    if isinstance(value, bool):
        return value
    v = value.lower()
    if v in {"true", "1", "yes", "y", "on"}:
        return True
    if v in {"false", "0", "no", "n", "off"}:
        return False
    raise argparse.ArgumentTypeError("expected a boolean value")


def parse_args(argv=None):
    p = argparse.ArgumentParser(description="Benchmark the block LR-AttnRes decoder on the HIP read kernels.")
    p.add_argument("--n_layer", type=int, default=12)
    p.add_argument("--n_head", type=int, default=12)
    p.add_argument("--n_embd", type=int, default=768)
    p.add_argument("--mlp_hidden_dim", type=int, default=None)
    p.add_argument("--block_size", type=int, default=1024)
    p.add_argument("--vocab_size", type=int, default=100277)
    p.add_argument("--attnres_num_blocks", type=int, default=6)
    p.add_argument("--batch_sizes", type=str, default="16")
    p.add_argument("--lrid_ranks", type=str, default="64")
    p.add_argument("--lrid_projection_rank", type=int, default=None,
                   help="physical width of the key part of each fused projection (>= rank; the extra columns are "
                        "padding the read ignores), as the reference's flag (bench_attnres.py:37)")
    p.add_argument("--attnres_block_average", type=_bool, default=True)
    p.add_argument("--attnres_block_average_mode", choices=("count", "sqrt"), default="count")
    p.add_argument("--attnres_block_count_prior", type=_bool, default=True)
    p.add_argument("--attnres_key_norm", type=_bool, default=True)
    p.add_argument("--attnres_training_torch_phase2", type=_bool, default=True)
    p.add_argument("--attnres_fuse_read_norm", type=_bool, default=True)
    p.add_argument("--fold_block_summary", type=_bool, default=True)
    p.add_argument("--fuse_block_accumulation", type=_bool, default=True)
    p.add_argument("--fuse_accumulate_read", type=_bool, default=True,
                   help="sublayers that do not end a block also form the next read")
    p.add_argument("--dtype", choices=("fp32", "bf16", "fp16"), default="bf16")
    p.add_argument("--phase", choices=("forward", "train"), default="train")
    p.add_argument("--loss", choices=("hidden_mse", "lm"), default="lm")
    p.add_argument("--optimizer_step", type=_bool, default=True)
    p.add_argument("--lr", type=float, default=1e-4)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--iters", type=int, default=10)
    p.add_argument("--cases", type=str, default="baseline,lrid_fused",
                   help="comma-separated: baseline (plain pre-norm), lrid_fused (block LR-AttnRes on HIP)")
    p.add_argument("--nonzero_attnres_queries", type=_bool, default=True)
    p.add_argument("--profile_iters", type=int, default=2,
                   help="extra steps under torch.profiler for the kernel share (0 = skip)")
    p.add_argument("--graph", type=_bool, default=False,
                   help="train steps with everything after the embedding lookup replayed from HIP graphs "
                        "(torch.cuda.make_graphed_callables); the lookup, its backward and the update stay eager")
    p.add_argument("--tunable_gemm", type=_bool, default=False,
                   help="let PyTorch's TunableOp pick the library GEMM kernels by timing them (both cases; the "
                        "tuning runs in the warmup steps, results kept in a file under $TMPDIR)")
    p.add_argument("--seed", type=int, default=1234)
    return p.parse_args(argv)


def resolve_dtype(name):
    return {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[name]


def make_config(args, use_attnres, rank):
    return AD.DecoderConfig(
        n_layer=args.n_layer, n_head=args.n_head, n_embd=args.n_embd, mlp_hidden_dim=args.mlp_hidden_dim,
        vocab_size=args.vocab_size, block_size=args.block_size, norm_pos="before", use_attnres=use_attnres,
        attnres_num_blocks=args.attnres_num_blocks, attnres_block_average=args.attnres_block_average,
        attnres_block_average_mode=args.attnres_block_average_mode,
        attnres_block_count_prior=args.attnres_block_count_prior, attnres_key_norm=args.attnres_key_norm,
        attnres_training_torch_phase2=args.attnres_training_torch_phase2,
        attnres_fuse_read_norm=args.attnres_fuse_read_norm, lrid_rank=rank or 64,
        lrid_projection_rank=args.lrid_projection_rank if use_attnres else None, lrid_num_heads=1,
        lrid_use_logit_scale=True, fold_block_summary=args.fold_block_summary,
        fuse_block_accumulation=args.fuse_block_accumulation, fuse_accumulate_read=args.fuse_accumulate_read)


def training_loss(args, model, idx, targets):
    if args.loss == "hidden_mse":
        return model(idx, return_hidden=True).float().square().mean()
    logits = model(idx)
    return F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.view(-1))


def train_step(args, model, idx, targets):
    for p in model.parameters():
        p.grad = None
    loss = training_loss(args, model, idx, targets)
    loss.backward()
    if args.optimizer_step:
        with torch.no_grad():
            for p in model.parameters():
                if p.grad is not None:
                    p.add_(p.grad, alpha=-args.lr)
    return loss


class _Body(torch.nn.Module):
    """The decoder between its embedding lookup and its head: ``x -> hidden``.

    The lookup's backward (a scatter whose sort / unique step has data-dependent
    sizes) cannot be replayed from a graph captured at other token ids, so a
    graphed step keeps the lookup eager; the head and the loss stay eager too
    (a few launches), which keeps large single-tensor reductions -- whose
    multi-workgroup form clears its counters with a memset node -- out of the
    graph."""

    def __init__(self, model):
        super().__init__()
        self.model = model

    def forward(self, x):
        m = self.model
        return m._forward_block_lrid(x) if m.config.use_attnres else m._forward_baseline(x)


def _loss_from_hidden(args, model, h, targets):
    if args.loss == "hidden_mse":
        return h.float().square().mean()
    logits = F.linear(h, model.transformer.wte.weight, None) if model.config.weight_tying else model.lm_head(h)
    return F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.view(-1))


def graphed_train_step(args, model, idx, targets):
    """A train step whose decoder body (everything between the embedding
    lookup and the head, forward and backward) replays HIP graphs; returns
    (step, check) where check(n) runs n graphed and n eager steps from the same
    weights and returns the largest relative difference of their losses (graph
    replays must match eager execution before their timing means anything)."""
    x0 = model.transformer.wte(idx).detach().requires_grad_(True)
    graphed = torch.cuda.make_graphed_callables(_Body(model), (x0,), allow_unused_input=True)
    params = [p for p in model.parameters()]

    def step():
        for p in params:
            p.grad = None
        h = graphed(model.transformer.wte(idx))
        loss = _loss_from_hidden(args, model, h, targets)
        loss.backward()
        if args.optimizer_step:
            with torch.no_grad():
                live = [p for p in params if p.grad is not None]
                torch._foreach_add_(live, [p.grad for p in live], alpha=-args.lr)
        return loss

    def check(n):
        start = [p.detach().clone() for p in params]
        losses = []
        for fn in (step, lambda: train_step(args, model, idx, targets)):
            with torch.no_grad():
                for p, s0 in zip(params, start):
                    p.copy_(s0)
            torch.cuda.synchronize()
            losses.append([float(fn().detach()) for _ in range(n)])
        with torch.no_grad():
            for p, s0 in zip(params, start):
                p.copy_(s0)
        return max(abs(a - b) / max(abs(b), 1e-6) for a, b in zip(*losses)), losses

    return step, check


def _device_time_us(event):
    for attr in ("self_device_time_total", "self_cuda_time_total"):
        if hasattr(event, attr):
            return float(getattr(event, attr))
    return 0.0


# Device-time categories of the step's kernels (first match wins), so that the
# AttnRes model's extra device time can be attributed beyond this library's
# own kernels: the GEMMs of the wider fused projections, the eager glue that
# builds logits and queries, etc.
KERNEL_CATEGORIES = (
    ("attnres", ("attnres::",)),
    ("gemm", ("cijk_", "gemm", "hipblaslt", "matmul", "wvsplitk", "mfma")),
    ("attention", ("attn", "fmha", "flash", "sdpa", "aotriton")),
    ("embedding_index", ("embedding", "index", "gather", "scatter", "partition", "radix", "sort", "unique",
                         "segment")),
    ("norm", ("norm",)),
    ("loss", ("softmax", "nll", "cross_entropy", "log_softmax")),
    ("reduce", ("reduce",)),
    ("elementwise", ("elementwise", "vectorized", "copy", "fill", "cat", "where", "pointwise")),
)


def kernel_category(name):
    n = name.lower()
    for cat, keys in KERNEL_CATEGORIES:
        if any(k in n for k in keys):
            return cat
    return "other"


def kernel_share(step, iters):
    """(attnres kernel µs per step, all kernels µs per step, µs per step by
    KERNEL_CATEGORIES, kernel launches per step by category) from
    torch.profiler, or Nones."""
    try:
        from torch.profiler import ProfilerActivity, profile
    except ImportError:
        return None, None, None, None
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(iters):
            step()
        torch.cuda.synchronize()
    total = attn = 0.0
    cats, counts = {}, {}
    for ev in prof.key_averages():
        t = _device_time_us(ev)
        if t == 0.0:
            continue
        total += t
        if ATTNRES_KERNEL_PREFIX in ev.key:
            attn += t
        c = kernel_category(ev.key)
        cats[c] = cats.get(c, 0.0) + t
        counts[c] = counts.get(c, 0) + ev.count
    if total == 0.0:
        return None, None, None, None
    return (attn / iters, total / iters, {k: v / iters for k, v in sorted(cats.items())},
            {k: v / iters for k, v in sorted(counts.items())})


def measure_case(args, device, dtype, batch, label, use_attnres, rank=None):
    torch.manual_seed(args.seed)
    cfg = make_config(args, use_attnres, rank)
    with torch.device(device):
        model = AD.Decoder(cfg)
    if args.nonzero_attnres_queries and use_attnres:
        with torch.no_grad():
            for q in model.transformer.lrid_queries:
                q.normal_(0.0, cfg.init_std)
    model.to(dtype=dtype)
    model.train(args.phase == "train")
    gen = torch.Generator(device=device).manual_seed(args.seed + 1)
    idx = torch.randint(0, args.vocab_size, (batch, args.block_size), device=device, generator=gen)
    targets = torch.randint(0, args.vocab_size, (batch, args.block_size), device=device, generator=gen)

    graph_check = None
    if args.tunable_gemm and args.phase == "train":
        # one eager step first: it meets every GEMM shape, so the tuning happens
        # here rather than inside the graph warmup
        train_step(args, model, idx, targets)
        torch.cuda.synchronize()
        print(f"# {label}: GEMM tuning step done", flush=True)
    if args.phase == "forward":
        def step():
            with torch.inference_mode():
                model(idx, return_hidden=True)
    elif args.graph:
        step, check = graphed_train_step(args, model, idx, targets)
        rel, losses = check(6)
        graph_check = {"max_rel_loss_diff": rel, "graph_losses": losses[0], "eager_losses": losses[1]}
        if rel > 1e-2:
            raise RuntimeError(f"graph replays do not match eager steps: {graph_check}")
    else:
        def step():
            train_step(args, model, idx, targets)

    try:
        for i in range(args.warmup):
            step()
            if args.tunable_gemm:  # GEMM tuning makes the first steps long: say where the run is
                torch.cuda.synchronize()
                print(f"# {label}: warmup step {i + 1}/{args.warmup} done", flush=True)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.iters):
            step()
        end.record()
        torch.cuda.synchronize()
        latency_ms = start.elapsed_time(end) / args.iters
        attn_us = total_us = cats_us = counts = None
        if args.profile_iters > 0:
            attn_us, total_us, cats_us, counts = kernel_share(step, args.profile_iters)
        n_params = model.get_num_params()
    finally:
        del model, idx, targets
        gc.collect()
        torch.cuda.empty_cache()
    return {
        "label": label,
        "batch": batch,
        "rank": rank or "",
        "projection_rank": cfg.lrid_projection_rank if use_attnres else "",
        "latency_ms": latency_ms,
        "tokens_per_s": batch * args.block_size / (latency_ms * 1e-3),
        "attnres_kernel_ms": None if attn_us is None else attn_us / 1000.0,
        "device_kernel_ms": None if total_us is None else total_us / 1000.0,
        "device_ms_by_category": None if cats_us is None else {k: v / 1000.0 for k, v in cats_us.items()},
        "kernels_by_category": counts,
        "params": n_params,
        "graph": bool(args.graph and args.phase == "train"),
        "graph_check": graph_check,
    }


def _fmt(x, spec):
    return "" if x is None else format(x, spec)


def main(argv=None):
    args = parse_args(argv)
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required for this benchmark")
    device = torch.device("cuda")
    if args.tunable_gemm:
        # TunableOp times the candidate GEMM solutions of each new shape once
        # and keeps the fastest: the fused [out | key] projections are d + r
        # wide (1056 at d1024 r32), a width the default choice fits badly
        import tempfile

        torch.cuda.tunable.set_filename(os.path.join(tempfile.gettempdir(), "attnres_tunableop.csv"))
        torch.cuda.tunable.set_max_tuning_duration(10)
        torch.cuda.tunable.set_max_tuning_iterations(20)
        torch.cuda.tunable.tuning_enable(True)
        torch.cuda.tunable.enable(True)
    dtype = resolve_dtype(args.dtype)
    batches = [int(x) for x in args.batch_sizes.split(",") if x.strip()]
    ranks = [int(x) for x in args.lrid_ranks.split(",") if x.strip()]
    cases = {x.strip() for x in args.cases.split(",") if x.strip()}
    unknown = cases - {"baseline", "lrid_fused"}
    if unknown:
        raise SystemExit(f"unknown cases: {sorted(unknown)}")

    print(f"dtype={args.dtype} phase={args.phase} loss={args.loss} optimizer_step={args.optimizer_step} "
          f"n_layer={args.n_layer} n_embd={args.n_embd} n_head={args.n_head} vocab={args.vocab_size} "
          f"T={args.block_size} blocks={args.attnres_num_blocks} fold_block_summary={args.fold_block_summary} "
          f"graph={args.graph} tunable_gemm={args.tunable_gemm} "
          f"torch={torch.__version__} device={torch.cuda.get_device_name(0)}", flush=True)
    print("case,batch,rank,latency_ms,overhead_vs_baseline_pct,tokens_per_s,attnres_kernel_ms,"
          "attnres_kernel_share_pct", flush=True)
    summary = []
    for batch in batches:
        rows = []
        base = None
        if "baseline" in cases:
            base = measure_case(args, device, dtype, batch, "baseline_prenorm", False)
            rows.append(base)
        if "lrid_fused" in cases:
            for rank in ranks:
                rows.append(measure_case(args, device, dtype, batch, "lrid_fused", True, rank))
        for row in rows:
            row["overhead_vs_baseline_pct"] = (None if base is None else
                                               100.0 * (row["latency_ms"] / base["latency_ms"] - 1.0))
            row["attnres_kernel_share_pct"] = (None if row["attnres_kernel_ms"] is None else
                                               100.0 * row["attnres_kernel_ms"] / row["latency_ms"])
            # where the extra device time goes, by kernel category (ms per step)
            bc = None if base is None else base.get("device_ms_by_category")
            rc = row.get("device_ms_by_category")
            row["device_ms_delta_by_category"] = (None if bc is None or rc is None else
                                                  {k: rc.get(k, 0.0) - bc.get(k, 0.0)
                                                   for k in sorted(set(bc) | set(rc))})
            # and the extra kernel launches (each costs a graph node's dispatch too)
            bn = None if base is None else base.get("kernels_by_category")
            rn = row.get("kernels_by_category")
            row["kernels_delta_by_category"] = (None if bn is None or rn is None else
                                                {k: rn.get(k, 0) - bn.get(k, 0) for k in sorted(set(bn) | set(rn))})
            print(f"{row['label']},{row['batch']},{row['rank']},{row['latency_ms']:.3f},"
                  f"{_fmt(row['overhead_vs_baseline_pct'], '.2f')},{row['tokens_per_s']:.0f},"
                  f"{_fmt(row['attnres_kernel_ms'], '.3f')},{_fmt(row['attnres_kernel_share_pct'], '.2f')}",
                  flush=True)
        summary.extend(rows)
    print(json.dumps({
        "metric": "whole-model step tokens/s; AttnRes share of step time",
        "workload": "c5" if (args.n_layer, args.n_embd, args.n_head, args.vocab_size, args.block_size,
                             args.attnres_num_blocks) == (12, 768, 12, 100277, 1024, 6) else "custom",
        "phase": args.phase, "loss": args.loss, "optimizer_step": args.optimizer_step, "dtype": args.dtype,
        "graph": bool(args.graph and args.phase == "train"),
        "tunable_gemm": bool(args.tunable_gemm),
        "data": "synthetic (uniform random token ids, random init)",
        "cases": summary,
    }), flush=True)
    return summary


if __name__ == "__main__":
    faulthandler.enable()  # a crash in native code prints the Python stack that led to it
    main()
