#!/usr/bin/env python3
"""Benchmark of the fused AttnRes read (forward + backward) on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config c3]

A "step" is one forward + one backward of the read over one batch of synthetic
input already resident in HBM, launched through the library's C ABI (the
drop-in boundary) on the current stream.  The default workload is BASELINE
config 3 (LR read, B8 T2048 d1024 N13 r64 H4, bf16), the configuration the
metric is quoted on.  Prints ONE JSON line.

Besides the contract fields the line carries:
  roofline      HBM roofline of the dominant kernel (the backward), from its
                average launch duration: HIP events that the library records
                on the launch stream around that kernel alone
  kernels       average durations and algorithmic GB/s of the fwd and bwd
                main kernels, and of the whole C calls (``*_call_ms``: the
                backward call adds the partial-sum reduction)
  api           ms/step through the Python autograd API (custom op + ctypes)
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "lr-attnres_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E peak

CONFIGS = {
    "c1": dict(kind="base", B=2, T=128, D=128, N=4, R=0, H=1, scale=1.0, dtype=torch.float32, qstd=0.02,
               fwd_only=True),
    # C2's sources as the configuration defines them (the embedding and 6 block
    # summaries of two sublayer outputs, count**-1); two input sets alternate
    # step by step, so that the ~200 MB one step touches is not served from the
    # previous step's copy in the 256 MB MALL
    "c2": dict(kind="base", B=8, T=1024, D=768, N=7, R=0, H=1, scale=1.0, dtype=torch.bfloat16, qstd=0.02,
               block_summaries=True, sets=2),
    "c3": dict(kind="lr", B=8, T=2048, D=1024, N=13, R=64, H=4, scale=0.25, dtype=torch.bfloat16, qstd=0.02),
    # C4 by its full definition: keys rms_norm(v_s) @ W_k (W_k ~ N(0, 0.02); produced
    # outside the timed step, as the model projects them once per source) plus a
    # static source key [N, 128] ~ N(0, 0.02) added inside the read
    "c4": dict(kind="lr_gated", B=4, T=4096, D=2048, N=17, R=128, H=8, scale=0.25, dtype=torch.bfloat16,
               qstd=0.02, value_keys=True, static_keys=True),
}


# cached-logit block schedule at the reference model's shape (12 layers, d768,
# 6 blocks: up to 6 completed sources read by the 4 sites of the next block);
# a step is phase 1 once + phase 2 at each of the Q sites, forward and backward
PHASE_CONFIGS = {
    "p5": dict(B=16, T=1024, D=768, S=6, Q=4, R=64, dtype=torch.bfloat16),
    # the block LR decoder's form (C5): phase 2 with the partial block's LR key
    # (r=64, key norm, logit scale 1/8), the lerp merge and the next sublayer's
    # fused pre-norm
    "p5lr": dict(B=16, T=1024, D=768, S=6, Q=4, R=64, dtype=torch.bfloat16, lr=True),
    # p5lr's block in the decoder's accumulate-and-read schedule (see p12ar)
    "p5ar": dict(B=16, T=1024, D=768, S=6, Q=4, R=64, dtype=torch.bfloat16, lr=True, fused_read=True),
    # the reference's published block (24 layers, d1024, 4 blocks: 12 read sites
    # over up to 4 completed sources, LR rank 32) on 16384 tokens
    "p12lr": dict(B=8, T=2048, D=1024, S=4, Q=12, R=32, dtype=torch.bfloat16, lr=True),
    # the same block in the block LR decoder's schedule: the Q - 1 sublayers that
    # do not end the block grow it and form the next site's merge in one pass
    # (attnres_accum_read_*), the last completes it (attnres_block_accum_*)
    "p12ar": dict(B=8, T=2048, D=1024, S=4, Q=12, R=32, dtype=torch.bfloat16, lr=True, fused_read=True),
}


def phase_bytes_per_token(c):
    """Algorithmic HBM bytes per token of each phase kernel (fp32 logits, lse)."""
    s = torch.finfo(c["dtype"]).bits // 8
    S, Q, D = c["S"], c["Q"], c["D"]
    p1f = S * D * s + Q * S * 4 + Q * D * s + Q * 4
    p1b = Q * D * s + Q * 4 + S * D * s + Q * S * 4 + S * D * s + Q * S * 4
    p2f = 2 * D * s + 4 + D * s
    p2b = 3 * D * s + 4 + 2 * D * s + 4
    if c.get("lr"):  # the partial key read (and its gradient written)
        p2f += c["R"] * s
        p2b += 2 * c["R"] * s
    # block accumulation, averaged over the Q sublayers of a block (the first has no
    # partial block to read): fwd reads y[:, :D+R] (+ partial value and key) and writes
    # value, key and the key's 1/rms; bwd reads both gradients, the raw key and 1/rms
    # and writes the projection's gradient
    R = c["R"]
    acf = (D + R) * s + (Q - 1) / Q * (D + R) * s + (D + R) * s + 4
    acb = (D + R) * s + R * s + 4 + (D + R) * s
    if c.get("fused_read"):
        # Q - 1 accumulate-and-read calls (the first without an old partial block)
        # and one completing accumulation.  Forward: y, the old block, inter and
        # lse read; the grown block, the key's 1/rms and the read written.
        # Backward: the read's gradient, the grown block, inter, lse, the block's
        # other gradients, the raw key and 1/rms read; d inter, d lse, the
        # projection's gradient and the old key's gradient written.
        old = (Q - 2) / (Q - 1)
        arf = (D + R) * s + old * (D + R) * s + D * s + 4 + (D + R) * s + 4 + D * s
        arb = (D * s + (D + R) * s + D * s + 4 + (D + R) * s + R * s + 4
               + D * s + 4 + (D + R) * s + old * R * s)
        acf = 3 * (D + R) * s + 4
        return dict(phase1_fwd=p1f, phase1_bwd=p1b, ar_fwd=arf, ar_bwd=arb, accum_fwd=acf, accum_bwd=acb)
    return dict(phase1_fwd=p1f, phase1_bwd=p1b, phase2_fwd=p2f, phase2_bwd=p2b, accum_fwd=acf, accum_bwd=acb)


class PhaseWorkload:
    """Phase-1 + phase-2 (base keys, key_norm, count bias, block-summary scale)
    descriptors over resident synthetic inputs, launched through the C ABI."""

    def __init__(self, c, device, seed=0):
        import _attnres_hip as H

        self.H = H
        lib = H.load()
        self.lib = lib
        g = torch.Generator(device=device).manual_seed(seed)
        B, T, D, S, Q, dt = c["B"], c["T"], c["D"], c["S"], c["Q"], c["dtype"]
        n = B * T
        self.n_tok, self.Q = n, Q
        rn = lambda *shape, std=1.0, dtype=dt: (torch.randn(shape, generator=g, device=device) * std).to(dtype)
        self.values = [rn(n, D) for _ in range(S)]
        self.logits = rn(Q, S, n, std=2.0, dtype=torch.float32)
        self.p1 = H.Phase1(self.values, self.logits, False)
        self.out = torch.empty((Q, n, D), device=device, dtype=dt)
        self.lse = torch.empty((Q, n), device=device, dtype=torch.float32)
        self.gout = rn(Q, n, D)
        self.glse = rn(Q, n, dtype=torch.float32)
        self.dvals = [torch.empty((n, D), device=device, dtype=dt) for _ in range(S)]
        self._dv = (ctypes.c_void_p * S)(*[t.data_ptr() for t in self.dvals])
        self.dlog = torch.empty((Q, S, n), device=device, dtype=torch.float32)
        self.partial = rn(n, D)
        self.lr = bool(c.get("lr"))
        if self.lr:
            R = c["R"]
            self.pkey = rn(n, R)
            self.query = rn(R, std=0.02)
            self.dpk = torch.empty((n, R), device=device, dtype=dt)
            self.p2 = [H.Phase2(self.partial, self.pkey, self.query, None, self.out[q], self.lse[q], H.MERGE_LERP,
                                True, True, 1.0 / math.sqrt(R), 0.693, None, 0.5, None, False) for q in range(Q)]
        else:
            self.query = rn(D, std=0.02)
            self.p2 = [H.Phase2(self.partial, None, self.query, None, self.out[q], self.lse[q], H.MERGE_ADDCMUL,
                                True, False, 1.0, 0.693, None, 0.5, None, False) for q in range(Q)]
        self.out2 = torch.empty((n, D), device=device, dtype=dt)
        self.g2 = rn(n, D)
        self.dp = torch.empty((n, D), device=device, dtype=dt)
        self.di = torch.empty((n, D), device=device, dtype=dt)
        self.dl = torch.empty((n,), device=device, dtype=torch.float32)
        self.dq = torch.empty_like(self.query)
        ws = lib.attnres_phase2_backward_workspace_size(ctypes.byref(self.p2[0].c))
        self.ws = torch.empty((max(1, ws),), device=device, dtype=torch.uint8)
        gr = H.Phase2Grads()
        gr.grad_out = self.g2.data_ptr()
        gr.dpartial_value = self.dp.data_ptr()
        gr.dquery = self.dq.data_ptr()
        gr.dinterblock_output = self.di.data_ptr()
        if self.lr:
            gr.dpartial_key = self.dpk.data_ptr()
        gr.dinterblock_lse = ctypes.cast(ctypes.c_void_p(self.dl.data_ptr()), ctypes.POINTER(ctypes.c_float))
        gr.workspace = self.ws.data_ptr()
        gr.workspace_bytes = ws
        self.gr = gr
        self.f = lambda t: ctypes.cast(ctypes.c_void_p(t.data_ptr()), ctypes.POINTER(ctypes.c_float))
        # the block's Q sublayers grow the partial block from their fused projections
        # [n, D + R]; the last completes it (scale 1/Q)
        R = c["R"]
        self.D, self.R = D, R
        self.ys = [rn(n, D + R) for _ in range(Q)]
        self.avals = [torch.empty((n, D), device=device, dtype=dt) for _ in range(Q)]
        self.akeys = [torch.empty((n, R), device=device, dtype=dt) for _ in range(Q)]
        self.ainv = [torch.empty((n, 1), device=device, dtype=torch.float32) for _ in range(Q)]
        self.agv = [rn(n, D) for _ in range(Q)]
        self.agk = [rn(n, R) for _ in range(Q)]
        self.agy = [torch.empty((n, D + R), device=device, dtype=dt) for _ in range(Q)]
        self.adesc = [H.block_accum_desc(self.ys[q], D, R, 1, True, self.avals[q - 1] if q else None,
                                         self.akeys[q - 1] if q else None, q == Q - 1, False, False, 1.0 / Q, None)
                      for q in range(Q)]
        self.fused_read = bool(c.get("fused_read"))
        if self.fused_read:
            # sublayer q < Q - 1 grows the block into avals[q] / akeys[q] and site
            # q + 1's merge (phase-1 read out[q]) reads it
            self.ar = []
            for q in range(Q - 1):
                acc = H.block_accum_desc(self.ys[q], D, R, 1, True, self.avals[q - 1] if q else None,
                                         self.akeys[q - 1] if q else None, False, False, False, 1.0, None)
                read = H.Phase2(self.avals[q], self.akeys[q], self.query, None, self.out[q], self.lse[q],
                                H.MERGE_LERP, True, True, 1.0 / math.sqrt(R), 0.693, None, 0.5, None, False)
                self.ar.append((H.accum_read_desc(acc, read), read))
            self.adpk = torch.empty((n, R), device=device, dtype=dt)
            gq = H.Phase2Grads()
            for f in ("grad_out", "dquery", "dinterblock_output", "dinterblock_lse", "workspace", "workspace_bytes"):
                setattr(gq, f, getattr(gr, f))
            self.gq = gq

    def _ok(self, rc):
        if rc:
            raise RuntimeError(self.lib.attnres_last_error().decode())

    def phase1_fwd(self, sv):
        self._ok(self.lib.attnres_phase1_forward(ctypes.byref(self.p1.c), ctypes.c_void_p(self.out.data_ptr()),
                                                 None, self.f(self.lse), None, sv))

    def phase1_bwd(self, sv):
        self._ok(self.lib.attnres_phase1_backward(ctypes.byref(self.p1.c), ctypes.c_void_p(self.gout.data_ptr()),
                                                  self.f(self.glse), None, None, self._dv,
                                                  ctypes.c_void_p(self.dlog.data_ptr()), sv))

    def phase2_fwd(self, sv):
        for d in self.p2:
            self._ok(self.lib.attnres_phase2_forward(ctypes.byref(d.c), ctypes.c_void_p(self.out2.data_ptr()), sv))

    def phase2_bwd(self, sv):
        for d in self.p2:
            self._ok(self.lib.attnres_phase2_backward(ctypes.byref(d.c), ctypes.byref(self.gr), sv))

    def ar_fwd(self, sv):
        for q, (d, _) in enumerate(self.ar):
            self._ok(self.lib.attnres_accum_read_forward(ctypes.byref(d), ctypes.c_void_p(self.avals[q].data_ptr()),
                                                         ctypes.c_void_p(self.akeys[q].data_ptr()),
                                                         self.f(self.ainv[q]), ctypes.c_void_p(self.out2.data_ptr()),
                                                         sv))

    def ar_bwd(self, sv):
        for q in reversed(range(len(self.ar))):
            self._ok(self.lib.attnres_accum_read_backward(
                ctypes.byref(self.ar[q][0]), ctypes.byref(self.gq), ctypes.c_void_p(self.agv[q].data_ptr()), self.D,
                ctypes.c_void_p(self.agk[q].data_ptr()), self.f(self.ainv[q]), ctypes.c_void_p(self.agy[q].data_ptr()),
                ctypes.c_void_p(self.adpk.data_ptr()) if q else None, sv))

    def accum_fwd(self, sv):
        if self.fused_read:  # only the completing accumulation is separate
            d, q = self.adesc[-1], len(self.adesc) - 1
            self._ok(self.lib.attnres_block_accum_forward(ctypes.byref(d), ctypes.c_void_p(self.avals[q].data_ptr()),
                                                          ctypes.c_void_p(self.akeys[q].data_ptr()),
                                                          self.f(self.ainv[q]), None, sv))
            return
        for q, d in enumerate(self.adesc):
            self._ok(self.lib.attnres_block_accum_forward(ctypes.byref(d), ctypes.c_void_p(self.avals[q].data_ptr()),
                                                          ctypes.c_void_p(self.akeys[q].data_ptr()),
                                                          self.f(self.ainv[q]), None, sv))

    def accum_bwd(self, sv):
        qs = [len(self.adesc) - 1] if self.fused_read else reversed(range(len(self.adesc)))
        for q in qs:
            self._ok(self.lib.attnres_block_accum_backward(
                ctypes.byref(self.adesc[q]), ctypes.c_void_p(self.agv[q].data_ptr()), self.D,
                ctypes.c_void_p(self.agk[q].data_ptr()), self.f(self.ainv[q]), None,
                ctypes.c_void_p(self.agy[q].data_ptr()), None, None, None, 0, sv))


def bench_phase(args, dev):
    c = PHASE_CONFIGS[args.config]
    wl = PhaseWorkload(c, dev)
    stream = torch.cuda.current_stream(dev)
    sv = ctypes.c_void_p(stream.cuda_stream)
    if c.get("fused_read"):
        parts = ("phase1_fwd", "phase1_bwd", "ar_fwd", "ar_bwd", "accum_fwd", "accum_bwd")
    else:
        parts = ("phase1_fwd", "phase1_bwd", "phase2_fwd", "phase2_bwd", "accum_fwd", "accum_bwd")
    for _ in range(args.warmup):
        for k in parts:
            getattr(wl, k)(sv)
    torch.cuda.synchronize()
    ev = {k: [] for k in parts}
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        for k in parts:
            getattr(wl, k)(sv)
    t1.record(stream)
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / args.steps
    for _ in range(args.steps):
        for k in parts:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            getattr(wl, k)(sv)
            b.record(stream)
            ev[k].append((a, b))
    torch.cuda.synchronize()
    bpt = phase_bytes_per_token(c)
    kern = {}
    for k in parts:
        # median over the steps: a pair that spans a gap in the host's
        # submission (the GPU idle between the two events) would skew a mean
        ms = statistics.median(a.elapsed_time(b) for a, b in ev[k])
        if c.get("fused_read"):
            calls = c["Q"] - 1 if k.startswith("ar_") else 1
        else:
            calls = c["Q"] if k.startswith(("phase2", "accum")) else 1
        gbs = bpt[k] * wl.n_tok * calls / (ms / 1e3) / 1e9
        kern[k] = {"ms": round(ms, 5), "calls": calls, "gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                   "bytes_per_token": bpt[k]}
    if c.get("fused_read"):
        workload = (f"{args.config}: phase1 S{c['S']} Q{c['Q']} + {c['Q'] - 1} x accumulate-and-read (block "
                    f"accumulation r{c['R']} key_norm + LR merge: lerp, output norm) + 1 x completing block "
                    f"accumulation, B{c['B']} T{c['T']} d{c['D']}")
    else:
        workload = (f"{args.config}: phase1 S{c['S']} Q{c['Q']} + {c['Q']} x phase2 "
                    + (f"(LR key r{c['R']}, key_norm, lerp, output norm) " if c.get("lr") else "(base, key_norm) ")
                    + f"+ {c['Q']} x block accumulation (r{c['R']}, key_norm, the last completing "
                    f"the block) B{c['B']} T{c['T']} d{c['D']}")
    metric = ("cached-logit block schedule (phase 1 + Q-1 accumulate-and-read calls + 1 completing accumulation) "
              "fwd+bwd tokens/s" if c.get("fused_read") else
              "cached-logit block schedule (phase 1 + Q phase-2 merges + Q partial-block accumulations) fwd+bwd tokens/s")
    print(json.dumps({
        "metric": metric,
        "value": round(wl.n_tok / (step_ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 5), "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "tokens": wl.n_tok,
                   "phase_ms": round(sum(kern[k]["ms"] for k in parts if k.startswith("phase")), 5)},
        # the parts' device time (ms_per_step also holds the host's gaps between
        # the Python-driven C calls)
        "device_ms": round(sum(kern[k]["ms"] for k in parts), 5),
        "kernels": kern}))


def bytes_per_token(c):
    """Algorithmic HBM bytes per token (fwd, bwd): every tensor the op must
    touch, once.  s = element size; saved softmax weights are fp32."""
    s = torch.finfo(c["dtype"]).bits // 8
    N, D, R, H = c["N"], c["D"], c["R"], c["H"]
    w = N * H * 4
    fwd = N * D * s + N * R * s + D * s + (w if not c.get("fwd_only") else 0)
    bwd = D * s + N * D * s + N * R * s + w + N * D * s + N * R * s
    if c["kind"] == "lr_gated":
        fwd += R * s + H * s
        bwd += 2 * R * s + 2 * H * s
    if c.get("fwd_only"):
        bwd = 0
    return fwd, bwd


class Workload:
    """Inputs, outputs and C descriptors of one configuration, allocated once."""

    def __init__(self, c, device, seed=0):
        import _attnres_hip as H

        self.H = H
        self.c = c
        g = torch.Generator(device=device).manual_seed(seed)
        B, T, D, N, R, Hh, dt = c["B"], c["T"], c["D"], c["N"], c["R"], c["H"], c["dtype"]
        self.n_tok = B * T
        rn = lambda *shape, std=1.0: (torch.randn(shape, generator=g, device=device) * std).to(dt)
        if c.get("block_summaries"):
            # the embedding, then summaries (a + b) * count**-1 of two N(0, 1) outputs
            # in the dtype's arithmetic (model.py:990-1001)
            self.values = [rn(B, T, D)] + [(rn(B, T, D) + rn(B, T, D)) * 0.5 for _ in range(N - 1)]
        else:
            self.values = [rn(B, T, D) for _ in range(N)]
        if c.get("value_keys"):
            import attnres_ops as ops
            with torch.no_grad():
                self.keys = ops.lrid_value_key_projection(self.values, rn(R, D, std=0.02))
        else:
            self.keys = [rn(B, T, R) for _ in range(N)] if R else []
        self.static = rn(N, R, std=0.02) if c.get("static_keys") else None
        if c["kind"] == "base":
            self.query = rn(D, std=c["qstd"])
        else:
            self.query = rn(Hh, R // Hh, std=c["qstd"])
        self.query_dyn = rn(B, T, R) if c["kind"] == "lr_gated" else None
        self.gate = rn(B, T, Hh) if c["kind"] == "lr_gated" else None
        self.grad_out = rn(B, T, D)
        gate_act = H.GATE_SIGMOID if self.gate is not None else H.GATE_NONE
        self.desc = H.Desc(self.values, self.keys, self.query, self.query_dyn, self.gate, None, Hh, c["scale"], True,
                           False, H.MODE_SOFTMAX, gate_act, self.gate is not None, static_keys=self.static)
        self.out = torch.empty((self.n_tok, D), device=device, dtype=dt)
        self.weights = torch.empty((self.n_tok, Hh, N), device=device, dtype=torch.float32)
        self.dvals = [torch.empty((self.n_tok, D), device=device, dtype=dt) for _ in range(N)]
        self.dkeys = [torch.empty((self.n_tok, R), device=device, dtype=dt) for _ in range(N)] if R else []
        self.dq = torch.empty_like(self.query)
        self.dqd = torch.empty((self.n_tok, R), device=device, dtype=dt) if self.query_dyn is not None else None
        self.dg = torch.empty_like(self.gate) if self.gate is not None else None
        lib = H.load()
        self.lib = lib
        ws = lib.attnres_read_backward_workspace_size(ctypes.byref(self.desc.c))
        self.ws = torch.empty((max(1, ws),), device=device, dtype=torch.uint8)
        gr = H.ReadGrads()
        gr.grad_out = self.grad_out.data_ptr()
        gr.weights = ctypes.cast(ctypes.c_void_p(self.weights.data_ptr()), ctypes.POINTER(ctypes.c_float))
        self._dv = (ctypes.c_void_p * N)(*[t.data_ptr() for t in self.dvals])
        gr.dvalues = self._dv
        if R:
            self._dk = (ctypes.c_void_p * N)(*[t.data_ptr() for t in self.dkeys])
            gr.dkeys = self._dk
        gr.dquery = self.dq.data_ptr()
        gr.dquery_dyn = self.dqd.data_ptr() if self.dqd is not None else None
        gr.dgate = self.dg.data_ptr() if self.dg is not None else None
        gr.workspace = self.ws.data_ptr()
        gr.workspace_bytes = ws
        self.dstatic = torch.empty_like(self.static) if self.static is not None else None
        gr.dstatic_keys = self.dstatic.data_ptr() if self.dstatic is not None else None
        self.grads = gr
        self.wptr = ctypes.cast(ctypes.c_void_p(self.weights.data_ptr()), ctypes.POINTER(ctypes.c_float))
        self.outptr = ctypes.c_void_p(self.out.data_ptr())
        self.fwd_only = bool(c.get("fwd_only"))

    def fwd(self, stream):
        rc = self.lib.attnres_read_forward(ctypes.byref(self.desc.c), self.outptr, None,
                                          None if self.fwd_only else self.wptr, None, stream)
        if rc:
            raise RuntimeError(self.lib.attnres_last_error().decode())

    def bwd(self, stream):
        if self.fwd_only:
            return
        rc = self.lib.attnres_read_backward(ctypes.byref(self.desc.c), ctypes.byref(self.grads), stream)
        if rc:
            raise RuntimeError(self.lib.attnres_last_error().decode())


class Rotation:
    """Several input sets of one configuration used in turn, one per step
    (forward and backward of a step on the same set)."""

    def __init__(self, sets):
        self.sets = sets
        self.i = 0
        w = sets[0]
        self.c, self.lib, self.n_tok, self.fwd_only = w.c, w.lib, w.n_tok, w.fwd_only

    def __getattr__(self, name):  # inputs for the API timing: the first set's
        return getattr(self.__dict__["sets"][0], name)

    def fwd(self, stream):
        self.sets[self.i].fwd(stream)
        if self.fwd_only:
            self.i = (self.i + 1) % len(self.sets)

    def bwd(self, stream):
        if self.fwd_only:
            return
        self.sets[self.i].bwd(stream)
        self.i = (self.i + 1) % len(self.sets)


def make_workload(c, device):
    if c.get("sets", 1) > 1:
        return Rotation([Workload(c, device, seed=i) for i in range(c["sets"])])
    return Workload(c, device)


def time_steps(wl, steps, warmup, stream, sv):
    for _ in range(warmup):
        wl.fwd(sv)
        wl.bwd(sv)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        wl.fwd(sv)
        wl.bwd(sv)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_kernels(wl, steps, stream, sv):
    """Average duration of each C call, bracketed by events on its stream."""
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        ev[i][0].record(stream)
        wl.fwd(sv)
        ev[i][1].record(stream)
        ev[i][2].record(stream)
        wl.bwd(sv)
        ev[i][3].record(stream)
    torch.cuda.synchronize()
    f = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    b = sum(e[2].elapsed_time(e[3]) for e in ev) / steps
    return f, b


def time_main_kernels(wl, steps, sv):
    """Average duration of the forward's and the backward's main kernel alone
    (the backward's partial-sum reduction excluded): HIP events that the
    library records on the call's stream around that kernel."""
    lib = wl.lib
    steps = min(steps, 128)  # two event pairs per step, 256 pairs in the library
    if lib.attnres_kernel_timing(1):
        raise RuntimeError(lib.attnres_last_error().decode())
    try:
        torch.cuda.synchronize()
        for _ in range(steps):
            wl.fwd(sv)
            wl.bwd(sv)
        buf = (ctypes.c_float * (2 * steps))()
        n = lib.attnres_kernel_times(buf, 2 * steps)
        if n < 0:
            raise RuntimeError(lib.attnres_last_error().decode())
    finally:
        lib.attnres_kernel_timing(0)
    per = 1 if wl.fwd_only else 2
    if n != per * steps:
        raise RuntimeError(f"expected {per * steps} timed kernels, got {n}")
    f = sum(buf[i] for i in range(0, n, per)) / steps
    b = sum(buf[i] for i in range(1, n, per)) / steps if per == 2 else 0.0
    return f, b


def time_api(c, wl, steps, warmup):
    """ms/step through the public autograd API (drop-in module)."""
    import attnres_ops as ops

    vals = [v.detach().requires_grad_(True) for v in wl.values]
    keys = [k.detach().requires_grad_(True) for k in wl.keys]
    q = wl.query.detach().float().requires_grad_(True)

    def step():
        for t in vals + keys + [q]:
            t.grad = None
        if c["kind"] == "base":
            out = ops.attention_residual_read(vals, q, True)
        elif c["kind"] == "lr":
            out = ops.lrid_attention_residual_read(vals, keys, q, c["H"], c["scale"], True)
        else:
            out = ops.lrid_attention_residual_read_gated(vals, keys, q, wl.query_dyn, wl.gate, c["H"], c["scale"],
                                                         True, gate_activation="sigmoid")
        if not c.get("fwd_only"):
            out.backward(wl.grad_out)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(c, budget_s):
    """The eager restatement (oracle/) on the host cores, on a bounded token
    sample (B=1, T=2048) of the workload: fp32 and bf16, each the median of
    >= 5 timed iterations after 2 warmups (time.perf_counter), as tokens/s and
    effective GB/s from the same byte formula as the GPU line.  ``value`` is
    the workload dtype's median."""
    from oracle import attnres_oracle as O

    cores = len(os.sched_getaffinity(0))
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)
    D, N, R, Hh = c["D"], c["N"], c["R"], c["H"]
    T, B = 2048, 1
    by = {}
    for name, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        g = torch.Generator().manual_seed(1)
        mk = lambda *s, std=1.0: (torch.randn(s, generator=g) * std).to(dt).requires_grad_(True)  # noqa: E731
        vals = [mk(B, T, D) for _ in range(N)]
        keys = [mk(B, T, R) for _ in range(N)] if R else []
        up = torch.randn(B, T, D, generator=g).to(dt)
        q = mk(D, std=c["qstd"]) if c["kind"] == "base" else mk(Hh, R // Hh, std=c["qstd"])
        qd = mk(B, T, Hh, R // Hh) if c["kind"] == "lr_gated" else None
        gt = mk(B, T, Hh) if c["kind"] == "lr_gated" else None

        def step():
            if c["kind"] == "base":
                out = O.attention_residual_read_ref(vals, q, True)
            elif c["kind"] == "lr":
                out = O.lrid_attention_residual_read_ref(vals, keys, q, Hh, c["scale"], True)
            else:
                qq = O.gated_query_ref(q.float(), qd.float(), gt.float(), Hh, "sigmoid")
                out = O.lrid_attention_residual_read_ref(vals, keys, qq, Hh, c["scale"], True)
            if not c.get("fwd_only"):
                out.backward(up)

        for _ in range(2):
            step()
        times = []
        t_end = time.perf_counter() + budget_s / 2
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
        med = sorted(times)[len(times) // 2]
        f_b, b_b = bytes_per_token(dict(c, dtype=dt))
        by[name] = {"tokens_per_s": round(B * T / med, 1), "gbs": round((f_b + b_b) * B * T / med / 1e9, 2),
                    "median_s": round(med, 5), "iterations": len(times)}
    main = "fp32" if c["dtype"] == torch.float32 else "bf16"
    return dict(value=by[main]["tokens_per_s"], unit="tokens/s", cores=cores, kind="port",
                sample=f"oracle eager fwd{'' if c.get('fwd_only') else '+bwd'} on B={B} T={T} tokens of the "
                       f"workload's rows, median of >= 5 iterations after 2 warmups, per dtype; value is {main}; "
                       f"torch {torch.__version__}",
                cpu_model=_cpu_model(), by_dtype=by)


def copy_calibration(steps, gib=1.0):
    """A plain device-to-device copy of known size: the achievable-bandwidth
    reference, and the kernel whose FETCH_SIZE / WRITE_SIZE counters scale the
    AttnRes kernels' counter readings to bytes."""
    n = int(gib * (1 << 30)) // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    nbytes = 2 * n * 4
    print(json.dumps({"copy_bytes_per_launch": nbytes, "ms": round(ms, 5), "gbs": round(nbytes / ms / 1e6, 1)}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + sorted(PHASE_CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-api", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="time a plain 1 GiB device copy instead (bandwidth / counter reference)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the AttnRes read shards "
              "by tokens with no exchange between GPUs", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(args.steps)
        return
    if args.config in PHASE_CONFIGS:
        bench_phase(args, dev)
        return
    c = CONFIGS[args.config]
    wl = make_workload(c, dev)
    stream = torch.cuda.current_stream(dev)
    sv = ctypes.c_void_p(stream.cuda_stream)

    ms = time_steps(wl, args.steps, args.warmup, stream, sv)
    f_ms, b_ms = time_kernels(wl, args.steps, stream, sv)
    fk_ms, bk_ms = time_main_kernels(wl, args.steps, sv)
    api_ms = None if args.no_api else time_api(c, wl, max(20, args.steps), 5)

    fwd_b, bwd_b = bytes_per_token(c)
    n_tok = wl.n_tok
    tok_s = n_tok / (ms / 1e3)
    gbs_step = (fwd_b + bwd_b) * n_tok / (ms / 1e3) / 1e9
    fwd_gbs = fwd_b * n_tok / (fk_ms / 1e3) / 1e9
    bwd_gbs = bwd_b * n_tok / (bk_ms / 1e3) / 1e9 if bwd_b else 0.0
    dom_gbs, dom_name, dom_bytes = (bwd_gbs, "backward", bwd_b) if bwd_b else (fwd_gbs, "forward", fwd_b)
    # HBM bytes per launch of the dominant kernel, measured with rocprofv3
    # FETCH_SIZE / WRITE_SIZE (scaled by a copy of known size) and kept in
    # profiles/traffic_<config>.json; null when no measurement is recorded
    # (only when the record names the kernel family this configuration runs)
    traffic = traffic_kernel = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            rec = json.load(f).get("kernels", {}).get("bwd" if bwd_b else "fwd")
        family = ("lr_" if c["kind"] != "base" else "base_") + ("bwd" if bwd_b else "fwd")
        if rec and family in rec.get("name", ""):
            traffic, traffic_kernel = rec["bytes_per_launch"], rec["name"]

    res = {
        "metric": "AttnRes fwd+bwd tokens/s (d=1024,N=13,r=64,bf16); HBM GB/s as % of peak",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float32: "f32", torch.float16: "f16"}[c["dtype"]],
        "data": "synthetic",
        "config": {"workload": f"{args.config}: " + ("LR" if c["kind"] != "base" else "base")
                   + f" read fwd+bwd B{c['B']} T{c['T']} d{c['D']} N{c['N']}"
                   + (f" r{c['R']} H{c['H']}" if c["R"] else "") + (" gated dyn query" if c["kind"] == "lr_gated"
                                                                    else "")
                   + (" keys rms_norm(v)W_k" if c.get("value_keys") else "")
                   + (" + static source keys" if c.get("static_keys") else ""),
                   "tokens": n_tok, "parallelism": "single GPU", "input_sets": c.get("sets", 1)},
        "hbm_gbs_step": round(gbs_step, 1),
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(dom_gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dom_gbs / PEAK_HBM_GBS, 4),
                     "bytes_per_token": dom_bytes, "algorithmic_bytes_per_launch": dom_bytes * n_tok,
                     "traffic": traffic, "traffic_kernel": traffic_kernel},
        "kernels": {"forward_ms": round(fk_ms, 5), "forward_gbs": round(fwd_gbs, 1),
                    "backward_ms": round(bk_ms, 5), "backward_gbs": round(bwd_gbs, 1),
                    "forward_call_ms": round(f_ms, 5), "backward_call_ms": round(b_ms, 5),
                    "bytes_per_token": {"fwd": fwd_b, "bwd": bwd_b}},
        "api": {"ms_per_step": round(api_ms, 4) if api_ms else None},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(c, args.cpu_seconds)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
