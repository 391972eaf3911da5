"""attnres_read_backward_noalloc against attnres_read_backward, through the C ABI.

The no-allocation entry point runs the same kernels with the partial sums in
the library's fixed per-device array, so every gradient must equal the
workspace entry point's bit for bit.  Two calls in a row, the second with a
smaller input (the array keeps the first call's contents), for the LR read
(static query and logit bias: query and bias partial sums), the LR read with a
per-site gate (gate partial sums), the LR read with per-source static keys
(their column sums go into the array after the partial rows), and the base read
(tiled partial rows).
"""

import ctypes

import pytest
import torch

import _attnres_hip as H

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    H.load()


def _inputs(seed, kind, B, T):
    g = torch.Generator(device=DEV).manual_seed(seed)
    rn = lambda *s, std=1.0: (torch.randn(s, generator=g, device=DEV) * std).to(torch.bfloat16)  # noqa: E731
    if kind == "base":
        D, N = 768, 7
        vals = [rn(B, T, D) for _ in range(N)]
        q = rn(D, std=0.1)
        bias = torch.randn(N, generator=g, device=DEV)
        desc = H.Desc(vals, [], q, None, None, bias, 1, 1.0, True, False, H.MODE_SOFTMAX, H.GATE_NONE, False)
        return desc, (vals, q, bias), dict(want_dquery=True, want_dgate=False, want_dbias=True,
                                           query_shape=tuple(q.shape), gate_shape=(0,), lr=False,
                                           has_query_dyn=False)
    D, N, R, Hh = 1024, 13, 64, 4
    vals = [rn(B, T, D) for _ in range(N)]
    keys = [rn(B, T, R) for _ in range(N)]
    if kind == "lr":
        q = rn(Hh, R // Hh, std=0.5)
        bias = torch.randn(N, generator=g, device=DEV)
        desc = H.Desc(vals, keys, q, None, None, bias, Hh, 0.25, True, False, H.MODE_SOFTMAX, H.GATE_NONE, False)
        return desc, (vals, keys, q, bias), dict(want_dquery=True, want_dgate=False, want_dbias=True,
                                                 query_shape=tuple(q.shape), gate_shape=(0,), lr=True,
                                                 has_query_dyn=False)
    if kind == "lr_static":
        q = rn(Hh, R // Hh, std=0.5)
        sk = rn(N, R, std=0.5)
        desc = H.Desc(vals, keys, q, None, None, None, Hh, 0.25, True, False, H.MODE_SOFTMAX, H.GATE_NONE, False,
                      static_keys=sk)
        return desc, (vals, keys, q, sk), dict(want_dquery=True, want_dgate=False, want_dbias=False,
                                               query_shape=tuple(q.shape), gate_shape=(0,), lr=True,
                                               has_query_dyn=False, want_dstatic=True)
    q = rn(Hh, R // Hh, std=0.5)
    qd = rn(B, T, R)
    gate = rn(Hh)
    desc = H.Desc(vals, keys, q, qd, gate, None, Hh, 0.25, True, False, H.MODE_SOFTMAX, H.GATE_LINEAR, False)
    return desc, (vals, keys, q, qd, gate), dict(want_dquery=True, want_dgate=True, want_dbias=False,
                                                 query_shape=tuple(q.shape), gate_shape=tuple(gate.shape), lr=True,
                                                 has_query_dyn=True)


def _noalloc_backward(desc, grad_out, weights, want):
    """The same gradient buffers _attnres_hip.backward allocates, filled by the no-allocation entry point."""
    lib = H.load()
    n, nt = desc.n_src, desc.n_tok
    dvals = [torch.empty((nt, desc.D), device=DEV, dtype=torch.bfloat16) for _ in range(n)]
    dkeys = [torch.empty((nt, desc.R), device=DEV, dtype=desc.key_dtype) for _ in range(n)] if want["lr"] else []
    dq = torch.empty(want["query_shape"], device=DEV, dtype=desc.query_dtype)
    dqd = torch.empty((nt, desc.R), device=DEV, dtype=desc.query_dtype) if want["has_query_dyn"] else None
    dg = torch.empty(want["gate_shape"], device=DEV, dtype=torch.bfloat16) if want["want_dgate"] else None
    db = torch.empty((n,), device=DEV, dtype=torch.float32) if want["want_dbias"] else None
    dsk = torch.empty((n, desc.R), device=DEV, dtype=desc.key_dtype) if want.get("want_dstatic") else None
    gr = H.ReadGrads()
    gr.grad_out = grad_out.data_ptr()
    gr.weights = ctypes.cast(ctypes.c_void_p(weights.data_ptr()), ctypes.POINTER(ctypes.c_float))
    dv_arr = (ctypes.c_void_p * n)(*[t.data_ptr() for t in dvals])
    gr.dvalues = dv_arr
    if dkeys:
        dk_arr = (ctypes.c_void_p * n)(*[t.data_ptr() for t in dkeys])
        gr.dkeys = dk_arr
    gr.dquery = dq.data_ptr()
    gr.dquery_dyn = dqd.data_ptr() if dqd is not None else None
    gr.dgate = dg.data_ptr() if dg is not None else None
    gr.dbias = ctypes.cast(ctypes.c_void_p(db.data_ptr()), ctypes.POINTER(ctypes.c_float)) if db is not None else None
    gr.dstatic_keys = dsk.data_ptr() if dsk is not None else None
    gr.workspace = None  # ignored by the no-allocation entry point
    gr.workspace_bytes = 0
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.attnres_read_backward_noalloc(ctypes.byref(desc.c), ctypes.byref(gr), stream)
    assert rc == 0, lib.attnres_last_error().decode()
    return dvals, dkeys, dq, dqd, dg, db, dsk


@pytest.mark.parametrize("kind", ["lr", "lr_gated", "lr_static", "base"])
def test_noalloc_backward_equals_the_workspace_backward(kind):
    for call, (B, T) in enumerate([(4, 1024), (1, 37)]):  # the second call is smaller
        print(f"no-alloc backward: {kind} call {call} B{B} T{T}", flush=True)
        desc, keep, want = _inputs(40 + call, kind, B, T)
        _, w, _, _ = H.forward(desc, torch.device(DEV), torch.bfloat16, True, False, True)
        g = torch.Generator(device=DEV).manual_seed(90 + call)
        grad_out = torch.randn((desc.n_tok, desc.D), generator=g, device=DEV).to(torch.bfloat16)
        ref = H.backward(desc, torch.device(DEV), torch.bfloat16, grad_out, None, None, w, **want)
        got = _noalloc_backward(desc, grad_out, w, want)
        torch.cuda.synchronize()
        dvals_r, dkeys_r, *rest_r = ref
        dvals_g, dkeys_g, *rest_g = got
        for a, b in zip(dvals_r + dkeys_r, dvals_g + dkeys_g):
            assert torch.equal(a, b)
        assert len(rest_r) == len(rest_g)
        for a, b in zip(rest_r, rest_g):
            assert (a is None) == (b is None)
            if a is not None:
                assert torch.equal(a, b), (kind, call, a, b)
