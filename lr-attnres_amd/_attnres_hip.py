"""ctypes binding of libattnres_hip.so (the C ABI in include/attnres_hip.h).

This is the whole host boundary: tensors become device pointers, row strides
and sizes; the call runs on the current HIP stream of the tensors' device.
There is no CPU path: a missing library or a non-GPU tensor raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libattnres_hip.so")

ABI_VERSION = 9
MAX_SOURCES = 64
NOALLOC_SCRATCH_BYTES = 32 << 20

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
MODE_SOFTMAX, MODE_AVERAGE = 0, 1
GATE_NONE, GATE_LINEAR, GATE_SIGMOID = 0, 1, 2
MERGE_ADDCMUL, MERGE_LERP = 0, 1
PHASE1_MAX_QUERIES = 16
PHASE_MAX_DIM = 4096
SITE_LOGITS_MAX_QUERIES = 256
SITE_LOGITS_MAX_RANK = 128
FLT_EPSILON = float(torch.finfo(torch.float32).eps)


class ReadDesc(ctypes.Structure):
    """attnres_read_desc (field order and types as in include/attnres_hip.h)."""

    _fields_ = [
        ("n_src", c_int32),
        ("dtype", c_int32),
        ("n_tok", c_int64),
        ("dim", c_int32),
        ("rank", c_int32),
        ("heads", c_int32),
        ("mode", c_int32),
        ("key_norm", c_int32),
        ("normalize_output", c_int32),
        ("logit_scale", c_float),
        ("norm_eps", c_float),
        ("values", POINTER(c_void_p)),
        ("value_row_stride", POINTER(c_int64)),
        ("keys", POINTER(c_void_p)),
        ("key_row_stride", POINTER(c_int64)),
        ("query", c_void_p),
        ("query_dyn", c_void_p),
        ("query_dyn_row_stride", c_int64),
        ("gate", c_void_p),
        ("gate_per_token", c_int32),
        ("gate_act", c_int32),
        ("logit_bias", POINTER(c_float)),
        ("key_dtype", c_int32),
        ("static_keys", c_void_p),
    ]


class ReadGrads(ctypes.Structure):
    """attnres_read_grads."""

    _fields_ = [
        ("grad_out", c_void_p),
        ("out_prenorm", c_void_p),
        ("out_inv_rms", POINTER(c_float)),
        ("weights", POINTER(c_float)),
        ("dvalues", POINTER(c_void_p)),
        ("dkeys", POINTER(c_void_p)),
        ("dquery", c_void_p),
        ("dquery_dyn", c_void_p),
        ("dgate", c_void_p),
        ("dbias", POINTER(c_float)),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("dstatic_keys", c_void_p),
    ]


class Phase1Desc(ctypes.Structure):
    """attnres_phase1_desc."""

    _fields_ = [
        ("n_src", c_int32),
        ("n_q", c_int32),
        ("dtype", c_int32),
        ("logits_dtype", c_int32),
        ("n_tok", c_int64),
        ("dim", c_int32),
        ("normalize_output", c_int32),
        ("norm_eps", c_float),
        ("values", POINTER(c_void_p)),
        ("value_row_stride", POINTER(c_int64)),
        ("logits", c_void_p),
        ("logit_q_stride", c_int64),
        ("logit_s_stride", c_int64),
        ("source_logits", POINTER(c_void_p)),
    ]


class SiteLogitsDesc(ctypes.Structure):
    """attnres_site_logits_desc."""

    _fields_ = [
        ("dtype", c_int32),
        ("logits_dtype", c_int32),
        ("n_tok", c_int64),
        ("rank", c_int32),
        ("n_q", c_int32),
        ("key_norm", c_int32),
        ("norm_eps", c_float),
        ("logit_scale", c_float),
        ("logit_bias", c_float),
        ("key", c_void_p),
        ("key_row_stride", c_int64),
        ("queries", c_void_p),
    ]


class KeyedLogitsDesc(ctypes.Structure):
    """attnres_keyed_logits_desc."""

    _fields_ = [
        ("n_src", c_int32),
        ("n_q", c_int32),
        ("dtype", c_int32),
        ("n_tok", c_int64),
        ("dim", c_int32),
        ("key_norm", c_int32),
        ("norm_eps", c_float),
        ("values", POINTER(c_void_p)),
        ("value_row_stride", POINTER(c_int64)),
        ("queries", c_void_p),
    ]


class Phase2Desc(ctypes.Structure):
    """attnres_phase2_desc."""

    _fields_ = [
        ("dtype", c_int32),
        ("n_tok", c_int64),
        ("dim", c_int32),
        ("rank", c_int32),
        ("logit_given", c_int32),
        ("merge", c_int32),
        ("key_norm", c_int32),
        ("normalize_output", c_int32),
        ("logit_scale", c_float),
        ("norm_eps", c_float),
        ("logit_bias", c_float),
        ("logit_bias_dev", POINTER(c_float)),
        ("value_scale", c_float),
        ("value_scale_dev", POINTER(c_float)),
        ("scale_key", c_int32),
        ("partial_value", c_void_p),
        ("partial_value_row_stride", c_int64),
        ("partial_key", c_void_p),
        ("partial_key_row_stride", c_int64),
        ("query", c_void_p),
        ("partial_logit", c_void_p),
        ("partial_logit_dtype", c_int32),
        ("interblock_output", c_void_p),
        ("interblock_row_stride", c_int64),
        ("interblock_lse", POINTER(c_float)),
    ]


class Phase2Grads(ctypes.Structure):
    """attnres_phase2_grads."""

    _fields_ = [
        ("grad_out", c_void_p),
        ("dpartial_value", c_void_p),
        ("dpartial_key", c_void_p),
        ("dquery", c_void_p),
        ("dinterblock_output", c_void_p),
        ("dinterblock_lse", POINTER(c_float)),
        ("dpartial_logit", c_void_p),
        ("dlogit_bias", POINTER(c_float)),
        ("dvalue_scale", POINTER(c_float)),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("dquery_rows", c_int32),
        ("dquery_row", c_int32),
    ]


_lib = None


def library_path() -> str:
    return LIB_PATH


class KeyedSplitDesc(ctypes.Structure):
    """attnres_keyed_split_desc (include/attnres_hip.h)."""
    _fields_ = [("dtype", c_int32), ("n_tok", c_int64), ("dim", c_int32), ("rank", c_int32),
                ("proj_cols", c_int32), ("heads", c_int32), ("key_norm", c_int32), ("norm_eps", c_float),
                ("projected", c_void_p), ("row_stride", c_int64)]


class BlockAccumDesc(ctypes.Structure):
    """attnres_block_accum_desc (include/attnres_hip.h)."""
    _fields_ = [("split", KeyedSplitDesc), ("complete", c_int32), ("partial_value", c_void_p),
                ("partial_key", c_void_p), ("value_norm", c_int32), ("scale_key", c_int32),
                ("value_scale", c_float), ("value_scale_dev", POINTER(c_float))]


class AccumReadDesc(ctypes.Structure):
    """attnres_accum_read_desc (include/attnres_hip.h): a block accumulation and the merge that reads it."""
    _fields_ = [("accum", BlockAccumDesc), ("read", Phase2Desc)]


class ValueKeyDesc(ctypes.Structure):
    """attnres_value_key_desc (include/attnres_hip.h)."""
    _fields_ = [("n_src", c_int32), ("dtype", c_int32), ("n_tok", c_int64), ("dim", c_int32),
                ("norm_eps", c_float), ("values", POINTER(c_void_p)), ("value_row_stride", POINTER(c_int64))]


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise with a build hint if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"attnres HIP library not found at {LIB_PATH}; build it with "
            "`python lr-attnres_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    lib.attnres_abi_version.restype = c_int
    lib.attnres_last_error.restype = ctypes.c_char_p
    lib.attnres_read_forward.restype = c_int
    lib.attnres_read_forward.argtypes = [POINTER(ReadDesc), c_void_p, c_void_p, POINTER(c_float), POINTER(c_float),
                                         c_void_p]
    lib.attnres_read_backward.restype = c_int
    lib.attnres_read_backward.argtypes = [POINTER(ReadDesc), POINTER(ReadGrads), c_void_p]
    lib.attnres_read_backward_workspace_size.restype = c_size_t
    lib.attnres_read_backward_workspace_size.argtypes = [POINTER(ReadDesc)]
    lib.attnres_read_backward_noalloc.restype = c_int
    lib.attnres_read_backward_noalloc.argtypes = [POINTER(ReadDesc), POINTER(ReadGrads), c_void_p]
    lib.attnres_phase1_forward.restype = c_int
    lib.attnres_phase1_forward.argtypes = [POINTER(Phase1Desc), c_void_p, c_void_p, POINTER(c_float),
                                           POINTER(c_float), c_void_p]
    lib.attnres_phase1_backward.restype = c_int
    lib.attnres_phase1_backward.argtypes = [POINTER(Phase1Desc), c_void_p, POINTER(c_float), c_void_p,
                                            POINTER(c_float), POINTER(c_void_p), c_void_p, c_void_p]
    lib.attnres_phase1_backward_sites.restype = c_int
    lib.attnres_phase1_backward_sites.argtypes = [POINTER(Phase1Desc), POINTER(c_void_p), POINTER(c_void_p),
                                                  c_void_p, POINTER(c_float), POINTER(c_void_p),
                                                  POINTER(c_void_p), c_int64, c_void_p]
    lib.attnres_site_logits_forward.restype = c_int
    lib.attnres_site_logits_forward.argtypes = [POINTER(SiteLogitsDesc), c_void_p, c_void_p]
    lib.attnres_site_logits_backward.restype = c_int
    lib.attnres_site_logits_backward.argtypes = [POINTER(SiteLogitsDesc), POINTER(c_void_p), c_void_p, c_void_p,
                                                 c_void_p, c_void_p]
    lib.attnres_keyed_logits_forward.restype = c_int
    lib.attnres_keyed_logits_forward.argtypes = [POINTER(KeyedLogitsDesc), c_void_p, POINTER(c_float), c_void_p]
    lib.attnres_keyed_logits_backward_workspace_size.restype = c_size_t
    lib.attnres_keyed_logits_backward_workspace_size.argtypes = [POINTER(KeyedLogitsDesc)]
    lib.attnres_keyed_logits_backward.restype = c_int
    lib.attnres_keyed_logits_backward.argtypes = [POINTER(KeyedLogitsDesc), c_void_p, POINTER(c_float),
                                                  POINTER(c_void_p), c_void_p, c_void_p, c_size_t, c_void_p]
    lib.attnres_phase2_forward.restype = c_int
    lib.attnres_phase2_forward.argtypes = [POINTER(Phase2Desc), c_void_p, c_void_p]
    lib.attnres_phase2_backward.restype = c_int
    lib.attnres_phase2_backward.argtypes = [POINTER(Phase2Desc), POINTER(Phase2Grads), c_void_p]
    lib.attnres_phase2_backward_workspace_size.restype = c_size_t
    lib.attnres_phase2_backward_workspace_size.argtypes = [POINTER(Phase2Desc)]
    lib.attnres_keyed_split_forward.restype = c_int
    lib.attnres_keyed_split_forward.argtypes = [POINTER(KeyedSplitDesc), c_void_p, c_void_p, POINTER(c_float),
                                                c_void_p]
    lib.attnres_keyed_split_backward.restype = c_int
    lib.attnres_keyed_split_backward.argtypes = [POINTER(KeyedSplitDesc), c_void_p, c_void_p, POINTER(c_float),
                                                 c_void_p, c_void_p]
    lib.attnres_accum_read_forward.restype = c_int
    lib.attnres_accum_read_forward.argtypes = [POINTER(AccumReadDesc), c_void_p, c_void_p, POINTER(c_float), c_void_p,
                                               c_void_p]
    lib.attnres_accum_read_backward.restype = c_int
    lib.attnres_accum_read_backward.argtypes = [POINTER(AccumReadDesc), POINTER(Phase2Grads), c_void_p, c_int64,
                                                c_void_p, POINTER(c_float), c_void_p, c_void_p, c_void_p]
    lib.attnres_block_accum_forward.restype = c_int
    lib.attnres_block_accum_forward.argtypes = [POINTER(BlockAccumDesc), c_void_p, c_void_p, POINTER(c_float),
                                                POINTER(c_float), c_void_p]
    lib.attnres_block_accum_backward_workspace_size.restype = c_size_t
    lib.attnres_block_accum_backward_workspace_size.argtypes = [POINTER(BlockAccumDesc)]
    lib.attnres_block_accum_backward.restype = c_int
    lib.attnres_block_accum_backward.argtypes = [POINTER(BlockAccumDesc), c_void_p, c_int64, c_void_p,
                                                 POINTER(c_float), POINTER(c_float), c_void_p, c_void_p,
                                                 POINTER(c_float), c_void_p, c_size_t, c_void_p]
    lib.attnres_value_norm_forward.restype = c_int
    lib.attnres_value_norm_forward.argtypes = [POINTER(ValueKeyDesc), c_void_p, POINTER(c_float), c_void_p]
    lib.attnres_value_norm_backward.restype = c_int
    lib.attnres_value_norm_backward.argtypes = [POINTER(ValueKeyDesc), c_void_p, POINTER(c_float),
                                                POINTER(c_void_p), c_void_p]
    lib.attnres_kernel_timing.restype = c_int
    lib.attnres_kernel_timing.argtypes = [c_int]
    lib.attnres_test_phase2_block_layout.restype = c_int
    lib.attnres_test_phase2_block_layout.argtypes = [c_int]
    lib.attnres_kernel_times.restype = c_int
    lib.attnres_kernel_times.argtypes = [POINTER(c_float), c_int]
    v = lib.attnres_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"libattnres_hip ABI {v} != expected {ABI_VERSION}; rebuild the library")
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
    except (OSError, RuntimeError):
        return False
    return torch.cuda.is_available()


def _ptr(t):
    return c_void_p(t.data_ptr()) if t is not None else c_void_p(0)


def _fptr(t):
    return ctypes.cast(c_void_p(t.data_ptr()), POINTER(c_float)) if t is not None else None


def _check(rc: int, what: str):
    if rc != 0:
        msg = load().attnres_last_error().decode(errors="replace")
        raise RuntimeError(f"attnres HIP {what} failed (code {rc}): {msg}")


def _stream(device) -> c_void_p:
    return c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _row_view_ok(t: torch.Tensor) -> bool:
    # [B,T,W] with a contiguous last dim and one uniform token stride
    return t.dim() == 3 and t.stride(-1) == 1 and t.stride(0) == t.size(1) * t.stride(1)


def as_rows(t: torch.Tensor) -> torch.Tensor:
    """A [B,T,W] tensor whose tokens are uniformly strided rows (copy if not)."""
    return t if t.is_contiguous() or _row_view_ok(t) else t.contiguous()


class Desc:
    """Builds the C descriptor for one read; keeps the ctypes arrays alive."""

    def __init__(self, values, keys, query, query_dyn, gate, bias, heads, logit_scale, key_norm,
                 normalize_output, mode, gate_act, gate_per_token, eps=FLT_EPSILON, static_keys=None):
        v0 = values[0]
        B, T, D = v0.shape
        n = len(values)
        # the descriptor holds raw device pointers: keep the tensors alive with it
        self._tensors = (list(values), list(keys), query, query_dyn, gate, bias, static_keys)
        self.has_static_keys = static_keys is not None
        self.n_src = n
        self.n_tok = B * T
        self.D = D
        self.R = keys[0].size(-1) if keys else 0
        self.heads = heads
        # gradient dtypes: keys' for the key gradients, the query's (the
        # logit dtype of an LR read) for the query gradients
        self.key_dtype = keys[0].dtype if keys else v0.dtype
        qref = query if query is not None else query_dyn
        self.query_dtype = qref.dtype if qref is not None else v0.dtype
        self._vals = (c_void_p * n)(*[t.data_ptr() for t in values])
        self._vstr = (c_int64 * n)(*[t.stride(1) for t in values])
        if keys:
            self._keys = (c_void_p * n)(*[t.data_ptr() for t in keys])
            self._kstr = (c_int64 * n)(*[t.stride(1) for t in keys])
        d = ReadDesc()
        d.n_src = n
        d.dtype = DTYPE_CODE[v0.dtype]
        d.n_tok = self.n_tok
        d.dim = D
        d.rank = self.R
        d.heads = heads
        d.mode = mode
        d.key_norm = int(bool(key_norm))
        d.normalize_output = int(bool(normalize_output))
        d.logit_scale = float(logit_scale)
        d.norm_eps = float(eps)
        d.values = self._vals
        d.value_row_stride = self._vstr
        if keys:
            d.keys = self._keys
            d.key_row_stride = self._kstr
        d.query = query.data_ptr() if query is not None else None
        d.query_dyn = query_dyn.data_ptr() if query_dyn is not None else None
        d.query_dyn_row_stride = query_dyn.stride(1) if query_dyn is not None else 0
        d.gate = gate.data_ptr() if gate is not None else None
        d.gate_per_token = int(bool(gate_per_token))
        d.gate_act = gate_act
        d.logit_bias = _fptr(bias)
        d.key_dtype = DTYPE_CODE[self.key_dtype]
        d.static_keys = static_keys.data_ptr() if static_keys is not None else None
        self.c = d


def forward(desc: Desc, device, dtype, need_weights: bool, normalize_output: bool, for_backward: bool):
    """Launch the forward.

    Returns (out [n_tok, D], weights [n_tok,H,N] | empty, inv_rms [n_tok] | empty,
    prenorm [n_tok, D] | empty); weights are written when ``need_weights``, the
    output-norm state when ``normalize_output and for_backward``.
    """
    lib = load()
    out = torch.empty((desc.n_tok, desc.D), device=device, dtype=dtype)
    if need_weights:
        w = torch.empty((desc.n_tok, desc.heads, desc.n_src), device=device, dtype=torch.float32)
    else:
        w = torch.empty((0,), device=device, dtype=torch.float32)
    keep = normalize_output and for_backward
    inv = torch.empty((desc.n_tok if keep else 0,), device=device, dtype=torch.float32)
    pre = torch.empty((desc.n_tok, desc.D) if keep else (0,), device=device, dtype=dtype)
    rc = lib.attnres_read_forward(ctypes.byref(desc.c), _ptr(out), _ptr(pre) if keep else None,
                                  _fptr(w) if need_weights else None, _fptr(inv) if keep else None, _stream(device))
    _check(rc, "forward")
    return out, w, inv, pre


def _row_blocks(count: int, n_tok: int, width: int, device, dtype, batched: bool, lead=None):
    """``count`` dense gradient buffers of shape ``lead + (width,)`` (``lead``
    defaults to ``(n_tok,)``): separate allocations, or (``batched``) views of
    one allocation."""
    shape = (tuple(lead) if lead is not None else (n_tok,)) + (width,)
    if not batched:
        return [torch.empty(shape, device=device, dtype=dtype) for _ in range(count)]
    return list(torch.empty((count,) + shape, device=device, dtype=dtype).unbind(0))


def backward(desc: Desc, device, dtype, grad_out, prenorm, inv_rms, weights, want_dquery: bool,
             want_dgate: bool, want_dbias: bool, query_shape, gate_shape, lr: bool, has_query_dyn: bool,
             batched: bool = False, lead=None, want_dstatic: bool = False):
    """Launch the backward; returns (dvalues list, dkeys list, dquery, dquery_dyn, dgate, dbias,
    dstatic_keys [N, R] | None).

    With ``batched`` the per-source gradients are views of one allocation per
    kind (fewer allocator calls); otherwise each is its own tensor (the
    library op's outputs may not alias one another).  ``lead`` shapes each
    per-source gradient as ``lead + (width,)`` (default ``(n_tok,)``)."""
    lib = load()
    n = desc.n_src
    dvals = _row_blocks(n, desc.n_tok, desc.D, device, dtype, batched, lead)
    dkeys = _row_blocks(n, desc.n_tok, desc.R, device, desc.key_dtype, batched, lead) if lr else []
    dq = torch.empty(query_shape, device=device, dtype=desc.query_dtype) if want_dquery else None
    dqd = torch.empty((desc.n_tok, desc.R), device=device, dtype=desc.query_dtype) if has_query_dyn else None
    dg = torch.empty(gate_shape, device=device, dtype=dtype) if want_dgate else None
    db = torch.empty((n,), device=device, dtype=torch.float32) if want_dbias else None
    dsk = torch.empty((n, desc.R), device=device, dtype=desc.key_dtype) if want_dstatic else None
    g = ReadGrads()
    g.grad_out = grad_out.data_ptr()
    g.out_prenorm = prenorm.data_ptr() if prenorm is not None and prenorm.numel() else None
    g.out_inv_rms = _fptr(inv_rms) if inv_rms is not None and inv_rms.numel() else None
    g.weights = _fptr(weights) if weights is not None and weights.numel() else None
    dv_arr = (c_void_p * n)(*[t.data_ptr() for t in dvals])
    g.dvalues = dv_arr
    if lr:
        dk_arr = (c_void_p * n)(*[t.data_ptr() for t in dkeys])
        g.dkeys = dk_arr
    g.dquery = dq.data_ptr() if dq is not None else None
    g.dquery_dyn = dqd.data_ptr() if dqd is not None else None
    g.dgate = dg.data_ptr() if dg is not None else None
    g.dbias = _fptr(db)
    g.dstatic_keys = dsk.data_ptr() if dsk is not None else None
    # workspace for the cross-token partial sums of the requested gradients
    ws_bytes = lib.attnres_read_backward_workspace_size(ctypes.byref(desc.c))
    ws = torch.empty((max(int(ws_bytes), 1),), device=device, dtype=torch.uint8)
    g.workspace = ws.data_ptr()
    g.workspace_bytes = int(ws_bytes)
    rc = lib.attnres_read_backward(ctypes.byref(desc.c), ctypes.byref(g), _stream(device))
    _check(rc, "backward")
    return dvals, dkeys, dq, dqd, dg, db, dsk


# ---------------------------------------------------------------------------
# cached-logit phases
# ---------------------------------------------------------------------------

class Phase1:
    """Descriptor of one phase-1 call: S value row tensors [n_tok, D] (any
    uniform row stride) and dense logits [Q, S, n_tok]."""

    def __init__(self, values, logits, normalize_output, eps=FLT_EPSILON):
        n = len(values)
        self._tensors = (list(values), logits)
        self.n_src = n
        self.n_q = logits.size(0)
        self.n_tok = values[0].size(0)
        self.D = values[0].size(1)
        self._vals = (c_void_p * n)(*[t.data_ptr() for t in values])
        self._vstr = (c_int64 * n)(*[t.stride(0) for t in values])
        d = Phase1Desc()
        d.n_src = n
        d.n_q = self.n_q
        d.dtype = DTYPE_CODE[values[0].dtype]
        d.logits_dtype = DTYPE_CODE[logits.dtype]
        d.n_tok = self.n_tok
        d.dim = self.D
        d.normalize_output = int(bool(normalize_output))
        d.norm_eps = float(eps)
        d.values = self._vals
        d.value_row_stride = self._vstr
        d.logits = logits.data_ptr()
        d.logit_q_stride = n * self.n_tok
        d.logit_s_stride = self.n_tok
        self.c = d


def phase1_forward(desc: Phase1, device, dtype, for_backward: bool):
    """Returns (out [Q, n_tok, D], lse [Q, n_tok], prenorm | empty, inv_rms | empty)."""
    lib = load()
    Q, n, D = desc.n_q, desc.n_tok, desc.D
    out = torch.empty((Q, n, D), device=device, dtype=dtype)
    lse = torch.empty((Q, n), device=device, dtype=torch.float32)
    keep = bool(desc.c.normalize_output) and for_backward
    pre = torch.empty((Q, n, D) if keep else (0,), device=device, dtype=dtype)
    inv = torch.empty((Q, n) if keep else (0,), device=device, dtype=torch.float32)
    rc = lib.attnres_phase1_forward(ctypes.byref(desc.c), _ptr(out), _ptr(pre) if keep else None, _fptr(lse),
                                    _fptr(inv) if keep else None, _stream(device))
    _check(rc, "phase-1 forward")
    return out, lse, pre, inv


def phase1_backward(desc: Phase1, device, dtype, logits_dtype, grad_out, grad_lse, prenorm, inv_rms,
                    batched: bool = False):
    """Returns (dvalues list of [n_tok, D], dlogits [Q, S, n_tok])."""
    lib = load()
    n = desc.n_src
    dvals = _row_blocks(n, desc.n_tok, desc.D, device, dtype, batched)
    dlog = torch.empty((desc.n_q, n, desc.n_tok), device=device, dtype=logits_dtype)
    dv_arr = (c_void_p * n)(*[t.data_ptr() for t in dvals])
    keep = prenorm is not None and prenorm.numel() > 0
    rc = lib.attnres_phase1_backward(ctypes.byref(desc.c), _ptr(grad_out),
                                     _fptr(grad_lse) if grad_lse is not None else None,
                                     _ptr(prenorm) if keep else None, _fptr(inv_rms) if keep else None, dv_arr,
                                     _ptr(dlog), _stream(device))
    _check(rc, "phase-1 backward")
    return dvals, dlog


class Phase1Sources:
    """Descriptor of one phase-1 call whose logits come per source: S value row
    tensors [n_tok, D] (any uniform row stride) and S logits tensors [Q, n_tok]
    (dense, one dtype), source s's logit for site q at logits[s][q]."""

    def __init__(self, values, logits, normalize_output, eps=FLT_EPSILON):
        n = len(values)
        self._tensors = (list(values), list(logits))
        self.n_src = n
        self.n_q = logits[0].size(0)
        self.n_tok = values[0].size(0)
        self.D = values[0].size(1)
        self._vals = (c_void_p * n)(*[t.data_ptr() for t in values])
        self._vstr = (c_int64 * n)(*[t.stride(0) for t in values])
        self._logits = (c_void_p * n)(*[t.data_ptr() for t in logits])
        d = Phase1Desc()
        d.n_src = n
        d.n_q = self.n_q
        d.dtype = DTYPE_CODE[values[0].dtype]
        d.logits_dtype = DTYPE_CODE[logits[0].dtype]
        d.n_tok = self.n_tok
        d.dim = self.D
        d.normalize_output = int(bool(normalize_output))
        d.norm_eps = float(eps)
        d.values = self._vals
        d.value_row_stride = self._vstr
        d.logits = None
        d.logit_q_stride = self.n_tok
        d.logit_s_stride = self.n_tok
        d.source_logits = self._logits
        self.c = d


def phase1_backward_sites(desc, device, dtype, logits_dtype, grads_out, grads_lse, prenorm, inv_rms):
    """Per-site upstream gradients (Q tensors [n_tok, D]; lse gradients [n_tok]
    or None each) -> (dvalues list of [n_tok, D], per-source dlogits list of
    [Q, n_tok])."""
    lib = load()
    n, Q = desc.n_src, desc.n_q
    dvals = _row_blocks(n, desc.n_tok, desc.D, device, dtype, False)
    dlog = torch.empty((n, Q, desc.n_tok), device=device, dtype=logits_dtype).unbind(0)
    dv_arr = (c_void_p * n)(*[t.data_ptr() for t in dvals])
    dl_arr = (c_void_p * n)(*[t.data_ptr() for t in dlog])
    go_arr = (c_void_p * Q)(*[t.data_ptr() for t in grads_out])
    gl_arr = (c_void_p * Q)(*[t.data_ptr() if t is not None else None for t in grads_lse])
    keep = prenorm is not None and prenorm.numel() > 0
    rc = lib.attnres_phase1_backward_sites(ctypes.byref(desc.c), go_arr, gl_arr, _ptr(prenorm) if keep else None,
                                           _fptr(inv_rms) if keep else None, dv_arr, dl_arr, desc.n_tok,
                                           _stream(device))
    _check(rc, "phase-1 backward")
    return dvals, list(dlog)


class SiteLogits:
    """Descriptor of one source's site logits: key rows [n_tok, R] (uniform row
    stride) against queries [n_q, R] (dense, key dtype)."""

    def __init__(self, key, queries, key_norm, logit_scale, logits_dtype, logit_bias=0.0, eps=FLT_EPSILON):
        self._tensors = (key, queries)
        self.n_tok, self.R = key.size(0), key.size(1)
        self.n_q = queries.size(0)
        self.dtype = key.dtype
        self.logits_dtype = logits_dtype
        d = SiteLogitsDesc()
        d.dtype = DTYPE_CODE[key.dtype]
        d.logits_dtype = DTYPE_CODE[logits_dtype]
        d.n_tok = self.n_tok
        d.rank = self.R
        d.n_q = self.n_q
        d.key_norm = int(bool(key_norm))
        d.norm_eps = float(eps)
        d.logit_scale = float(logit_scale)
        d.logit_bias = float(logit_bias)
        d.key = key.data_ptr()
        d.key_row_stride = key.stride(0)
        d.queries = queries.data_ptr()
        self.c = d


def site_logits_forward(desc: SiteLogits, device):
    """Returns logits [n_q, n_tok] (logits dtype)."""
    out = torch.empty((desc.n_q, desc.n_tok), device=device, dtype=desc.logits_dtype)
    _check(load().attnres_site_logits_forward(ctypes.byref(desc.c), _ptr(out), _stream(device)), "site-logits forward")
    return out


def site_logits_backward(desc: SiteLogits, device, grads):
    """Per-site logit gradients (n_q tensors [n_tok]) -> (dkey [n_tok, R],
    grad_scaled [n_q, n_tok], key_hat [n_tok, R])."""
    dkey = torch.empty((desc.n_tok, desc.R), device=device, dtype=desc.dtype)
    du = torch.empty((desc.n_q, desc.n_tok), device=device, dtype=desc.dtype)
    khat = torch.empty((desc.n_tok, desc.R), device=device, dtype=desc.dtype)
    g_arr = (c_void_p * desc.n_q)(*[t.data_ptr() for t in grads])
    rc = load().attnres_site_logits_backward(ctypes.byref(desc.c), g_arr, _ptr(dkey), _ptr(du), _ptr(khat),
                                             _stream(device))
    _check(rc, "site-logits backward")
    return dkey, du, khat


class KeyedLogits:
    """Descriptor of the query-bank logits: S value row tensors [n_tok, D]
    (any uniform row stride) and queries [Q, D] (value dtype, contiguous)."""

    def __init__(self, values, queries, key_norm, eps=FLT_EPSILON):
        n = len(values)
        self._tensors = (list(values), queries)
        self.n_src = n
        self.n_q = queries.size(0)
        self.n_tok = values[0].size(0)
        self.D = values[0].size(1)
        self._vals = (c_void_p * n)(*[t.data_ptr() for t in values])
        self._vstr = (c_int64 * n)(*[t.stride(0) for t in values])
        d = KeyedLogitsDesc()
        d.n_src = n
        d.n_q = self.n_q
        d.dtype = DTYPE_CODE[values[0].dtype]
        d.n_tok = self.n_tok
        d.dim = self.D
        d.key_norm = int(bool(key_norm))
        d.norm_eps = float(eps)
        d.values = self._vals
        d.value_row_stride = self._vstr
        d.queries = queries.data_ptr()
        self.c = d


def keyed_logits_forward(desc: KeyedLogits, device, dtype, for_backward: bool):
    """Returns (logits [Q, S, n_tok] in the value dtype, inv_rms [S, n_tok] | empty)."""
    lib = load()
    logits = torch.empty((desc.n_q, desc.n_src, desc.n_tok), device=device, dtype=dtype)
    keep = bool(desc.c.key_norm) and for_backward
    inv = torch.empty((desc.n_src, desc.n_tok) if keep else (0,), device=device, dtype=torch.float32)
    rc = lib.attnres_keyed_logits_forward(ctypes.byref(desc.c), _ptr(logits), _fptr(inv) if keep else None,
                                          _stream(device))
    _check(rc, "keyed-logits forward")
    return logits, inv


def keyed_logits_backward(desc: KeyedLogits, device, dtype, dlogits, inv_rms, want_dq: bool):
    """Returns (dvalues list of [n_tok, D], dqueries [Q, D] | None)."""
    lib = load()
    n = desc.n_src
    dvals = _row_blocks(n, desc.n_tok, desc.D, device, dtype, True)
    dv_arr = (c_void_p * n)(*[t.data_ptr() for t in dvals])
    dq = torch.empty((desc.n_q, desc.D), device=device, dtype=dtype) if want_dq else None
    ws_bytes = lib.attnres_keyed_logits_backward_workspace_size(ctypes.byref(desc.c)) if want_dq else 0
    ws = torch.empty((max(1, ws_bytes),), device=device, dtype=torch.uint8) if want_dq else None
    keep = inv_rms is not None and inv_rms.numel() > 0
    rc = lib.attnres_keyed_logits_backward(ctypes.byref(desc.c), _ptr(dlogits), _fptr(inv_rms) if keep else None,
                                           dv_arr, _ptr(dq) if want_dq else None, _ptr(ws) if want_dq else None,
                                           ws_bytes, _stream(device))
    _check(rc, "keyed-logits backward")
    return dvals, dq


class Phase2:
    """Descriptor of one phase-2 merge over [n_tok] rows."""

    def __init__(self, partial_value, partial_key, query, partial_logit, inter, lse, merge, key_norm,
                 normalize_output, logit_scale, bias_value, bias_tensor, scale_value, scale_tensor, scale_key,
                 eps=FLT_EPSILON):
        self._tensors = (partial_value, partial_key, query, partial_logit, inter, lse, bias_tensor, scale_tensor)
        self.n_tok = partial_value.size(0)
        self.D = partial_value.size(1)
        self.R = partial_key.size(1) if partial_key is not None else 0
        d = Phase2Desc()
        d.dtype = DTYPE_CODE[partial_value.dtype]
        d.n_tok = self.n_tok
        d.dim = self.D
        d.rank = self.R
        d.logit_given = int(partial_logit is not None)
        d.merge = merge
        d.key_norm = int(bool(key_norm))
        d.normalize_output = int(bool(normalize_output))
        d.logit_scale = float(logit_scale)
        d.norm_eps = float(eps)
        d.logit_bias = float(bias_value)
        d.logit_bias_dev = _fptr(bias_tensor)
        d.value_scale = float(scale_value)
        d.value_scale_dev = _fptr(scale_tensor)
        d.scale_key = int(bool(scale_key))
        d.partial_value = partial_value.data_ptr()
        d.partial_value_row_stride = partial_value.stride(0)
        if partial_key is not None:
            d.partial_key = partial_key.data_ptr()
            d.partial_key_row_stride = partial_key.stride(0)
        d.query = query.data_ptr() if query is not None else None
        if partial_logit is not None:
            d.partial_logit = partial_logit.data_ptr()
            d.partial_logit_dtype = DTYPE_CODE[partial_logit.dtype]
        d.interblock_output = inter.data_ptr()
        d.interblock_row_stride = inter.stride(0)
        d.interblock_lse = _fptr(lse)
        self.c = d


def phase2_forward(desc: Phase2, device, dtype):
    lib = load()
    out = torch.empty((desc.n_tok, desc.D), device=device, dtype=dtype)
    rc = lib.attnres_phase2_forward(ctypes.byref(desc.c), _ptr(out), _stream(device))
    _check(rc, "phase-2 forward")
    return out


def phase2_backward(desc: Phase2, device, dtype, grad_out, want_dquery, query_shape, logit_dtype, want_dbias,
                    want_dscale, query_row=None):
    """Returns (dpartial, dpartial_key | None, dquery | None, dinter, dlse, dlogit | None, dbias | None,
    dscale | None).  With query_row, query_shape is a bank's [rows, width] and dquery the bank's
    gradient: the query's gradient in row query_row, zeros elsewhere."""
    lib = load()
    n, D, R = desc.n_tok, desc.D, desc.R
    lr = R > 0
    dp = torch.empty((n, D), device=device, dtype=dtype)
    dpk = torch.empty((n, R), device=device, dtype=dtype) if lr else None
    dq = torch.empty(query_shape, device=device, dtype=dtype) if want_dquery else None
    di = torch.empty((n, D), device=device, dtype=dtype)
    dl = torch.empty((n,), device=device, dtype=torch.float32)
    dlg = torch.empty((n,), device=device, dtype=logit_dtype) if logit_dtype is not None else None
    db = torch.empty((1,), device=device, dtype=torch.float32) if want_dbias else None
    ds = torch.empty((1,), device=device, dtype=torch.float32) if want_dscale else None
    g = Phase2Grads()
    g.grad_out = grad_out.data_ptr()
    g.dpartial_value = dp.data_ptr()
    g.dpartial_key = dpk.data_ptr() if dpk is not None else None
    g.dquery = dq.data_ptr() if dq is not None else None
    g.dinterblock_output = di.data_ptr()
    g.dinterblock_lse = _fptr(dl)
    g.dpartial_logit = dlg.data_ptr() if dlg is not None else None
    g.dlogit_bias = _fptr(db)
    g.dvalue_scale = _fptr(ds)
    if dq is not None and query_row is not None:
        g.dquery_rows = int(query_shape[0])
        g.dquery_row = int(query_row)
    ws_bytes = lib.attnres_phase2_backward_workspace_size(ctypes.byref(desc.c))
    ws = torch.empty((max(int(ws_bytes), 1),), device=device, dtype=torch.uint8)
    g.workspace = ws.data_ptr()
    g.workspace_bytes = int(ws_bytes)
    rc = lib.attnres_phase2_backward(ctypes.byref(desc.c), ctypes.byref(g), _stream(device))
    _check(rc, "phase-2 backward")
    return dp, dpk, dq, di, dl, dlg, db, ds


def keyed_split_desc(dtype, n_tok: int, proj_cols: int, row_stride: int, ptr, dim: int, rank: int, heads: int,
                     key_norm: bool) -> KeyedSplitDesc:
    """Descriptor of a projection y [n_tok, proj_cols] whose rows are row_stride elements apart."""
    if dtype not in DTYPE_CODE:
        raise RuntimeError(f"keyed split: dtype {dtype} is not supported (fp32, bf16, fp16)")
    d = KeyedSplitDesc()
    d.dtype = DTYPE_CODE[dtype]
    d.n_tok = n_tok
    d.dim = dim
    d.rank = rank
    d.proj_cols = proj_cols
    d.heads = heads
    d.key_norm = 1 if key_norm else 0
    d.norm_eps = FLT_EPSILON
    d.projected = ptr
    d.row_stride = row_stride
    return d


def keyed_split_forward(y2d: torch.Tensor, dim: int, rank: int, heads: int, key_norm: bool):
    """(out [n_tok, dim], key [n_tok, rank], key_inv_rms [n_tok, heads] fp32, or [0] without key norm)."""
    lib = load()
    n, P = y2d.size(0), y2d.size(1)
    d = keyed_split_desc(y2d.dtype, n, P, y2d.stride(0) if n > 1 else P, y2d.data_ptr() if n else None, dim, rank,
                         heads, key_norm)
    out = torch.empty((n, dim), device=y2d.device, dtype=y2d.dtype)
    key = torch.empty((n, rank), device=y2d.device, dtype=y2d.dtype)
    inv = torch.empty((n, heads) if key_norm else (0,), device=y2d.device, dtype=torch.float32)
    rc = lib.attnres_keyed_split_forward(ctypes.byref(d), _ptr(out), _ptr(key), _fptr(inv) if key_norm else None,
                                         _stream(y2d.device))
    _check(rc, "keyed split forward")
    return out, key, inv


def keyed_split_backward(y2d, n: int, P: int, dim: int, rank: int, heads: int, key_norm: bool, grad_out, grad_key,
                         inv, dtype, device):
    """Gradient of y, dense [n, P].  y2d (the forward's projection) is read only for the key norm."""
    lib = load()
    if y2d is not None:
        d = keyed_split_desc(dtype, n, P, y2d.stride(0) if n > 1 else P, y2d.data_ptr() if n else None, dim, rank,
                             heads, key_norm)
    else:
        d = keyed_split_desc(dtype, n, P, P, None, dim, rank, heads, key_norm)
    gy = torch.empty((n, P), device=device, dtype=dtype)
    rc = lib.attnres_keyed_split_backward(ctypes.byref(d), _ptr(grad_out), _ptr(grad_key),
                                          _fptr(inv) if key_norm else None, _ptr(gy), _stream(device))
    _check(rc, "keyed split backward")
    return gy


def block_accum_desc(y2d, dim: int, rank: int, heads: int, key_norm: bool, partial_value, partial_key,
                     complete: bool, value_norm: bool, scale_key: bool, scale_value: float, scale_tensor):
    """Descriptor of one block accumulation over a projection y [n_tok, proj_cols]; partial rows dense."""
    n, P = y2d.size(0), y2d.size(1)
    d = BlockAccumDesc()
    d.split = keyed_split_desc(y2d.dtype, n, P, y2d.stride(0) if n > 1 else P, y2d.data_ptr() if n else None, dim,
                               rank, heads, key_norm)
    d.complete = int(bool(complete))
    d.partial_value = partial_value.data_ptr() if partial_value is not None else None
    d.partial_key = partial_key.data_ptr() if partial_key is not None else None
    d.value_norm = int(bool(value_norm))
    d.scale_key = int(bool(scale_key))
    d.value_scale = float(scale_value)
    d.value_scale_dev = _fptr(scale_tensor)
    return d


def block_accum_forward(d: BlockAccumDesc, device, dtype, dim: int, rank: int, heads: int, key_norm: bool,
                        value_norm: bool):
    """(value [n, dim], key [n, rank], key_inv_rms [n, heads] | [0], value_inv_rms [n] | [0])."""
    lib = load()
    n = d.split.n_tok
    value = torch.empty((n, dim), device=device, dtype=dtype)
    key = torch.empty((n, rank), device=device, dtype=dtype)
    kinv = torch.empty((n, heads) if key_norm else (0,), device=device, dtype=torch.float32)
    vinv = torch.empty((n,) if value_norm else (0,), device=device, dtype=torch.float32)
    rc = lib.attnres_block_accum_forward(ctypes.byref(d), _ptr(value), _ptr(key), _fptr(kinv) if key_norm else None,
                                         _fptr(vinv) if value_norm else None, _stream(device))
    _check(rc, "block accumulation forward")
    return value, key, kinv, vinv


def block_accum_backward(d: BlockAccumDesc, device, dtype, grad_value, grad_key, kinv, vinv, want_dpk: bool,
                         want_dscale: bool):
    """(grad_projected [n, proj_cols], grad_partial_key [n, rank] | None, grad_scale fp32 [1] | None).
    grad_value may be a row-strided [n, dim] view."""
    lib = load()
    n, P = d.split.n_tok, d.split.proj_cols
    gy = torch.empty((n, P), device=device, dtype=dtype)
    dpk = torch.empty((n, d.split.rank), device=device, dtype=dtype) if want_dpk else None
    ds = torch.empty((1,), device=device, dtype=torch.float32) if want_dscale else None
    ws_bytes = lib.attnres_block_accum_backward_workspace_size(ctypes.byref(d)) if want_dscale else 0
    ws = torch.empty((max(1, ws_bytes),), device=device, dtype=torch.uint8) if ws_bytes else None
    rc = lib.attnres_block_accum_backward(
        ctypes.byref(d), _ptr(grad_value), grad_value.stride(0) if grad_value is not None else 0, _ptr(grad_key),
        _fptr(kinv) if kinv is not None and kinv.numel() else None, _fptr(vinv) if vinv is not None and vinv.numel() else None,
        _ptr(gy), _ptr(dpk), _fptr(ds), _ptr(ws), ws_bytes, _stream(device))
    _check(rc, "block accumulation backward")
    return gy, dpk, ds


def accum_read_desc(accum: BlockAccumDesc, read: Phase2) -> AccumReadDesc:
    d = AccumReadDesc()
    d.accum = accum
    d.read = read.c
    return d


def accum_read_forward(d: AccumReadDesc, value, key, kinv, out, device):
    """Block accumulation fused with the next merge: writes the grown block into value [n, dim] / key
    [n, rank], the key's 1/rms into kinv (with key norm) and the read into out [n, dim]."""
    lib = load()
    rc = lib.attnres_accum_read_forward(ctypes.byref(d), _ptr(value), _ptr(key), _fptr(kinv) if kinv.numel() else None,
                                        _ptr(out), _stream(device))
    _check(rc, "accumulate-and-read forward")


def accum_read_backward(d: AccumReadDesc, device, dtype, grad_out, grad_value, grad_key, kinv, want_dquery,
                        query_shape, query_row, want_dbias, want_dscale, want_dpk_old):
    """(grad_projected [n, proj_cols], grad_partial_key [n, rank] | None, dquery | None, dinter, dlse,
    dbias | None, dscale | None).  grad_value may be a row-strided [n, dim] view, grad_key dense."""
    lib = load()
    n, D, R, P = d.read.n_tok, d.read.dim, d.read.rank, d.accum.split.proj_cols
    gy = torch.empty((n, P), device=device, dtype=dtype)
    dpk = torch.empty((n, R), device=device, dtype=dtype) if want_dpk_old else None
    dq = torch.empty(query_shape, device=device, dtype=dtype) if want_dquery else None
    di = torch.empty((n, D), device=device, dtype=dtype)
    dl = torch.empty((n,), device=device, dtype=torch.float32)
    db = torch.empty((1,), device=device, dtype=torch.float32) if want_dbias else None
    ds = torch.empty((1,), device=device, dtype=torch.float32) if want_dscale else None
    g = Phase2Grads()
    g.grad_out = grad_out.data_ptr()
    g.dquery = dq.data_ptr() if dq is not None else None
    g.dinterblock_output = di.data_ptr()
    g.dinterblock_lse = _fptr(dl)
    g.dlogit_bias = _fptr(db)
    g.dvalue_scale = _fptr(ds)
    if dq is not None and query_row is not None:
        g.dquery_rows = int(query_shape[0])
        g.dquery_row = int(query_row)
    ws_bytes = lib.attnres_phase2_backward_workspace_size(ctypes.byref(d.read))
    ws = torch.empty((max(int(ws_bytes), 1),), device=device, dtype=torch.uint8)
    g.workspace = ws.data_ptr()
    g.workspace_bytes = int(ws_bytes)
    gv_stride = grad_value.stride(0) if grad_value is not None else D
    rc = lib.attnres_accum_read_backward(ctypes.byref(d), ctypes.byref(g), _ptr(grad_value), gv_stride,
                                         _ptr(grad_key),
                                         _fptr(kinv) if kinv is not None and kinv.numel() else None, _ptr(gy),
                                         _ptr(dpk), _stream(device))
    _check(rc, "accumulate-and-read backward")
    return gy, dpk, dq, di, dl, db, ds


# ---------------------------------------------------------------------------
# value-derived keys (rms-norm around the key projection GEMM)
# ---------------------------------------------------------------------------

class ValueKey:
    """Descriptor of the rms-norm of N value sources [B, T, D] (last dim contiguous)."""

    def __init__(self, values, eps=FLT_EPSILON):
        n = len(values)
        v0 = values[0]
        self._tensors = list(values)
        self.n_src = n
        self.n_tok = v0.size(0) * v0.size(1)
        self.D = v0.size(-1)
        self._vals = (c_void_p * n)(*[t.data_ptr() for t in values])
        self._vstr = (c_int64 * n)(*[t.stride(1) for t in values])
        d = ValueKeyDesc()
        d.n_src = n
        d.dtype = DTYPE_CODE[v0.dtype]
        d.n_tok = self.n_tok
        d.dim = self.D
        d.norm_eps = float(eps)
        d.values = self._vals
        d.value_row_stride = self._vstr
        self.c = d


def value_norm_forward(d: ValueKey, device, dtype):
    """(normed [N * n_tok, D] dense, inv_rms [N, n_tok] fp32)."""
    lib = load()
    normed = torch.empty((d.n_src * d.n_tok, d.D), device=device, dtype=dtype)
    inv = torch.empty((d.n_src, d.n_tok), device=device, dtype=torch.float32)
    rc = lib.attnres_value_norm_forward(ctypes.byref(d.c), _ptr(normed), _fptr(inv), _stream(device))
    _check(rc, "value norm forward")
    return normed, inv


def value_norm_backward(d: ValueKey, device, dtype, grad_normed, inv, lead):
    """The values' gradients (N tensors lead + (D,)) from the normed rows' gradient [N * n_tok, D]."""
    lib = load()
    dvals = _row_blocks(d.n_src, d.n_tok, d.D, device, dtype, True, lead)
    arr = (c_void_p * d.n_src)(*[t.data_ptr() for t in dvals])
    rc = lib.attnres_value_norm_backward(ctypes.byref(d.c), _ptr(grad_normed.contiguous()), _fptr(inv), arr,
                                         _stream(device))
    _check(rc, "value norm backward")
    return dvals
