"""CPU checks of the boundary: the C-ABI library loads, exports every symbol the
header declares, lays out its structs as ctypes does, and validates arguments
on the host (no kernel is launched here); the Python drop-in fails loudly
without a GPU and keeps the reference's argument errors."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "attnres_hip.h")

import _attnres_hip as H  # noqa: E402
import attnres_ops as ops  # noqa: E402


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(attnres_[a-z0-9_]+)\s*\(", text)))


needs_lib = pytest.mark.skipif(not os.path.exists(H.LIB_PATH), reason="libattnres_hip.so not built")


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(H.LIB_PATH)
    names = _declared_functions()
    assert names == sorted(["attnres_abi_version", "attnres_last_error", "attnres_read_backward",
                            "attnres_read_backward_workspace_size", "attnres_read_forward",
                            "attnres_phase1_forward", "attnres_phase1_backward", "attnres_phase2_forward",
                            "attnres_phase2_backward", "attnres_phase2_backward_workspace_size",
                            "attnres_keyed_split_forward", "attnres_keyed_split_backward",
                            "attnres_keyed_logits_forward", "attnres_keyed_logits_backward",
                            "attnres_keyed_logits_backward_workspace_size", "attnres_kernel_timing",
                            "attnres_kernel_times", "attnres_read_backward_noalloc", "attnres_test_phase2_block_layout",
                            "attnres_value_norm_forward", "attnres_value_norm_backward",
                            "attnres_block_accum_forward", "attnres_block_accum_backward",
                            "attnres_block_accum_backward_workspace_size", "attnres_phase1_backward_sites",
                            "attnres_site_logits_forward", "attnres_site_logits_backward",
                            "attnres_accum_read_forward", "attnres_accum_read_backward"])
    for n in names:
        assert hasattr(lib, n), n
    nm = subprocess.run(["nm", "-D", "--defined-only", H.LIB_PATH], capture_output=True, text=True).stdout
    for n in names:
        assert re.search(rf"\bT {n}\b", nm), f"{n} not exported"


@needs_lib
def test_abi_version_and_error_reporting():
    lib = H.load()
    assert lib.attnres_abi_version() == 9
    rc = lib.attnres_read_forward(None, None, None, None, None, None)
    assert rc == -1
    assert b"desc is NULL" in lib.attnres_last_error()
    assert lib.attnres_phase1_forward(None, None, None, None, None, None) == -1
    assert lib.attnres_phase2_forward(None, None, None) == -1
    assert b"desc is NULL" in lib.attnres_last_error()
    assert lib.attnres_keyed_split_forward(None, None, None, None, None) == -1
    assert lib.attnres_keyed_split_backward(None, None, None, None, None, None) == -1


STRUCTS = ((H.ReadDesc, "attnres_read_desc"), (H.ReadGrads, "attnres_read_grads"),
           (H.Phase1Desc, "attnres_phase1_desc"), (H.Phase2Desc, "attnres_phase2_desc"),
           (H.Phase2Grads, "attnres_phase2_grads"), (H.KeyedSplitDesc, "attnres_keyed_split_desc"),
           (H.BlockAccumDesc, "attnres_block_accum_desc"), (H.ValueKeyDesc, "attnres_value_key_desc"),
           (H.AccumReadDesc, "attnres_accum_read_desc"))


def _c_layout():
    """offsetof / sizeof of the C-ABI structs, from a C compile of the header."""
    src = r'''
#include <stdio.h>
#include <stddef.h>
#include "attnres_hip.h"
#define P(s, f) printf(#s " " #f " %zu\n", offsetof(s, f));
int main(void) {
''' + "".join(f'  printf("{n} sizeof %zu\\n", sizeof({n}));\n' for _, n in STRUCTS) + \
        "".join(f"  P({n}, {f})\n" for cls, n in STRUCTS for f, _ in cls._fields_) + "  return 0;\n}\n"
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "p.c")
        exe = os.path.join(d, "p")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    res = {}
    for line in out.strip().splitlines():
        s, f, v = line.split()
        res[(s, f)] = int(v)
    return res


def test_ctypes_structs_match_the_header():
    lay = _c_layout()
    for cls, name in STRUCTS:
        assert ctypes.sizeof(cls) == lay[(name, "sizeof")]
        for f, _ in cls._fields_:
            assert getattr(cls, f).offset == lay[(name, f)], (name, f)


def _desc(n_src=3, n_tok=16, dim=64, rank=16, heads=2, **kw):
    vals = (ctypes.c_void_p * n_src)(*([0x1000] * n_src))
    vstr = (ctypes.c_int64 * n_src)(*([dim] * n_src))
    keys = (ctypes.c_void_p * n_src)(*([0x2000] * n_src))
    kstr = (ctypes.c_int64 * n_src)(*([rank] * n_src))
    d = H.ReadDesc()
    d.n_src, d.dtype, d.n_tok, d.dim, d.rank, d.heads = n_src, 1, n_tok, dim, rank, heads
    d.mode, d.key_norm, d.logit_scale, d.norm_eps = 0, 1, 0.25, H.FLT_EPSILON
    d.key_dtype = 1
    d.values, d.value_row_stride = vals, vstr
    if rank:
        d.keys, d.key_row_stride = keys, kstr
    d.query = 0x3000
    for k, v in kw.items():
        setattr(d, k, v)
    d._keep = (vals, vstr, keys, kstr)
    return d


@needs_lib
def test_host_validation_rejects_bad_descriptions_without_launching():
    lib = H.load()
    cases = [
        (dict(n_src=0), -2, b"n_src"),
        (dict(n_src=65), -2, b"n_src"),
        (dict(heads=3), -1, b"heads"),
        (dict(rank=0, heads=2), -1, b"heads == 1"),
        (dict(dtype=7), -1, b"dtype"),
        (dict(query=None), -1, b"query"),
        (dict(key_dtype=9), -1, b"key dtype"),
        (dict(key_dtype=0, gate=0x5000, query_dyn=0x6000, query_dyn_row_stride=16, gate_act=2), -2,
         b"gated query needs keys in the value dtype"),
        (dict(rank=0, heads=1, static_keys=0x7000), -1, b"static_keys apply to LR reads only"),
    ]
    for kw, code, msg in cases:
        n_src = kw.pop("n_src", 3)
        d = _desc(n_src=max(1, min(n_src, 64)), **{k: v for k, v in kw.items() if k not in ("dtype",)})
        d.n_src = n_src
        if "dtype" in kw:
            d.dtype = kw["dtype"]
        rc = lib.attnres_read_forward(ctypes.byref(d), ctypes.c_void_p(0x4000), None, None, None, None)
        assert rc == code, (kw, rc, lib.attnres_last_error())
        assert msg in lib.attnres_last_error(), lib.attnres_last_error()


@needs_lib
def test_workspace_size_is_a_host_computation():
    lib = H.load()
    d = _desc(n_src=13, n_tok=16384, dim=1024, rank=64, heads=4)
    # 4096 workgroups x (64 query slots) floats; no bias
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == 4096 * 64 * 4
    bias = (ctypes.c_float * 13)()
    d.logit_bias = ctypes.cast(bias, ctypes.POINTER(ctypes.c_float))
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == 4096 * (64 + 13) * 4
    d.n_tok = 5
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == 5 * (64 + 13) * 4
    d.n_tok = 0
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == 0
    # static keys: their column sums follow the partial rows (on a 256-byte
    # boundary), one fp32 row of rank per source and chunk of >= 128 tokens (<= 128 chunks)
    d = _desc(n_src=17, n_tok=16384, dim=2048, rank=128, heads=8, static_keys=0x7000)
    rows = 4096 * 128 * 4
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == rows + 17 * 128 * 128 * 4
    d.n_tok = 1000
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == 1000 * 128 * 4 + 17 * 8 * 128 * 4
    d.n_tok = 3
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == (3 * 128 * 4 + 255) // 256 * 256 + 17 * 128 * 4


@needs_lib
def test_static_key_gradient_needs_static_keys():
    lib = H.load()
    d = _desc()
    g = H.ReadGrads()
    dv = (ctypes.c_void_p * 3)(*([0x8000] * 3))
    g.grad_out, g.weights, g.dvalues, g.dkeys = 0x9000, ctypes.cast(ctypes.c_void_p(0xa000), ctypes.POINTER(ctypes.c_float)), dv, dv
    g.dstatic_keys = 0xb000
    assert lib.attnres_read_backward(ctypes.byref(d), ctypes.byref(g), None) == -1
    assert b"dstatic_keys without static_keys" in lib.attnres_last_error()


@needs_lib
def test_static_key_workspace_is_checked_before_any_launch():
    """A workspace sized without the static keys' column sums is refused on the
    host, before the backward launches anything (every output untouched)."""
    lib = H.load()
    d = _desc(n_src=13, n_tok=16384, dim=1024, rank=64, heads=4, static_keys=0x7000)
    need = lib.attnres_read_backward_workspace_size(ctypes.byref(d))
    rows = 4096 * 64 * 4
    assert need > rows
    g = H.ReadGrads()
    dv = (ctypes.c_void_p * 13)(*([0x8000] * 13))
    g.grad_out, g.weights, g.dvalues, g.dkeys = 0x9000, ctypes.cast(ctypes.c_void_p(0xa000), ctypes.POINTER(ctypes.c_float)), dv, dv
    g.dquery = 0xc000
    g.dstatic_keys = 0xb000
    g.workspace, g.workspace_bytes = 0xd000, rows  # the partial rows only
    assert lib.attnres_read_backward(ctypes.byref(d), ctypes.byref(g), None) == -4
    assert f"workspace of {need} bytes needed, got {rows}".encode() in lib.attnres_last_error()


@needs_lib
def test_noalloc_backward_refuses_descriptions_beyond_its_scratch():
    """The no-allocation backward checks the partial-sum size against its fixed
    per-device array before it looks the array up or launches anything."""
    lib = H.load()
    d = _desc(n_src=64, n_tok=1 << 20, dim=8192, rank=0, heads=1)  # base read: 64 x 8192 fp32 partials per group
    need = lib.attnres_read_backward_workspace_size(ctypes.byref(d))
    assert need > H.NOALLOC_SCRATCH_BYTES
    g = H.ReadGrads()
    dv = (ctypes.c_void_p * 64)(*([0x8000] * 64))
    g.grad_out, g.weights, g.dvalues = 0x9000, ctypes.cast(ctypes.c_void_p(0xa000), ctypes.POINTER(ctypes.c_float)), dv
    g.dquery = 0xc000
    assert lib.attnres_read_backward_noalloc(ctypes.byref(d), ctypes.byref(g), None) == -4
    err = lib.attnres_last_error()
    assert f"needs {need} bytes of partial sums".encode() in err and b"holds 33554432" in err


def test_static_keys_shape_is_checked_on_the_host():
    vs = [torch.randn(1, 2, 8) for _ in range(3)]
    ks = [torch.randn(1, 2, 4) for _ in range(3)]
    with pytest.raises(RuntimeError, match="static_keys must be"):
        ops.lrid_attention_residual_read(vs, ks, torch.zeros(1, 4), 1, 1.0, True, static_keys=torch.zeros(3, 5))
    assert ops._static_keys([torch.ones(4)] * 3, 3, 4, torch.bfloat16, "x").shape == (3, 4)


def test_product_path_fails_loudly_on_cpu_tensors():
    vs = [torch.randn(1, 2, 8) for _ in range(3)]
    ks = [torch.randn(1, 2, 4) for _ in range(3)]
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lrid_attention_residual_read(vs, ks, torch.zeros(1, 4), 1, 1.0, True)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention_residual_read(vs, torch.zeros(8), True)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention_residual_average_read(vs)


def test_reference_argument_errors_are_kept():
    vs = [torch.randn(1, 2, 8) for _ in range(3)]
    with pytest.raises(RuntimeError, match="mutually exclusive"):
        ops._source_logit_bias([1, 2, 3], [0.0, 0.0, 0.0], 3, "cpu")
    with pytest.raises(RuntimeError, match="length must match"):
        ops._source_logit_bias([1, 2], None, 3, "cpu")
    with pytest.raises(RuntimeError, match="must be positive"):
        ops._source_logit_bias([1, 0, 2], None, 3, "cpu")
    with pytest.raises(RuntimeError, match="value sources"):
        ops.lrid_attention_residual_read(vs, vs[:2], torch.zeros(1, 8), 1, 1.0, True)
    with pytest.raises(RuntimeError, match="must divide"):
        ops.lrid_attention_residual_read(vs, [torch.randn(1, 2, 6)] * 3, torch.zeros(6), 4, 1.0, True)
    # single source is the identity, as in the reference (no GPU needed)
    assert ops.lrid_attention_residual_read(vs[:1], [torch.randn(1, 2, 4)], torch.zeros(1, 4), 1, 1.0, True) is vs[0]
    assert ops.attention_residual_read(vs[:1], torch.zeros(8), True) is vs[0]
    torch.testing.assert_close(ops.attention_residual_read(vs[:1], torch.zeros(8), True, normalize_output=True),
                               torch.nn.functional.rms_norm(vs[0], (8,)))


def _p1desc(n_src=3, n_q=2, n_tok=16, dim=64, **kw):
    vals = (ctypes.c_void_p * n_src)(*([0x1000] * n_src))
    vstr = (ctypes.c_int64 * n_src)(*([dim] * n_src))
    d = H.Phase1Desc()
    d.n_src, d.n_q, d.dtype, d.logits_dtype, d.n_tok, d.dim = n_src, n_q, 1, 0, n_tok, dim
    d.norm_eps = H.FLT_EPSILON
    d.values, d.value_row_stride = vals, vstr
    d.logits = 0x2000
    d.logit_q_stride, d.logit_s_stride = n_src * n_tok, n_tok
    for k, v in kw.items():
        setattr(d, k, v)
    d._keep = (vals, vstr)
    return d


def _p2desc(n_tok=16, dim=64, rank=0, **kw):
    d = H.Phase2Desc()
    d.dtype, d.n_tok, d.dim, d.rank, d.merge, d.key_norm = 1, n_tok, dim, rank, 0, 1
    d.norm_eps, d.value_scale = H.FLT_EPSILON, 1.0
    d.partial_value, d.partial_value_row_stride = 0x1000, dim
    d.interblock_output, d.interblock_row_stride = 0x2000, dim
    d.interblock_lse = ctypes.cast(ctypes.c_void_p(0x3000), ctypes.POINTER(ctypes.c_float))
    d.query = 0x4000
    if rank:
        d.partial_key, d.partial_key_row_stride = 0x5000, rank
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@needs_lib
def test_phase_host_validation_rejects_bad_descriptions_without_launching():
    lib = H.load()
    out = ctypes.c_void_p(0x6000)
    lse = ctypes.cast(ctypes.c_void_p(0x7000), ctypes.POINTER(ctypes.c_float))
    cases1 = [
        (dict(n_q=0), -2, b"n_q"),
        (dict(n_q=17), -2, b"n_q"),
        (dict(dim=5000), -2, b"dim"),
        (dict(logits=None), -1, b"logits"),
        (dict(logit_s_stride=8), -1, b"overlap"),
        (dict(logits_dtype=9), -1, b"dtype"),
    ]
    for kw, code, msg in cases1:
        d = _p1desc(**kw)
        rc = lib.attnres_phase1_forward(ctypes.byref(d), out, None, lse, None, None)
        assert rc == code, (kw, rc, lib.attnres_last_error())
        assert msg in lib.attnres_last_error(), lib.attnres_last_error()
    cases2 = [
        (dict(merge=5), -1, b"merge"),
        (dict(rank=4096), -2, b"rank"),
        (dict(logit_given=1), -1, b"partial_logit"),
        (dict(rank=16, partial_key=None), -1, b"partial_key"),
        (dict(query=None), -1, b"query"),
        (dict(partial_value_row_stride=8), -1, b"stride"),
    ]
    for kw, code, msg in cases2:
        d = _p2desc(**kw)
        rc = lib.attnres_phase2_forward(ctypes.byref(d), out, None)
        assert rc == code, (kw, rc, lib.attnres_last_error())
        assert msg in lib.attnres_last_error(), lib.attnres_last_error()


@needs_lib
def test_phase2_workspace_size_is_a_host_computation():
    lib = H.load()
    d = _p2desc(n_tok=16384, dim=768)
    # 4096 workgroups x (768 query + 1 bias + 1 value-scale slots), rows padded to tiles of 16 slots
    assert lib.attnres_phase2_backward_workspace_size(ctypes.byref(d)) == 4096 * 784 * 4
    d = _p2desc(n_tok=100, dim=768, rank=64, scale_key=1)
    # LR: 64 query slots, bias, value- and key-scale slots (67, padded to 80)
    assert lib.attnres_phase2_backward_workspace_size(ctypes.byref(d)) == 100 * 80 * 4
    d = _p2desc(n_tok=0, dim=768)
    assert lib.attnres_phase2_backward_workspace_size(ctypes.byref(d)) == 0


def test_phase_ops_fail_loudly_on_cpu_tensors():
    vs = [torch.randn(1, 2, 8) for _ in range(3)]
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention_residual_phase1_from_logits(vs, torch.randn(2, 3, 1, 2))
    p = torch.randn(1, 2, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention_residual_phase2(p, torch.randn(8), p.clone(), torch.zeros(1, 2), True)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lrid_attention_residual_phase2_torch(p, torch.randn(1, 2, 4), torch.randn(1, 4), p.clone(),
                                                 torch.zeros(1, 2), 0.5, True)
    with pytest.raises(RuntimeError, match=r"logits must be \[Q, 3"):
        ops.attention_residual_phase1_from_logits(vs, torch.randn(2, 4, 1, 2))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention_residual_phase1(vs, torch.randn(2, 8), True)
    with pytest.raises(RuntimeError, match=r"queries must be \[Q, 8\]"):
        ops.attention_residual_phase1(vs, torch.randn(2, 7), True)


def _kldesc(n_src=3, n_q=2, n_tok=1000, dim=768, key_norm=1):
    d = H.KeyedLogitsDesc()
    d.n_src, d.n_q, d.dtype, d.n_tok, d.dim, d.key_norm = n_src, n_q, 1, n_tok, dim, key_norm
    d.norm_eps = 1e-6
    d._vals = (ctypes.c_void_p * n_src)(*([0x1000] * n_src))
    d._str = (ctypes.c_int64 * n_src)(*([dim] * n_src))
    d.values = d._vals
    d.value_row_stride = d._str
    d.queries = 0x2000
    return d


@needs_lib
def test_keyed_logits_workspace_and_validation_are_host_computations():
    lib = H.load()
    # query-gradient partial rows: min(n_tok, 128) x Q x D floats
    assert lib.attnres_keyed_logits_backward_workspace_size(ctypes.byref(_kldesc())) == 128 * 2 * 768 * 4
    assert lib.attnres_keyed_logits_backward_workspace_size(ctypes.byref(_kldesc(n_tok=5))) == 5 * 2 * 768 * 4
    assert lib.attnres_keyed_logits_backward_workspace_size(ctypes.byref(_kldesc(n_tok=0))) == 0
    # invalid descriptions: no workspace, and the entry points refuse them before any launch
    for bad in (_kldesc(n_q=17), _kldesc(n_src=0), _kldesc(dim=4097)):
        assert lib.attnres_keyed_logits_backward_workspace_size(ctypes.byref(bad)) == 0
        assert lib.attnres_keyed_logits_forward(ctypes.byref(bad), ctypes.c_void_p(0x3000), None, None) != 0
    rc = lib.attnres_keyed_logits_forward(ctypes.byref(_kldesc()), None, None, None)
    assert rc != 0 and b"logits" in lib.attnres_last_error()


def _ksdesc(**kw):
    d = H.keyed_split_desc(torch.bfloat16, 16, 832, 832, 0x1000, 768, 64, 1, True)
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@needs_lib
def test_keyed_split_host_validation_rejects_bad_descriptions_without_launching():
    lib = H.load()
    out, key = ctypes.c_void_p(0x6000), ctypes.c_void_p(0x7000)
    inv = ctypes.cast(ctypes.c_void_p(0x8000), ctypes.POINTER(ctypes.c_float))
    cases = [
        (dict(rank=512, proj_cols=1280, row_stride=1280), -2, b"rank"),
        (dict(heads=3), -1, b"heads"),
        (dict(heads=0), -1, b"heads"),
        (dict(heads=2, rank=96, proj_cols=864, row_stride=864), -2, b"head width"),
        (dict(proj_cols=800), -1, b"proj_cols"),
        (dict(row_stride=800), -1, b"row_stride"),
        (dict(projected=None), -1, b"projected"),
        (dict(dtype=7), -1, b"dtype"),
    ]
    for kw, code, msg in cases:
        d = _ksdesc(**kw)
        rc = lib.attnres_keyed_split_forward(ctypes.byref(d), out, key, inv, None)
        assert rc == code, (kw, rc, lib.attnres_last_error())
        assert msg in lib.attnres_last_error(), lib.attnres_last_error()
    d = _ksdesc()
    assert lib.attnres_keyed_split_forward(ctypes.byref(d), out, key, None, None) == -1
    assert b"key_inv_rms" in lib.attnres_last_error()
    assert lib.attnres_keyed_split_backward(ctypes.byref(d), None, key, None, None, None) == -1
    assert b"grad_projected" in lib.attnres_last_error()
    d = _ksdesc(n_tok=0)
    assert lib.attnres_keyed_split_forward(ctypes.byref(d), None, None, None, None) == 0


def test_keyed_split_fails_loudly_on_cpu_tensors():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lrid_fused_projection_split(torch.randn(2, 3, 80), 64, 16)
    with pytest.raises(RuntimeError, match="columns"):
        ops.lrid_fused_projection_split(torch.randn(2, 3, 70), 64, 16)



@needs_lib
def test_kernel_times_need_timing_enabled():
    # host-only paths: disabling when off and reading times when off make no HIP call
    lib = H.load()
    assert lib.attnres_kernel_timing(0) == 0
    buf = (ctypes.c_float * 4)()
    assert lib.attnres_kernel_times(buf, 4) == -1
    assert b"not enabled" in lib.attnres_last_error()


def test_lrid_list_dims_within_triton_limits_keeps_the_reference_answers():
    """tests/test_attnres_ops.py:515-520 of the reference, against the drop-in."""
    values = [torch.empty(1, 1, 1024), torch.empty(1, 1, 1024)]
    keys = [torch.empty(1, 1, 512), torch.empty(1, 1, 512)]
    assert not ops._lrid_list_dims_within_triton_limits(values, keys, num_heads=1)
    assert ops._lrid_list_dims_within_triton_limits(values, keys, num_heads=2)
    assert ops._lrid_list_head_dims(values, keys, 3) is None
    assert ops._lrid_list_head_dims(values, keys, "x") is None
    assert ops._lrid_list_head_dims(values, keys, 4) == (256, 128)


def test_mixed_dtype_sources_are_promoted_like_torch_stack():
    a = torch.randn(1, 2, 8)
    b = torch.randn(1, 2, 8).to(torch.bfloat16)
    c = torch.randn(1, 2, 8).to(torch.float16)
    out = ops._promote([b, a, c])
    assert [t.dtype for t in out] == [torch.stack([b, a, c]).dtype] * 3
    assert out[1] is a  # sources already in the common dtype are not copied
    assert ops._promote([b, b])[0] is b
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.attention_residual_read([a, b], torch.zeros(8), True)
    with pytest.raises(RuntimeError, match="not supported"):
        ops.attention_residual_read([a, a.double()], torch.zeros(8), True)


@needs_lib
def test_noalloc_backward_rejects_needs_beyond_its_scratch_on_the_host():
    """A base read with 4096 query slots over 4096 workgroups needs 64 MiB of
    partial sums, twice the fixed array: refused before anything is launched."""
    lib = H.load()
    d = _desc(n_src=8, n_tok=65536, dim=4096, rank=0, heads=1)
    assert lib.attnres_read_backward_workspace_size(ctypes.byref(d)) == 4096 * 4096 * 4 > H.NOALLOC_SCRATCH_BYTES
    g = H.ReadGrads()
    assert lib.attnres_read_backward_noalloc(ctypes.byref(d), ctypes.byref(g), None) == -4
    assert b"no-allocation entry point holds 33554432" in lib.attnres_last_error()
    assert lib.attnres_read_backward_noalloc(ctypes.byref(d), None, None) == -1
    assert lib.attnres_read_backward_noalloc(None, ctypes.byref(g), None) == -1


def _badesc(**kw):
    d = H.BlockAccumDesc()
    d.split = _ksdesc()
    d.complete = 1
    d.value_scale = 0.5
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@needs_lib
def test_block_accum_host_validation_rejects_bad_descriptions_without_launching():
    lib = H.load()
    out, key = ctypes.c_void_p(0x6000), ctypes.c_void_p(0x7000)
    scale = ctypes.cast(ctypes.c_void_p(0x9000), ctypes.POINTER(ctypes.c_float))
    cases = [
        (dict(complete=2), b"complete"),
        (dict(complete=0, value_norm=1), b"completed block source only"),
        (dict(complete=0, scale_key=1), b"completed block source only"),
        (dict(complete=0, value_scale_dev=scale), b"completed block source only"),
        (dict(value_norm=1, scale_key=1), b"value_norm"),
        (dict(value_norm=1, value_scale_dev=scale), b"value_norm"),
    ]
    for kw, msg in cases:
        d = _badesc(**kw)
        assert lib.attnres_block_accum_forward(ctypes.byref(d), out, key, None, None, None) == -1, kw
        assert msg in lib.attnres_last_error(), (kw, lib.attnres_last_error())
        assert lib.attnres_block_accum_backward_workspace_size(ctypes.byref(d)) == 0
    # the split's own checks apply
    d = _badesc()
    d.split.heads = 3
    assert lib.attnres_block_accum_forward(ctypes.byref(d), out, key, None, None, None) == -1
    assert b"heads" in lib.attnres_last_error()
    # workspace only for a learned scale's gradient, one fp32 pair per backward workgroup
    assert lib.attnres_block_accum_backward_workspace_size(ctypes.byref(_badesc())) == 0
    d = _badesc(value_scale_dev=scale)
    ws = lib.attnres_block_accum_backward_workspace_size(ctypes.byref(d))
    assert ws > 0 and ws % 8 == 0
    rc = lib.attnres_block_accum_backward(ctypes.byref(d), None, 0, None, ctypes.cast(ctypes.c_void_p(0x8000), ctypes.POINTER(ctypes.c_float)),
                                          None, ctypes.c_void_p(0xa000), None, scale, None, 0, None)
    assert rc == -4 and b"workspace" in lib.attnres_last_error()
    # the backward needs the forward's inverse rms values
    d = _badesc()
    assert lib.attnres_block_accum_backward(ctypes.byref(d), None, 0, None, None, None, ctypes.c_void_p(0xa000),
                                            None, None, None, 0, None) == -1
    assert b"key_inv_rms" in lib.attnres_last_error()
    d = _badesc(value_norm=1)
    d.split.key_norm = 0
    assert lib.attnres_block_accum_backward(ctypes.byref(d), ctypes.c_void_p(0xb000), 768, None, None, None,
                                            ctypes.c_void_p(0xa000), None, None, None, 0, None) == -1
    assert b"value_inv_rms" in lib.attnres_last_error()
    d = _badesc()
    d.split.key_norm = 0
    assert lib.attnres_block_accum_backward(ctypes.byref(d), ctypes.c_void_p(0xb000), 700, None, None, None,
                                            ctypes.c_void_p(0xa000), None, None, None, 0, None) == -1
    assert b"grad_value_row_stride" in lib.attnres_last_error()
    # nothing to do for zero tokens
    d = _badesc()
    d.split.n_tok = 0
    assert lib.attnres_block_accum_forward(ctypes.byref(d), None, None, None, None, None) == 0


def _ardesc(**kw):
    d = H.AccumReadDesc()
    d.accum = _badesc(complete=0, value_scale=1.0)
    d.read = _p2desc(n_tok=16, dim=768, rank=64)
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@needs_lib
def test_accum_read_host_validation_rejects_bad_descriptions_without_launching():
    lib = H.load()
    value, key, out = ctypes.c_void_p(0x6000), ctypes.c_void_p(0x7000), ctypes.c_void_p(0x8000)
    inv = ctypes.cast(ctypes.c_void_p(0x9000), ctypes.POINTER(ctypes.c_float))
    d = _ardesc()
    d.accum.complete = 1
    assert lib.attnres_accum_read_forward(ctypes.byref(d), value, key, inv, out, None) == -1
    assert b"complete = 0" in lib.attnres_last_error()
    d = _ardesc()
    d.read = _p2desc(n_tok=16, dim=768, rank=0)
    assert lib.attnres_accum_read_forward(ctypes.byref(d), value, key, inv, out, None) == -1
    assert b"LR merge" in lib.attnres_last_error()
    d = _ardesc()
    d.read.n_tok = 32
    assert lib.attnres_accum_read_forward(ctypes.byref(d), value, key, inv, out, None) == -1
    assert b"disagree" in lib.attnres_last_error()
    # the block accumulation's own checks apply
    d = _ardesc()
    d.accum.split.heads = 3
    assert lib.attnres_accum_read_forward(ctypes.byref(d), value, key, inv, out, None) == -1
    assert b"heads" in lib.attnres_last_error()
    # key norm needs the 1/rms output
    assert lib.attnres_accum_read_forward(ctypes.byref(_ardesc()), value, key, None, out, None) == -1
    assert b"key_inv_rms" in lib.attnres_last_error()
    # the fused kernels take one-wave 16-bit rows only: the caller composes the two calls otherwise
    d = _ardesc()
    d.accum.split = _ksdesc(rank=64, proj_cols=864, row_stride=864, dim=800)
    d.read = _p2desc(n_tok=16, dim=800, rank=64)
    assert lib.attnres_accum_read_forward(ctypes.byref(d), value, key, inv, out, None) == -2
    assert b"rank <= 256" in lib.attnres_last_error()
    # backward: grads, the projection gradient and grad_value's row stride
    d = _ardesc()
    g = H.Phase2Grads()
    assert lib.attnres_accum_read_backward(ctypes.byref(d), None, None, 768, None, inv, ctypes.c_void_p(0xa000),
                                           None, None) == -1
    assert b"grads is NULL" in lib.attnres_last_error()
    assert lib.attnres_accum_read_backward(ctypes.byref(d), ctypes.byref(g), ctypes.c_void_p(0xb000), 700, None,
                                           inv, ctypes.c_void_p(0xa000), None, None) == -1
    assert b"grad_value_row_stride" in lib.attnres_last_error()
    assert lib.attnres_accum_read_backward(ctypes.byref(d), ctypes.byref(g), None, 768, None, inv, None, None,
                                           None) == -1
    assert b"grad_projected" in lib.attnres_last_error()
    # nothing to do for zero tokens
    d = _ardesc()
    d.accum.split.n_tok = 0
    d.read.n_tok = 0
    assert lib.attnres_accum_read_forward(ctypes.byref(d), None, None, None, None, None) == 0


def test_block_accumulate_rejects_bad_calls_on_the_host():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lrid_block_accumulate(torch.randn(2, 3, 80), None, None, 64, 16)
    with pytest.raises(RuntimeError, match="columns"):
        ops.lrid_block_accumulate(torch.randn(2, 3, 70), None, None, 64, 16)
    with pytest.raises(RuntimeError, match="complete=True only"):
        ops.lrid_block_accumulate(torch.randn(2, 3, 80), None, None, 64, 16, partial_scale=0.5)
    with pytest.raises(RuntimeError, match="value_norm"):
        ops.lrid_block_accumulate(torch.randn(2, 3, 80), None, None, 64, 16, complete=True, value_norm=True,
                                  scale_key=True)


@needs_lib
def test_phase2_layout_hook_validates_and_kernel_times_need_timing():
    lib = H.load()
    assert lib.attnres_test_phase2_block_layout(2) == -1
    assert b"on must be 0 or 1" in lib.attnres_last_error()
    assert lib.attnres_test_phase2_block_layout(0) == 0
    buf = (ctypes.c_float * 4)()
    assert lib.attnres_kernel_times(buf, 4) == -1
    assert b"not enabled" in lib.attnres_last_error()


@needs_lib
def test_value_norm_host_validation():
    lib = H.load()
    vals = (ctypes.c_void_p * 2)(0x1000, 0x1000)
    vstr = (ctypes.c_int64 * 2)(2048, 2048)
    d = H.ValueKeyDesc()
    d.n_src, d.dtype, d.n_tok, d.dim, d.norm_eps = 2, 1, 8, 2048, H.FLT_EPSILON
    d.values, d.value_row_stride = vals, vstr
    inv = ctypes.cast(ctypes.c_void_p(0x3000), ctypes.POINTER(ctypes.c_float))
    assert lib.attnres_value_norm_forward(ctypes.byref(d), None, inv, None) == -1
    assert b"normed" in lib.attnres_last_error()
    d.dim = 4104
    vstr[0] = vstr[1] = 4104
    assert lib.attnres_value_norm_forward(ctypes.byref(d), ctypes.c_void_p(0x2000), inv, None) == -2
    assert b"exceeds 4096" in lib.attnres_last_error()
    d.dim = 600  # unaligned rows are held at one element per lane vector: 512 at most
    vstr[0] = vstr[1] = 601
    assert lib.attnres_value_norm_forward(ctypes.byref(d), ctypes.c_void_p(0x2000), inv, None) == -2
    assert b"unaligned" in lib.attnres_last_error()
    d.dim, d.n_src = 64, 0
    assert lib.attnres_value_norm_forward(ctypes.byref(d), ctypes.c_void_p(0x2000), inv, None) == -2
    d.n_src, d.n_tok = 2, 0
    assert lib.attnres_value_norm_backward(ctypes.byref(d), None, None, None, None) == 0


def test_value_key_projection_fails_loudly_on_cpu_tensors():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lrid_value_key_projection([torch.randn(1, 2, 8)] * 2, torch.randn(4, 8))


def test_accumulate_read_rejects_bad_calls_on_the_host():
    proj, inter, lse = torch.randn(2, 3, 288), torch.randn(2, 3, 256), torch.randn(2, 3)
    bank = torch.randn(4, 32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lrid_block_accumulate_read(proj.bfloat16(), None, None, bank.bfloat16(), inter.bfloat16(), lse, 256, 32,
                                       0.2, query_row=1)
    with pytest.raises(RuntimeError, match=r"interblock_output must be \[B, T, 256\]"):
        ops.lrid_block_accumulate_read(proj, None, None, bank, inter[0], lse, 256, 32, 0.2, query_row=1)
    with pytest.raises(RuntimeError, match=r"interblock_output must be \[B, T, 256\]"):
        ops.lrid_block_accumulate_read(proj, None, None, bank, inter[..., :128], lse, 256, 32, 0.2, query_row=1)
