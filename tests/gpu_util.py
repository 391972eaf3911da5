"""Shared helpers for the GPU parity tests (compare the HIP path with the CPU oracle).

Tolerances (written here once and used by every GPU test):

* fp32: normwise relative error ``max|a - e| <= 1e-5 * max|e|`` (elementwise
  relative error is meaningless for near-zero entries of a sum).
* bf16 / fp16: ``mean|a - e| <= 1e-3`` and, element by element,
  ``|a - e| <= max(2e-2, ulp(e))`` where ``ulp(e)`` is one storage ulp of the
  reference value: two correctly rounded results of computations that differ
  only in fp32 summation order can land one ulp apart, and for |e| > 4 a bf16
  ulp (>= 0.03) already exceeds 2e-2.  For gradients that are sums over all
  tokens (static query, per-site gate, bias) the bounds are applied relative
  to the reference magnitude ``max(1, max|e|)``.
* softmax weights sum to 1 within 1e-6.
"""

import torch

DEV = "cuda"


def err(a, e):
    d = (a.detach().float().cpu() - e.detach().float().cpu()).abs()
    return float(d.max()) if d.numel() else 0.0, float(d.mean()) if d.numel() else 0.0


def assert_close(a, e, dtype, name="", reduced=False):
    a = a.detach().float().cpu()
    e = e.detach().float().cpu()
    assert a.shape == e.shape, (name, a.shape, e.shape)
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    mx, mean = err(a, e)
    scale = max(1.0, float(e.abs().max())) if e.numel() else 1.0
    if dtype == torch.float32:
        ref = float(e.abs().max()) if e.numel() else 0.0
        assert mx <= 1e-5 * max(ref, 1e-30) + 1e-12, f"{name}: fp32 max err {mx:.3e} vs |ref| {ref:.3e}"
    else:
        s = scale if reduced else 1.0
        mant = 7 if dtype == torch.bfloat16 else 10
        _, ex = torch.frexp(e)
        ulp = torch.ldexp(torch.ones_like(e), ex - 1 - mant)  # one storage ulp of |e|
        bound = torch.clamp(ulp, min=2e-2 * s)
        over = (a - e).abs() - bound
        worst = float(over.max()) if over.numel() else 0.0
        assert worst <= 0.0, f"{name}: max err {mx:.3e} exceeds max(2e-2, 1 ulp) by {worst:.3e}"
        assert mean <= 1e-3 * s, f"{name}: mean err {mean:.3e} (bound {1e-3 * s:.3e}, max err {mx:.3e})"


def leaf(t, device=DEV):
    return t.detach().to(device).clone().requires_grad_(True)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(g, shape, dtype, std=1.0):
    return (torch.randn(shape, generator=g) * std).to(dtype)
