"""Shared helpers for the GPU parity tests (compare the HIP path with the CPU oracle).

Tolerances (written here once and used by every GPU test):

* fp32: normwise relative error ``max|a - e| <= 1e-5 * max|e|`` (elementwise
  relative error is meaningless for near-zero entries of a sum).
* bf16 / fp16: ``mean|a - e| <= 1e-3`` and, element by element,
  ``|a - e| <= max(2e-2, ulp(e))`` where ``ulp(e)`` is one storage ulp of the
  reference value: two correctly rounded results of computations that differ
  only in fp32 summation order can land one ulp apart, and for |e| >= 4 a bf16
  ulp (>= 0.03) already exceeds 2e-2.  Every element beyond the flat 2e-2
  bound must therefore be a single-ulp difference at a magnitude where one ulp
  exceeds 2e-2 (|e| >= 4 for bf16, >= 32 for fp16); how many there are is
  recorded per comparison (``FLAT_REPORT``, printed at the end of the run).
  For gradients that are sums over all tokens (static query, per-site gate,
  bias) the bounds are applied relative to the reference magnitude
  ``max(1, max|e|)``.
* softmax weights sum to 1 within 1e-6.

Comparisons run on the GPU when the result is there (the reference is moved
to it): full-size configurations compare hundreds of millions of elements.
"""

import os

import torch

DEV = "cuda"

# (name, dtype, elements, elements beyond the flat bound, smallest |e| among them)
FLAT_REPORT = []


def err(a, e):
    d = (a.detach().float().cpu() - e.detach().float().cpu()).abs()
    return float(d.max()) if d.numel() else 0.0, float(d.mean()) if d.numel() else 0.0


def assert_close(a, e, dtype, name="", reduced=False):
    dev = a.device if a.is_cuda else torch.device("cpu")
    a = a.detach().to(dev).float()
    e = e.detach().to(dev).float()
    assert a.shape == e.shape, (name, a.shape, e.shape)
    assert bool(torch.isfinite(a).all()), f"{name}: non-finite values"
    if e.numel() == 0:
        return
    d = (a - e).abs()
    mx, mean = float(d.max()), float(d.mean(dtype=torch.float64))
    emax = float(e.abs().max())
    scale = max(1.0, emax)
    if dtype == torch.float32:
        assert mx <= 1e-5 * max(emax, 1e-30) + 1e-12, f"{name}: fp32 max err {mx:.3e} vs |ref| {emax:.3e}"
        return
    s = scale if reduced else 1.0
    mant = 7 if dtype == torch.bfloat16 else 10
    _, ex = torch.frexp(e)
    ulp = torch.ldexp(torch.ones_like(e), ex - 1 - mant)  # one storage ulp of |e|
    flat = 2e-2 * s
    over = d > flat
    n_over = int(over.sum())
    if n_over:
        # beyond the flat bound only where one ulp itself exceeds it, and by one ulp at most
        bad = over & ((d > ulp) | (ulp <= flat))
        n_bad = int(bad.sum())
        if n_bad:
            i = int(torch.nonzero(bad.reshape(-1))[0])
            raise AssertionError(f"{name}: {n_bad} of {n_over} elements beyond the flat bound {flat:.3e} are not "
                                 f"single-ulp cases (first: |a-e|={float(d.reshape(-1)[i]):.4e}, "
                                 f"e={float(e.reshape(-1)[i]):.4e}, ulp={float(ulp.reshape(-1)[i]):.4e})")
        min_e = float(e.abs()[over].min())
    else:
        min_e = None
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0].split("::")[-1]
    FLAT_REPORT.append((f"{test}:{name}", str(dtype).replace("torch.", ""), e.numel(), n_over, min_e))
    assert mean <= 1e-3 * s, f"{name}: mean err {mean:.3e} (bound {1e-3 * s:.3e}, max err {mx:.3e})"


def leaf(t, device=DEV):
    return t.detach().to(device).clone().requires_grad_(True)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(g, shape, dtype, std=1.0):
    return (torch.randn(shape, generator=g) * std).to(dtype)
