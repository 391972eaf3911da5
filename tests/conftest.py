"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X; run with ``-m gpu``)
* puts the repo root (for ``oracle``) and ``lr-attnres_amd`` (for the drop-in
  ``attnres_ops`` module) on ``sys.path``
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lr-attnres_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def pytest_terminal_summary(terminalreporter):
    """How many 16-bit elements exceeded the flat 2e-2 bound (each a checked single-ulp case)."""
    try:
        from gpu_util import FLAT_REPORT
    except ImportError:
        return
    if not FLAT_REPORT:
        return
    tr = terminalreporter
    n_el = sum(r[2] for r in FLAT_REPORT)
    n_over = sum(r[3] for r in FLAT_REPORT)
    tr.write_sep("-", "16-bit comparisons beyond the flat 2e-2 bound (all single-ulp, |e| where one ulp > 2e-2)")
    tr.write_line(f"{len(FLAT_REPORT)} comparisons, {n_el} elements, {n_over} beyond the flat bound")
    for name, dt, n, k, min_e in sorted(FLAT_REPORT, key=lambda r: -r[3])[:12]:
        if k:
            tr.write_line(f"  {name} ({dt}): {k} of {n}, smallest |e| {min_e:.4g}")
