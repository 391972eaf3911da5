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
