"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root (for ``oracle``) and the package root (for
  ``mini_vllm`` and ``benchmarks``) on ``sys.path``.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "mini-vllm-continuous-batching-lab_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libmvattn.so")
