"""Shared test configuration.

* Registers the ``gpu`` marker: tests that launch HIP kernels.  The CPU suite
  runs ``-m "not gpu"``; the GPU suite runs ``-m gpu`` on an MI355X.
* Puts the package directory (``flash-attn-triton_amd/``) and the repo root
  (for ``oracle``) on ``sys.path``.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-attn-triton_amd")
for path in (PKG, ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test launches HIP kernels and needs an MI355X")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
