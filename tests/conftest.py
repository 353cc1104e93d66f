"""Test configuration: registers the ``gpu`` marker and puts the repo root on sys.path.

``gpu`` tests need an MI355X (gfx950) and the built HIP library; they fail
(rather than skip) when no GPU is visible, so a GPU run can never pass
vacuously.  Run the CPU suite with ``-m "not gpu"``.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _require_gpu(request):
    if request.node.get_closest_marker("gpu") is not None:
        import torch

        if not torch.cuda.is_available():
            pytest.fail("gpu test run without a visible GPU")
        name = request.node.nodeid
        print(f"\n[gpu-test] {name}", flush=True)
    yield
