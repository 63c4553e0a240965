"""Shared pytest configuration.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU and never calls into GPU code.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (gfx950)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; skips when this machine has none."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    from hanuman_amd import _lib
    _lib.lib()  # raises if the HIP library is missing: there is no fallback
    return torch.device("cuda:0")
