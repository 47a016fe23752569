"""Shared pytest setup: the ``gpu`` marker and import paths.

``-m "not gpu"`` tests run on any CPU host; ``-m gpu`` tests need a gfx950 GPU
and the in-tree build (``python kernelgen-challenge_amd/build.py``).
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "kernelgen-challenge_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a gfx950 GPU and the built HIP extension")


@pytest.fixture(scope="session")
def gpu_sa():
    """The drop-in module with its extension loaded; fails loudly if absent."""
    import torch
    import submission
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    submission.load_extension()
    submission.set_index_check(True)
    return submission
