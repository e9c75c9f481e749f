"""Shared pytest setup: the ``gpu`` marker and repo-root imports."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The loaded HIP library on cuda:0; fails (never skips) when a gpu test runs without it."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible GPU")
    from mtplx_amd import _lib

    return _lib.load()
