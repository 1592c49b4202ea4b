"""Shared pytest configuration.

Markers
-------
gpu : needs an MI355X (gfx950) and the built HIP library.  The CPU suite runs
      with ``-m "not gpu"``; GPU tests fail loudly (never skip silently) when the
      library is missing on a GPU box.
"""

from __future__ import annotations

import importlib
import os
import sys
import zlib

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG_NAME = "simple-inference-autoresearch_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def load_pkg():
    """Import the product package (its directory name has hyphens)."""
    return importlib.import_module(PKG_NAME)


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def gpu_pkg():
    """The package with the HIP library loaded on a visible GPU."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    p = load_pkg()
    p.require_library()
    return p


@pytest.fixture(autouse=True)
def _seed_global_generators(request):
    """Seed torch's default generators (host and every GPU) per test from its node id.

    Inputs drawn without an explicit generator are then reproducible from the
    test's name alone; the seed is printed so a failure log names it.
    """
    import torch

    seed = zlib.crc32(request.node.nodeid.encode()) & 0x7FFFFFFF
    torch.manual_seed(seed)   # also seeds every visible GPU's default generator
    print(f"[seed] {request.node.nodeid}: torch.manual_seed({seed})", flush=True)
    yield
