"""Shared test setup: the `gpu` marker, the package (loaded by path) and the CPU oracle."""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def oracle():
    import build as oracle_build  # oracle/build.py
    oracle_build.build(force=False)
    import oracle as orc
    # per-tile loops on up to 16 host threads (the GPU box's CPU share); images do not depend
    # on the thread count
    orc.set_threads(min(16, os.cpu_count() or 1))
    return orc


@pytest.fixture(scope="session")
def tdgs():
    import tdgs_amd
    return tdgs_amd


@pytest.fixture(scope="session")
def gpu():
    """The product library on cuda:0; fails loudly if HIP or the library is unavailable."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from tdgs_amd import core
    core.lib()
    return core
