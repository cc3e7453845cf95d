"""Shared test setup: the `gpu` marker, the package (loaded by path) and the CPU oracle."""
import json
import os
import sys

import numpy as np
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


def stacked_faint_gaussians(k, seed=0):
    """k wide, faint (opacity 0.005-0.008), isotropic Gaussians within 0.3 of the axis of a
    camera at (0, 0, -4), at distinct depths, the farthest one on the axis. Seen on a one-tile
    8 x 8 or 16 x 16 image (k <= 1027), the tile's list holds all k of them, no pixel's
    transmittance falls below 1e-3 (so no pixel stops early) and the last record contributes:
    every record of the list is blended, also in the last, partly filled batch."""
    from tdgs_amd import host
    rng = np.random.default_rng(seed)
    mo = np.zeros((k, 4), np.float32)
    mo[:, 0:2] = rng.uniform(-0.3, 0.3, (k, 2))
    mo[:, 2] = np.linspace(-1.0, 1.0, k, dtype=np.float32) if k > 1 else 0.0
    mo[-1, 0:2] = 0.0
    op = rng.uniform(0.005, 0.008, k).astype(np.float32)
    mo[:, 3] = np.log(op / (1 - op))
    sc = np.full((k, 3), np.log(1.5), np.float32)
    rot = np.zeros((k, 4), np.float32)
    rot[:, 0] = 1.0
    sh = np.zeros((k, 3, 1), np.float32)
    sh[:, :, 0] = rng.uniform(-1.0, 1.0, (k, 3))
    return host.HostGaussians(mo, sc, rot, sh)


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
