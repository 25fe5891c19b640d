"""Shared fixtures and helpers.

Markers: ``gpu`` tests need a ROCm GPU and the built HIP library; they are
skipped when no GPU is visible and fail (not skip) when the GPU is there but
the library is missing. Everything else runs on the CPU.
"""
import glob
import json
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and libsilogic_hip.so")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


def random_bits(*shape):
    return (torch.rand(*shape) > 0.5).float()


class Fixture:
    """One ``tests/golden/tiny_*.npz`` (written by make_golden.py)."""

    def __init__(self, path):
        z = np.load(path, allow_pickle=False)
        self.name = os.path.basename(path)[5:-4]
        self.meta = json.loads(bytes(z["meta"]).decode())
        self.spec = (self.meta["ctor"], self.meta["args"])
        self.sd = {k[3:]: torch.from_numpy(z[k].copy()) for k in z.files if k.startswith("sd/")}
        self.arrays = {k: torch.from_numpy(z[k].copy()) for k in z.files
                       if not k.startswith("sd/") and k != "meta"}
        self.x = self.arrays["x"]
        self.kind = self.meta["kind"]

    def __repr__(self):
        return f"Fixture({self.name})"


FIXTURE_PATHS = sorted(glob.glob(os.path.join(GOLDEN, "tiny_*.npz")))
FIXTURE_IDS = [os.path.basename(p)[5:-4] for p in FIXTURE_PATHS]


def load_fixture(name):
    return Fixture(os.path.join(GOLDEN, f"tiny_{name}.npz"))


@pytest.fixture(params=FIXTURE_PATHS, ids=FIXTURE_IDS)
def fixture(request):
    return Fixture(request.param)


def build_product(spec):
    """The silogic_amd model for ``spec`` with the reference's seeding."""
    import silogic_amd
    ctor, args = spec
    torch.manual_seed(0)
    return getattr(silogic_amd, ctor)(seed=0, **args)
