import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    """Expected outputs produced by the compiled reference kernels."""
    return np.load(GOLDEN / "kernels.npz")


@pytest.fixture(scope="session")
def golden_workloads():
    return json.loads((GOLDEN / "workloads.json").read_text())


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import abi

    return abi.load("oracle")


@pytest.fixture(scope="session")
def hip():
    """The product's native module with the HIP library loaded on a GPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from quantanything_amd import native

    native.require()
    return native
