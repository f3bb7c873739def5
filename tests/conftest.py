"""Shared test setup: import paths, the `gpu` marker, and the libraries under test.

`-m "not gpu"` tests run anywhere (the oracle against golden vectors and closed forms,
the C ABI's layout and exports, refusals that never reach a launch); `-m gpu` tests
call the HIP library through its C entries on an MI355X and compare with the oracle.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "uniserve-v1_amd"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib

    return oracle_lib


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert name.startswith("gfx950"), f"these kernels are built for gfx950, the device is {name}"
    from uniserve_moe import library

    library()  # fails loudly when the HIP library is not built
    return torch.device("cuda:0")
