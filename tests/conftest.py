"""Test configuration: markers, import paths, shared fixtures.

CPU tests (``-m "not gpu"``) pin the oracle against the reference's golden
vectors and check the C ABI and the host bridge without launching kernels.
GPU tests (``-m gpu``) compare the HIP kernels, called through the C ABI,
with the oracle on the same inputs.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "oracle", ROOT / "kernel-craft_amd" / "python", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

LIB_PATH = ROOT / "build" / "libkernels.so"
HEADER = ROOT / "include" / "kernel_craft.h"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU check (set KC_SLOW=1)")


def pytest_collection_modifyitems(config, items):
    if os.environ.get("KC_SLOW") == "1":
        return
    skip = pytest.mark.skip(reason="slow check; set KC_SLOW=1 to run")
    for item in items:
        if "slow" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    with np.load(ROOT / "tests" / "golden" / "reference_kats.npz", allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


@pytest.fixture(scope="session")
def oracle():
    import kc_oracle
    kc_oracle.lib()
    return kc_oracle


@pytest.fixture(scope="session")
def gpu():
    """torch with a visible GPU, and the HIP library loaded; fails loudly."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    if not LIB_PATH.exists():
        pytest.fail(f"{LIB_PATH} missing: run __graft_entry__.build() first")
    import kc_abi
    kc_abi.lib()
    return torch
