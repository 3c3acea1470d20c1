"""Shared pytest setup.

Markers: `gpu` tests need a HIP device (MI355X) and call the product through
its C-ABI; everything else runs on the CPU.  The CPU oracle
(oracle/libneon_oracle.so) is test infrastructure and is built on demand
with gcc when missing.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs on the GPU box")
    config.addinivalue_line("markers", "slow: long-running (full 20b shape)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    if not os.path.exists(o._LIB_PATH):
        o.build()
    o.lib()
    return o


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "hf_gptoss_fixtures.npz")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
