"""Shared pytest setup: the `gpu` marker and repository paths.

Tests marked `gpu` need a real MI355X and call the HIP library through its
C-ABI; everything else runs on the CPU (oracle vs golden vectors, host-side
format / validation logic, and the library's exported-symbol check).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bitsqueeze-llm_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long CPU test")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    d = os.path.join(ROOT, "tests", "golden")
    return {
        "nf4": dict(np.load(os.path.join(d, "nf4_golden.npz"), allow_pickle=False)),
        "topk": dict(np.load(os.path.join(d, "topk_golden.npz"), allow_pickle=False)),
    }
