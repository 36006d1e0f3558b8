"""Shared test setup: import paths, markers and lazily-built handles.

`-m "not gpu"` tests run on any host (oracle pins, golden fixtures, C-ABI
exports). `-m gpu` tests need an MI355X and call libapus_hip.so through its
C ABI, checking it against the CPU oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "apus-deepseek-v4-flash_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")
    config.addinivalue_line("markers", "slow: long-running CPU check")


@pytest.fixture(scope="session")
def oracle():
    from pyoracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from pyoracle import Reference, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref/libapus_ref.so not built (apus sources absent)")
    return Reference()


@pytest.fixture(scope="session")
def hip():
    import apus_hip
    apus_hip.enable()
    return apus_hip


@pytest.fixture
def rng():
    return np.random.default_rng(20260729)


def pytest_terminal_summary(terminalreporter):
    from helpers import SUMMARY_LINES
    if SUMMARY_LINES:
        terminalreporter.section("figures reported by the tests")
        for line in SUMMARY_LINES:
            terminalreporter.write_line(line)
