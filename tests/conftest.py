"""Shared test setup: import paths, the `gpu` marker, device fixtures.

CPU tests (-m "not gpu") cover the oracle against the reference's known-answer
vectors, the host logic and the C ABI's exported symbols.  GPU tests (-m gpu)
are the parity tests proper: libsgq on a gfx950 device vs the CPU oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "super-gemma_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libsgq.so")


@pytest.fixture(scope="session")
def ctx():
    import torch
    import sgq

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return sgq.GpuContext(0)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o
