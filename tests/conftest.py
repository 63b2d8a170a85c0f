"""pytest configuration: the `gpu` marker and shared fixtures.

`-m "not gpu"` runs the oracle checks, host logic and the ABI export check (no GPU calls);
`-m gpu` runs the parity tests through the C ABI on an MI355X.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libva_hip.so kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def ctx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vectoraccelerate_amd import GPUContext

    c = GPUContext(0)
    yield c
    c.close()
