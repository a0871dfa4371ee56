"""Shared test setup: import paths for the fp8lin package and the CPU oracle,
the `gpu` marker, and helpers to compare BF16 outputs with the oracle."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "a100-vision-infer_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def fp8lin():
    import fp8lin as F
    F.lib()
    return F


@pytest.fixture(scope="session")
def gpu(fp8lin):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    rc = fp8lin.lib().fp8lin_init()
    assert rc == 0, fp8lin.lib().fp8lin_last_error()
    return torch.device("cuda:0")
