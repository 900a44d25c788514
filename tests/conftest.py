import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "quixicore-cpu_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    return o


@pytest.fixture(scope="session")
def ref():
    import oracle as o
    if not o.Reference.available():
        pytest.skip("oracle/_ref not built (needs the reference sources: make -C oracle ref)")
    return o.Reference()


@pytest.fixture(scope="session")
def synth():
    from quixicore_hip import synth as s
    return s


@pytest.fixture(scope="session")
def qc():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import quixicore_hip
    return quixicore_hip


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


def xorshift32_unit(seed, count):
    """The reference tests' RNG (tests/correctness/test_qgemv.cpp:31-43):
    xorshift32, value (state >> 8) * 2/2^24 - 1."""
    s = seed & 0xFFFFFFFF
    out = np.empty(count, dtype=np.float32)
    for i in range(count):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = np.float32(s >> 8) * np.float32(2.0 / 16777216.0) - np.float32(1.0)
    return out
