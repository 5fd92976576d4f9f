import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (os.path.join(ROOT, "chat-wgpu_amd"), os.path.join(ROOT, "oracle"), GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def ctx():
    import cw
    try:
        c = cw.Context(0)
    except cw.CwError as e:
        msg = str(e)
        if "of 0" in msg or "no ROCm-capable device" in msg or "hipErrorNoDevice" in msg:
            pytest.skip(f"no HIP device: {msg}")
        raise
    info = c.info()
    print(f"\n[ctx] device {info}", flush=True)
    yield c
    c.close()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
