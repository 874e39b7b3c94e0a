import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "herbert-metal-bf16_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The HIP context of device 0.  A GPU test that cannot open it fails:
    no CPU fallback exists."""
    import herbert_hip as hb
    g = hb.Gpu(0)
    print("[gpu]", g.summary(), flush=True)
    yield g
    g.close()
