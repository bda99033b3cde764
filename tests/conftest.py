import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "infer.net_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def device():
    """A QuantizedHip context on cuda:0. GPU tests fail (not skip) when the library is
    missing or no gfx950 device is present."""
    import torch
    import deepinfer_hip as dh
    assert torch.cuda.is_available(), "GPU test without a visible GPU"
    torch.cuda.init()
    dev = dh.QuantizedHip()
    yield dev
    dev.dispose()
