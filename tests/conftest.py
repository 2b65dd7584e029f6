import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "nyion.rs_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0.  GPU tests fail (never skip) when it is absent."""
    import torch
    import nyion_hip

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    nyion_hip.init(0)
    return nyion_hip
