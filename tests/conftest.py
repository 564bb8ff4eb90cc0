import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "vk-shei_amd"), os.path.join(ROOT, "tests")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ctx():
    """One gfx950 context on torch's current stream for the whole GPU session."""
    import torch
    import mslim_attn

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = mslim_attn.Context()
    c.use_torch_stream()
    yield c
    c.synchronize()
    c.close()
