import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "mlx-confucius4-tts_amd")
for p in (os.path.join(REPO, "oracle"), PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def gpu_ctx():
    """Library context on cuda:0. The library must be built (no fallback)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test collected without a visible GPU")
    import c4s
    ctx = c4s.Context(0)
    yield ctx
    torch.cuda.synchronize()
    ctx.close()
