import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "ziggy-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libziggy_hip.so")
    config.addinivalue_line("markers", "slow: builds a large synthetic model")


@pytest.fixture(scope="session")
def hip_ctx():
    from zhip import hip
    ctx = hip.Context(0)
    yield ctx
    ctx.close()
