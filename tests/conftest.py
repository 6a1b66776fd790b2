import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "gemma4-webgpu_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libg4hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One device context for the whole GPU session (fails loudly if absent)."""
    import g4hip

    c = g4hip.Context(0)
    info = c.info()
    print(f"\n[g4] device: {info}", flush=True)
    yield c
    c.close()


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O
