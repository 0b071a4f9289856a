import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libhfmoe.so")


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(GOLDEN, "reference_vectors.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def hf():
    """The initialised library on device 0 (GPU tests only)."""
    from hummingflight_amd import capi
    capi.load()
    capi.call("hfmoe_init", 0)
    yield capi
    capi.load().hfmoe_shutdown()
