import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU; runs on the GPU box")
    # torch bundles its own HIP runtime (SONAME libamdhip64.so.7).  Importing
    # it before any of our libraries makes them bind to that same runtime; if
    # one of ours loaded first, the system runtime and torch's would both be
    # mapped and torch could not initialise the GPU.
    import torch  # noqa: F401


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle
