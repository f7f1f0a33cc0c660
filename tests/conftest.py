import os
import sys

import pytest

# torch ships its own libamdhip64 (same soname as ROCm's).  Loading it before
# libsnapjudge_hip.so makes both share one HIP runtime in this process; the
# other order loads two runtimes and torch then sees no GPU.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle

    return Oracle()
