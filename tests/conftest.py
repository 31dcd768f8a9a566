import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libkvad_hip on cuda:0)")


@pytest.fixture(scope="session")
def ctx():
    """One kh_ctx for the GPU tests (device 0)."""
    import kvad_amd

    c = kvad_amd.Context(0)
    yield c
    c.close()
