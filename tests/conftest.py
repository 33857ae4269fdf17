import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X, gfx950)")


@pytest.fixture(scope="session")
def qs():
    """The product package (directory name is not an identifier)."""
    return importlib.import_module("quant-studio_amd")
