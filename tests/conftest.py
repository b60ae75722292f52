import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_golden(name):
    return json.loads((GOLDEN / name).read_text())


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail loudly when the HIP library cannot be loaded."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from aspec_amd import _lib

    _lib.load()
    return torch.device("cuda:0")
