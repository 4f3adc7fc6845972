import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # As in the reference (tests/conftest.py:5-13): `gpu` tests are skipped, not failed, on machines
    # without a GPU, so the CPU suite runs cleanly.
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
