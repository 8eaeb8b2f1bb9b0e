import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "d2-sd_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden" / "cascade_golden.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def golden():
    data = np.load(GOLDEN, allow_pickle=False)
    cases = {}
    for key in data.files:
        case, name = key.split("/", 1)
        cases.setdefault(case, {})[name] = data[key]
    return cases
