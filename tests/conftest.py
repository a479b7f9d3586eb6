import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__ as ge  # noqa: E402

GOLDEN_DIR = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture(scope="session")
def s3dx():
    return ge.load_package()


@pytest.fixture(scope="session")
def O():
    return ge.load_oracle()


@pytest.fixture(scope="session")
def W(s3dx):
    return s3dx.workloads


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN_DIR / "golden.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    manifest = json.loads((GOLDEN_DIR / "manifest.json").read_text())
    return arrays, manifest


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), np.finfo(np.float64).tiny))
