import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "pk_address_golden.npz")
    blob = np.load(path)
    names = sorted({k.split(".")[0] for k in blob.files})
    return {n: {f: blob[f"{n}.{f}"] for f in ("z", "keys1", "keys2", "k", "sv", "si")} for n in names}
