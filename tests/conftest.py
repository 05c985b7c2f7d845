import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    import json

    import numpy as np

    here = ROOT / "tests" / "golden"
    meta = json.loads((here / "golden.json").read_text())
    with np.load(here / "golden.npz", allow_pickle=False) as data:
        arrays = {name: data[name] for name in data.files}
    return meta, arrays
