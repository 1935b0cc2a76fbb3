import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
TESTS = Path(__file__).resolve().parent
for p in (str(ROOT), str(TESTS), str(TESTS / "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    # GPU tests skip only where no GPU exists at all; on a GPU box a missing
    # library or kernel failure is an error, never a skip.
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    try:
        import torch

        has_gpu = torch.cuda.device_count() > 0
    except Exception:  # pragma: no cover
        has_gpu = False
    if not has_gpu:
        skip = pytest.mark.skip(reason="no GPU in this environment")
        for it in gpu_items:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    data = np.load(TESTS / "golden" / "golden.npz", allow_pickle=False)
    meta = json.loads((TESTS / "golden" / "golden.json").read_text())
    return data, meta


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.lib()
    return oracle
