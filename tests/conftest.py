import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and libdmhip.so")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the GPU tests (fails loudly without a device)."""
    from diskmule_amd import HipContext
    c = HipContext(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def golden():
    import json
    import numpy as np
    here = os.path.join(ROOT, "tests", "golden")
    with open(os.path.join(here, "kat_reference.json")) as f:
        kat = json.load(f)
    seeded = dict(np.load(os.path.join(here, "seeded_small.npz")))
    return kat, seeded
