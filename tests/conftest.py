import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "karaoke-platform-sidecar-native_amd"))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


@pytest.fixture(scope="session")
def ref_pack():
    """Seeded synthetic pack in the reference shape (267,386,408 bytes)."""
    from vocalarc_hip import pack
    from vocalarc_hip.dims import REFERENCE_DIMS
    return pack.synthetic_pack(REFERENCE_DIMS, 1234)


@pytest.fixture(scope="session")
def rng():
    return np.random.default_rng(20261201)
