import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "compress-zip_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

MODEL_PATH = os.path.join(ROOT, "models", "v001_eng.czm")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")
    config.addinivalue_line("markers", "slow: longer CPU test")


def _ensure_oracle():
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    return O


@pytest.fixture(scope="session")
def orc():
    return _ensure_oracle()


@pytest.fixture(scope="session")
def shipped(orc):
    return orc.Model.from_file(MODEL_PATH)


def gpu_available() -> bool:
    try:
        import czip_amd
        return czip_amd.device_count() > 0
    except Exception:
        return False
