import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: a large model or long context")


@pytest.fixture(scope="session")
def hip():
    """The hip device on GPU 0, shared by the GPU tests of a session."""
    from titania_amd import Hip

    dev = Hip(0)
    yield dev
    dev.close()
