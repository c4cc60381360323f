import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def co():
    """The process-wide device context (loads the built HIP library; no fallback)."""
    from cusr_amd.kernel import co_inproc
    return co_inproc.get_inproc_co(0, "ad")
