import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parent / "coding-basic-hw-2_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session", autouse=True)
def _checker_libs():
    """Build the CPU oracle and the KAT replayer if they are not built yet (CPU only)."""
    import oracle_lib
    oracle_lib.oracle()
    oracle_lib.katgen()
