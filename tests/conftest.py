import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "lightbridge-engine_amd"
for p in (ROOT, PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"
REF_FIXTURES = GOLDEN / "reference"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import lb_oracle
    lb_oracle.lib()
    return lb_oracle


def read_fixture(name: str) -> bytes:
    return (REF_FIXTURES / name).read_bytes()
