import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "vspec-engine_amd"
for p in (ROOT, PKG / "python"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference's own C path, compiled from its sources into oracle/_ref."""
    from oracle.oracle import REF_SO, Reference

    if not REF_SO.exists():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return Reference()


@pytest.fixture(autouse=True)
def _clean_numerics_env():
    saved = {k: os.environ.get(k) for k in ("VSPEC_3BIT_RUNTIME_MODULE", "VSPEC_FUSED_BITS", "VSPEC_3BIT_BLOCK_SIZE")}
    yield
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
