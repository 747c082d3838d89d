import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: larger CPU cases")


@pytest.fixture(scope="session")
def port():
    from oracle import oracle as O
    if not O.available("port"):
        O.build(ref=False)
    return O.Oracle("port")


@pytest.fixture(scope="session")
def ref():
    """The reference's own quant.cpp/tier.cpp build, when it exists (this container only)."""
    from oracle import oracle as O
    if not O.available("reference"):
        if os.path.isdir(os.path.join(O.REF_SRC, "src")):
            O.build(ref=True)
        else:
            pytest.skip("reference build oracle/_ref not available")
    return O.Oracle("reference", avx512=False)
