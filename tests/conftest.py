import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels through the C-ABI")
    config.addinivalue_line("markers", "slow: longer CPU checks (still part of the default CPU suite)")


@pytest.fixture(scope="session")
def oracle():
    import cabi
    if not os.path.exists(cabi.ORACLE_SO):
        pytest.fail("oracle/libsjo.so is not built: run __graft_entry__.build() or make -C oracle")
    return cabi.oracle()


@pytest.fixture(scope="session")
def ref():
    import cabi
    r = cabi.reference()
    if r is None:
        pytest.skip("oracle/_ref (the reference compiled from its header) is not built here")
    return r
