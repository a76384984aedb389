import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle as ox

    ox.build()
    return ox


@pytest.fixture(scope="session")
def native_lib():
    """The product library, built in-tree if missing (no GPU needed to load it)."""
    from linuxformer_amd import mk_build

    if not os.path.exists(mk_build.LIB):
        mk_build.build()
    return mk_build.load()
