import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import helpers  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built library")


@pytest.fixture(scope="session")
def oracle():
    mod = helpers.oracle_module()
    if not os.path.exists(mod.LIB_PATH):
        mod.build()
    return mod.Oracle()


@pytest.fixture(scope="session")
def oracle_mod():
    return helpers.oracle_module()


@pytest.fixture(scope="session")
def pkg():
    return helpers.package()


@pytest.fixture(scope="session")
def syn():
    return helpers.synthetic()


@pytest.fixture(scope="session")
def lib(pkg):
    """The product library on the GPU. No fallback: a missing library or
    device fails the test."""
    lib = pkg.load()
    assert lib.pgpu_device_init() == 1, pkg.last_error(lib)
    return lib
