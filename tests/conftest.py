"""Shared fixtures.  `gpu`-marked tests need a gfx950 device and the built
libulspec.so; everything else runs on the CPU."""
import importlib.util
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "universal-loader_amd")
sys.path.insert(0, os.path.join(REPO, "oracle"))


def load_package():
    if "universal_loader_amd" in sys.modules:
        return sys.modules["universal_loader_amd"]
    spec = importlib.util.spec_from_file_location(
        "universal_loader_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["universal_loader_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def ora():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def ctx(pkg):
    c = pkg.Context(0)
    yield c
    c.close()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
