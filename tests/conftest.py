"""Shared test set-up: the `gpu` marker, import paths and package loading."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Import the `tau.rs_amd` directory as the module `tau_rs_amd`."""
    if "tau_rs_amd" in sys.modules:
        return sys.modules["tau_rs_amd"]
    pkg_dir = os.path.join(ROOT, "tau.rs_amd")
    spec = importlib.util.spec_from_file_location(
        "tau_rs_amd", os.path.join(pkg_dir, "__init__.py"),
        submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["tau_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def tau():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o
