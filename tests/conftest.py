"""Shared test setup.

* registers the `gpu` marker (tests that need an MI355X);
* imports the product package `longbow-fletcher_amd/` as `longbow_fletcher_amd`
  (its directory name is not a Python identifier);
* puts oracle/ (the CPU restatement of the reference path, used only as the
  checker) on sys.path.
"""
import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _load_package():
    name = "longbow_fletcher_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "longbow-fletcher_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


_load_package()
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X / gfx950)")


@pytest.fixture(scope="session")
def fl():
    return sys.modules["longbow_fletcher_amd"]


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ctx(fl):
    c = fl.Context(0)
    yield c
    c.close()
