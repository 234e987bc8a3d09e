"""Shared test set-up: the `gpu` marker, import paths and the golden fixture."""

import importlib.util
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))

TINY = ROOT / "tests" / "golden" / "tiny"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


def load_package():
    """Imports slm.use_amd/ (a folder whose name is not an identifier) as `slm_use_amd`."""
    if "slm_use_amd" in sys.modules:
        return sys.modules["slm_use_amd"]
    spec = importlib.util.spec_from_file_location(
        "slm_use_amd", ROOT / "slm.use_amd" / "__init__.py",
        submodule_search_locations=[str(ROOT / "slm.use_amd")])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["slm_use_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def tiny_dir():
    return TINY


@pytest.fixture(scope="session")
def pkg():
    return load_package()
