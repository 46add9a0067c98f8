"""Test setup: the `gpu` marker, and the package loaded from its directory.

GPU tests compare the HIP library (through its C ABI) with the CPU oracle on
the same seeded inputs; CPU tests pin the oracle itself and the host logic.
"""
import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_package():
    if "ppocr_native_amd" in sys.modules:
        return sys.modules["ppocr_native_amd"]
    pkg_dir = ROOT / "ppocr-native_amd"
    spec = importlib.util.spec_from_file_location(
        "ppocr_native_amd", pkg_dir / "__init__.py", submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ppocr_native_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o
