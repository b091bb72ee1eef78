import importlib.util
import os
import sys

import pytest

try:  # import once at collection, outside per-test time limits
    import torch  # noqa: F401
except ImportError:  # pragma: no cover
    torch = None

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Import voxtral.cpp_amd/ (not a Python identifier) as `voxtral_cpp_amd`."""
    if "voxtral_cpp_amd" in sys.modules:
        return sys.modules["voxtral_cpp_amd"]
    pkg_dir = os.path.join(ROOT, "voxtral.cpp_amd")
    spec = importlib.util.spec_from_file_location(
        "voxtral_cpp_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["voxtral_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_package()
