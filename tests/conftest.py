import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG_NAME = "r9700_lru_expert_cache_amd"
PKG_DIR = ROOT / "r9700-lru-expert-cache_amd"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_pkg():
    """Import the package directory (its name is not a Python identifier) as PKG_NAME."""
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(
        PKG_NAME, PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


def gpu_case(msg: str) -> None:
    """Name the case before each GPU step, flushed, so a fault still says what ran."""
    print(f"[gpu-case] {msg}", flush=True)
