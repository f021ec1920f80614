import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "gemma4-12b-snapdragonx2elite_amd"
PKG_NAME = "g4mi"

if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_pkg():
    """Import the package directory (its name is not a Python identifier) as ``g4mi``."""
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(PKG_NAME, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libq4mi.so")


@pytest.fixture(scope="session")
def g4():
    return load_pkg()


@pytest.fixture(scope="session")
def gpu(g4):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    ops = importlib.import_module(f"{PKG_NAME}.ops")
    return ops


@pytest.fixture
def tune(g4):
    """Plan overrides (q4_tune_set) for one test: ``tune("gemv_rows", 16)``;
    every override is cleared when the test ends."""
    ops = importlib.import_module(f"{PKG_NAME}.ops")
    ops.tune_reset()
    yield ops.tune_set
    ops.tune_reset()
