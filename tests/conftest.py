"""Shared test setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root on sys.path so ``oracle`` imports;
* ``vo`` fixture: the product package ``vllm-oxide_amd`` (loaded by path,
  since the directory name is not a Python identifier).
"""
import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950)")


def load_vo():
    """Import vllm-oxide_amd as module `vllm_oxide_amd`."""
    name = "vllm_oxide_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "vllm-oxide_amd"
    spec = importlib.util.spec_from_file_location(
        name, pkg_dir / "__init__.py", submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def vo():
    return load_vo()


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def gpu_backend(vo):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return vo.HipBackend(device=0)
