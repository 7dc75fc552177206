"""Shared fixtures: the product binding (through the C ABI) and the CPU oracle."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_package():
    """Import the mono-qwen27_amd package directory (its name is not a Python identifier)."""
    if "mono_qwen27_amd" in sys.modules:
        return sys.modules["mono_qwen27_amd"]
    pkg_dir = os.path.join(ROOT, "mono-qwen27_amd")
    spec = importlib.util.spec_from_file_location(
        "mono_qwen27_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["mono_qwen27_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # noqa: E402
    return oracle


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def m27q():
    return load_package().m27q


@pytest.fixture(scope="session")
def ora():
    return load_oracle()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    return torch.device("cuda:0")
