"""Shared test setup: markers, package/oracle loading, GPU gating."""

from __future__ import annotations

import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "onnxruntime-mlx_amd")
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_package():
    """Import onnxruntime-mlx_amd/ as the module `ortmi` (the directory name has a hyphen)."""
    if "ortmi" in sys.modules:
        return sys.modules["ortmi"]
    spec = importlib.util.spec_from_file_location(
        "ortmi", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ortmi"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def ortmi():
    import torch  # noqa: F401  (torch first: it brings the HIP runtime the library binds to)

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o
