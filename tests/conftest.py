"""Test configuration: the ``gpu`` marker and the package loader.

The package directory ``qwen3.5-35b-dflash_amd`` is not a Python identifier;
it is loaded under the alias ``qwen35_dflash_amd``.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "qwen3.5-35b-dflash_amd"
PKG_NAME = "qwen35_dflash_amd"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_package():
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(PKG_NAME, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    module = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = module
    spec.loader.exec_module(module)
    return module


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def device(pkg):
    # GPU tests must run on the GPU: a missing device is a failure, never a skip.
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    pkg._lib.load()
    return torch.device("cuda:0")
