import importlib
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

PKG_NAME = "inference-engine_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def _ensure_built():
    """CPU-only hosts build the in-tree libraries if missing (hipcc cross-compiles); a GPU box
    uses what the snapshot carries and never builds inside a test run."""
    lib = REPO / PKG_NAME / "lib"
    if (lib / "libie_attn.so").exists() and (lib / "_ie_torch_ops.so").exists():
        return
    if _gpu_available():
        return
    build = importlib.import_module(f"{PKG_NAME}.build")
    build.build()


@pytest.fixture(scope="session")
def ie():
    _ensure_built()
    return importlib.import_module(PKG_NAME)


@pytest.fixture(scope="session")
def workloads(ie):
    return importlib.import_module(f"{PKG_NAME}.workloads")


@pytest.fixture(scope="session")
def step_inputs(ie):
    return importlib.import_module(f"{PKG_NAME}.step_inputs")


@pytest.fixture(scope="session")
def native(ie):
    return importlib.import_module(f"{PKG_NAME}._native")


@pytest.fixture(scope="session")
def dev():
    return "cuda:0"
