"""Shared fixtures. `gpu` marks tests that need an MI355X (or any HIP GPU);
everything else runs on the CPU."""

import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "grpc-unlimited-ocr_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


def load_backend():
    """The package grpc-unlimited-ocr_amd (its directory name is not an
    identifier, so it is loaded by path) as module `uocr_rocm`."""
    if "uocr_rocm" in sys.modules:
        return sys.modules["uocr_rocm"]
    spec = importlib.util.spec_from_file_location("uocr_rocm", os.path.join(PKG_DIR, "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["uocr_rocm"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def backend():
    return load_backend()


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle
