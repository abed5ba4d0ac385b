"""Shared pytest setup: import paths, the `gpu` marker, and library fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
PACKAGE_DIR = REPO_ROOT / "spaceslug-main_amd"
for p in (str(REPO_ROOT), str(PACKAGE_DIR), str(REPO_ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def runtime_lib_path():
    from spaceslug_amd.backend import library_path

    path = library_path()
    if not path.is_file():
        import build_native

        build_native.build()
    return path


@pytest.fixture(scope="session")
def session(runtime_lib_path):
    from spaceslug_amd import BackendSession

    return BackendSession(library=runtime_lib_path)


@pytest.fixture(scope="session")
def gpu(session):
    """Skips nothing: a GPU test must run on a GPU, so a missing device is a failure."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible GPU")
    return torch.device("cuda:0")
