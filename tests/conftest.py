"""pytest configuration: `gpu` marker, package registration, shared fixtures."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)
# ComfyUI is not installed: a minimal stand-in of the modules the plugin uses
FAKE_COMFY = os.path.join(TESTS, "fake_comfy")
if FAKE_COMFY not in sys.path:
    sys.path.insert(0, FAKE_COMFY)

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def rt():
    return __graft_entry__._submodule("_hip_runtime")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.build()
    return o


@pytest.fixture(scope="session")
def dev(rt):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not rt.KERNELS_AVAILABLE:
        raise RuntimeError(f"INT-Crush kernels not loaded on a GPU box: {rt.LOAD_ERROR}")
    return torch.device("cuda:0")
