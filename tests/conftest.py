"""Test configuration: the `gpu` marker and repo-root imports.

Tests marked `gpu` need a ROCm GPU and the built libmce.so; everything else
runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmce.so")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("this test needs a GPU (run with -m 'not gpu' on a CPU host)")
    return torch.device("cuda:0")


def pytest_runtest_setup(item):
    if "gpu" in item.keywords:
        # name the case before anything touches the GPU, so a crash is attributable
        print(f"\n[gpu-test] {item.nodeid}", flush=True)
