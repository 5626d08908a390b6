"""Shared pytest configuration: the `gpu` marker and common helpers."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        'markers', 'gpu: needs an MI355X (runs the HIP kernels)')


@pytest.fixture
def cuda():
    """The GPU device; a gpu-marked test fails (not skips) without one."""
    import torch
    assert torch.cuda.is_available(), 'gpu test run without a visible GPU'
    return torch.device('cuda', 0)


def announce(msg):
    """Print the case about to run on the GPU, flushed, so a crash names it."""
    print(f'[case] {msg}', flush=True)
