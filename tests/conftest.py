"""Shared pytest setup: the `gpu` marker and helpers for the parity tests."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libwdrz_attn.so on cuda:0)")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from whisperdrz_amd import _lib

    _lib.load()  # a GPU box without the built library is a failure, not a skip
    return torch.device("cuda", 0)
