"""Test configuration: the ``gpu`` marker (tests that launch the HIP kernels on an MI355X).

``python -m pytest tests -m "not gpu"`` runs the CPU suite (oracle vs golden vectors and
closed forms, host logic, the C-ABI library's exports); ``-m gpu`` the parity tests, which
call the kernels through the C ABI and compare them with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels through the C ABI)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible (run on the MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    import torch

    return torch.device("cuda", 0)
