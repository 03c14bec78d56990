"""Test configuration: import paths, the ``gpu`` marker, shared helpers."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "resihp-reproduction_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) GPU and the built libresihp_hip.so")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP GPU visible")
    from resihp import _hip

    _hip.load()  # a GPU without the built library is a failure, not a skip
    return torch.device("cuda")


def rel_inf(a, b) -> float:
    """max|a - b| / max|b| (the reference's own band form, tests/test_reference.py:154-156)."""
    import torch

    # computed in fp64 on b's device (a GPU for the full-size workloads, whose logits alone
    # are 4e8 elements)
    b = b.detach().double()
    a = a.detach().to(b.device).double()
    scale = b.abs().max().item()
    diff = (a - b).abs().max().item()
    return diff / scale if scale > 0 else diff
