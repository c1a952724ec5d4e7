"""pytest setup: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle pins, golden fixtures, host logic and the
C-ABI load/export checks on the CPU; ``-m gpu`` runs the parity tests that
call the HIP kernels through the C ABI on an MI355X.
"""

import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "unlimited-ocr_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libsrswa.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Repeat the parity figures (near-tie counts, plain max-abs errors) the
    tests reported, so they are visible in a quiet run's log."""
    try:
        from parity_report import LINES
    except ImportError:
        return
    if LINES:
        terminalreporter.section("parity figures")
        for line in LINES:
            terminalreporter.write_line(line)
