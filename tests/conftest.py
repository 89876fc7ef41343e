import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "teco-ops_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


# Parity figures (max abs error, DIFF1, ...) that tests record with
# helpers.record(); printed after the run, also under -q.
FIGURES = []


def pytest_terminal_summary(terminalreporter):
    if FIGURES:
        terminalreporter.section("parity figures")
        for line in FIGURES:
            terminalreporter.write_line(line)
