import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests cannot run without a device; keep them collected (so -m gpu
    # selects them) but skip them cleanly where torch sees no GPU.
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The measured errors of the tolerance checks that ran (see
    helpers.margin), so the margins show in a plain ``-q`` run."""
    try:
        from helpers import MARGINS
    except ImportError:
        return
    if MARGINS:
        terminalreporter.section("parity margins (measured error vs bar)")
        for line in MARGINS:
            terminalreporter.write_line(line)
