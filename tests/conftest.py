import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _have_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _have_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter):
    """Achieved max-abs error of every parity check against the oracle."""
    try:
        from tests import tolerance
    except ImportError:
        return
    if not tolerance.RESULTS:
        return
    terminalreporter.write_sep("-", "decode parity: achieved max-abs error vs oracle (bar 2e-3)")
    worst = max(tolerance.RESULTS, key=lambda r: r[1])
    for name, err, mx in tolerance.RESULTS:
        terminalreporter.write_line(f"{err:9.3e}  (max |ref| {mx:8.3g})  {name}")
    terminalreporter.write_line(f"worst: {worst[1]:.3e} in {worst[0]}")
