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
    terminalreporter.write_sep("-", "decode parity vs the oracle: achieved error")
    terminalreporter.write_line("max-abs |ref|<=2   err/bar   err/bar |ref|>2   max-abs all   "
                                "max|ref|  case")
    for name, small, ratio, m, mx, bf16, big in tolerance.RESULTS:
        terminalreporter.write_line(f"{small:14.3e} {ratio:9.3f} {big:17.3f} {m:13.3e} {mx:10.3g}  "
                                    f"{name}" + (" (bf16 output)" if bf16 else ""))
    worst = max(tolerance.RESULTS, key=lambda r: r[2])
    worst_big = max(tolerance.RESULTS, key=lambda r: r[6])
    f16 = [r[1] for r in tolerance.RESULTS if not r[5]]
    b16 = [r[1] for r in tolerance.RESULTS if r[5]]
    terminalreporter.write_line(
        f"worst err/bar {worst[2]:.3f} in {worst[0]}; worst err/bar where |ref| > 2: "
        f"{worst_big[6]:.3f} in {worst_big[0]} (bar 2e-3 + 2^-11 |ref| fp16, one side rounded)")
    terminalreporter.write_line(
        f"worst max-abs at |ref|<=2: {max(f16, default=0.0):.3e} with fp16 output (bar 2e-3), "
        f"{max(b16, default=0.0):.3e} with bf16 output (bar 2e-3 + (2^-8 + 2^-11) |ref|)")
