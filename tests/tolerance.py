"""The decode parity bar, and a record of the error each GPU case achieved.

Bar: max |gpu - oracle| <= 2e-3 against the oracle's
fp32 dequantise -> SDPA result before output rounding.  Where |oracle| > 2
the fp16 output spacing is 2^-9 or more, so half an ulp of the rounding both
sides apply independently is added there (2^-10 |oracle|); at and below 2
the bar is the plain 2e-3.  bf16 outputs carry the bf16 rounding instead
(relative 2^-8, half an ulp) at every magnitude.

Each check records the achieved max-abs error, which conftest prints in the
terminal summary, so a regression from 1e-3 to 1.9e-3 shows up in the log.
"""
from __future__ import annotations

import numpy as np

ATOL = 2e-3
F16_KNEE = 2.0
RTOL_F16 = 2.0 ** -10
RTOL_BF16 = 2.0 ** -8

# (case, max-abs error where |ref| <= 2, max error / bar over all elements,
#  max-abs error over all elements, max |ref|, bf16 output)
RESULTS: list[tuple[str, float, float, float, float, bool]] = []


def bound(ref: np.ndarray, bf16: bool = False) -> np.ndarray:
    a = np.abs(ref)
    if bf16:
        return ATOL + RTOL_BF16 * a
    return np.where(a <= F16_KNEE, ATOL, ATOL + RTOL_F16 * a)


def check(name: str, got: np.ndarray, ref: np.ndarray, bf16: bool = False) -> float:
    """Assert got is within the bar of ref (both float arrays, NaN-free) and
    record the max-abs error under `name`; returns it."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    err = np.abs(got - ref)
    m = float(err.max()) if err.size else 0.0
    b = bound(ref, bf16)
    small = np.abs(ref) <= F16_KNEE
    RESULTS.append((name, float(err[small].max()) if small.any() else 0.0,
                    float((err / b).max()) if err.size else 0.0, m,
                    float(np.abs(ref).max()) if ref.size else 0.0, bf16))
    over = err > b
    assert not over.any(), (f"{name}: max abs err {m:.3e}; {int(over.sum())} elements over "
                            f"the bar, worst at |ref| = {float(np.abs(ref)[over].max()):.3g}")
    return m
