"""The decode parity bar, and a record of the error each GPU case achieved.

Bar: max |gpu - oracle| <= 2e-3 against the oracle's
fp32 dequantise -> SDPA result before output rounding.  Only the GPU side is
rounded to the output type there, so above |oracle| = 2 the bar adds what
that one rounding can contribute:

* fp16 output: half an fp16 ulp, at most 2^-11 |x| (an fp16 in [2^e, 2^(e+1))
  has spacing 2^(e-10));
* bf16 output: the kernel rounds fp32 -> fp16 -> bf16 (F:886-894, then the
  output tensor's dtype), so half a bf16 ulp plus half an fp16 ulp,
  2^-8 |x| + 2^-11 |x|, at every magnitude (bf16 rounding alone exceeds 2e-3
  from |x| = 0.5 on).

At and below |oracle| = 2 the fp16 bar is the plain 2e-3.

Where both sides are GPU outputs rounded to the same type (one schedule
against another on the same inputs), each may round to a different
neighbour, so the allowance is a full ulp instead of half: 2^-10 |x| (fp16).

Each check records the achieved max-abs error, which conftest prints in the
terminal summary, with the worst error/bar ratio where |ref| > 2 apart, so a
regression on large outputs (the x20 outlier channels) shows up in the log.
"""
from __future__ import annotations

import numpy as np

ATOL = 2e-3
F16_KNEE = 2.0
RTOL_F16 = 2.0 ** -11          # half an fp16 ulp (one side rounded)
RTOL_F16_BOTH = 2.0 ** -10     # one fp16 ulp (both sides rounded)
RTOL_BF16 = 2.0 ** -8 + 2.0 ** -11   # fp32 -> fp16 -> bf16, one side rounded

# (case, max-abs error where |ref| <= 2, max error / bar over all elements,
#  max-abs error over all elements, max |ref|, bf16 output,
#  max error / bar where |ref| > 2 (0 when there is none))
RESULTS: list[tuple[str, float, float, float, float, bool, float]] = []


def bound(ref: np.ndarray, bf16: bool = False, both_rounded: bool = False) -> np.ndarray:
    a = np.abs(ref)
    if bf16:
        return ATOL + (2 * RTOL_BF16 if both_rounded else RTOL_BF16) * a
    return np.where(a <= F16_KNEE, ATOL, ATOL + (RTOL_F16_BOTH if both_rounded else RTOL_F16) * a)


def check(name: str, got: np.ndarray, ref: np.ndarray, bf16: bool = False,
          both_rounded: bool = False) -> float:
    """Assert got is within the bar of ref (both float arrays, NaN-free) and
    record the max-abs error under `name`; returns it.  `both_rounded`: ref
    is itself a GPU output rounded to the same type."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    err = np.abs(got - ref)
    m = float(err.max()) if err.size else 0.0
    b = bound(ref, bf16, both_rounded)
    small = np.abs(ref) <= F16_KNEE
    big = ~small
    RESULTS.append((name, float(err[small].max()) if small.any() else 0.0,
                    float((err / b).max()) if err.size else 0.0, m,
                    float(np.abs(ref).max()) if ref.size else 0.0, bf16,
                    float((err[big] / b[big]).max()) if big.any() else 0.0))
    over = err > b
    assert not over.any(), (f"{name}: max abs err {m:.3e}; {int(over.sum())} elements over "
                            f"the bar, worst at |ref| = {float(np.abs(ref)[over].max()):.3g}")
    return m
