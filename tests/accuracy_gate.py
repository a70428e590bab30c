"""The reference's three-way accuracy gate, restated in numpy.

``ref/chunk_gated_delta_rule/tests/assets/impl/compare.py:32-35,55-196`` compares a device
output (``npu``) and a third-party bf16 benchmark (``bench``) with the fp32 CPU golden, and
passes the device when its errors stay within fixed multiples of the benchmark's:

  max_re = max |x - g| / (|g| + 1e-3)     ratio < 5
  avg_re = mean |x - g| / (|g| + 1e-3)    ratio < 1.5
  rmse   = sqrt(mean (x - g)^2)           ratio < 1.5
  smra   = share of the golden's small values (|g| < 2^-10) where |x - g| > 1e-16,  ratio < 2

each ratio being ``npu / max(bench, 2^-8)`` (1 when both are 0, inf when only the benchmark's
is), or unconditionally when the device's max_re is below 2^-7 (``:157-161``).  Here the
golden is the exact recurrence ``fwd_h(rounding=None)`` and the benchmark the bf16-state
recurrence ``fwd_h_bf16_state`` of the oracle.
"""

from __future__ import annotations

import numpy as np

MIN_ERR = 1e-3
ERR_THRESHOLD = 2.0 ** -8
SMALL_VALUE = 2.0 ** -10
SMALL_VALUE_ATOL = 1e-16
THRESHOLDS = dict(max_re=5.0, avg_re=1.5, rmse=1.5, smra=2.0)
ESCAPE_MAX_RE = 2.0 ** -7


def errors(x, g) -> dict:
    x = np.asarray(x, np.float32).reshape(-1)
    g = np.asarray(g, np.float32).reshape(-1)
    rel = np.abs(x - g) / (np.abs(g) + np.float32(MIN_ERR))
    small = np.abs(g) < SMALL_VALUE
    n_small = int(small.sum())
    smra = 0.0 if n_small == 0 else int((small & (np.abs(g - x) > SMALL_VALUE_ATOL)).sum()) / n_small
    return dict(max_re=float(rel.max()), avg_re=float(rel.mean()),
                rmse=float(np.sqrt(np.mean(np.square(x - g)))), smra=smra)


def _ratio(num: float, den: float) -> float:
    if den == 0:
        return 1.0 if num == 0 else float("inf")
    return float(num / max(den, ERR_THRESHOLD))


def cross_check(npu, golden, bench) -> dict:
    """Ratios of the device's errors to the benchmark's, and the verdict."""
    e_npu, e_bench = errors(npu, golden), errors(bench, golden)
    ratios = {k: _ratio(e_npu[k], e_bench[k]) for k in THRESHOLDS}
    passed = all(ratios[k] < THRESHOLDS[k] for k in THRESHOLDS) or e_npu["max_re"] < ESCAPE_MAX_RE
    return dict(passed=passed, ratios=ratios, npu=e_npu, bench=e_bench)
