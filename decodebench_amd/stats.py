"""Order statistics for right-skewed latency samples (no parametric tests).

Mirrors ``src/decodebench/stats.py:7-57`` of the reference: the same
``Summary`` fields, the same validation messages, and a percentile bootstrap of
``median(a) - median(b)`` that draws from ``numpy.random.default_rng(seed)`` in
the same order (one index matrix for ``a``, then one for ``b``, per chunk), so
that for equal inputs and seed the interval endpoints are identical.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np


@dataclass(frozen=True)
class Summary:
    median: float
    p25: float
    p75: float
    n: int

    @property
    def iqr(self) -> float:
        return self.p75 - self.p25


def _as_samples(values, who: str, empty_msg: str) -> np.ndarray:
    arr = np.asarray(values, dtype=np.float64)
    if arr.size == 0:
        raise ValueError(empty_msg)
    if arr.ndim != 1:
        raise ValueError(f"{who} samples must be one-dimensional")
    if not np.isfinite(arr).all():
        raise ValueError(f"{who} samples must all be finite")
    return arr


def summarize(samples: Sequence[float]) -> Summary:
    """Median and quartiles (numpy's linear interpolation) of one sample set."""
    arr = _as_samples(samples, "summarize()",
                      "summarize() requires at least one sample")
    p25, med, p75 = np.percentile(arr, [25.0, 50.0, 75.0])
    return Summary(median=float(med), p25=float(p25), p75=float(p75),
                   n=int(arr.size))


def bootstrap_diff_ci(a, b, n_resamples: int = 10000, ci: float = 0.95,
                      seed: int = 42) -> tuple[float, float, float]:
    """Percentile-bootstrap interval of ``median(a) - median(b)``.

    Returns ``(lo, hi, point)``.  Resampling runs in chunks of at most about
    one million indices so long sample vectors cannot blow up memory.
    """
    rng = np.random.default_rng(seed)
    msg = "bootstrap_diff_ci() requires non-empty samples"
    xa = np.asarray(a, dtype=np.float64)
    xb = np.asarray(b, dtype=np.float64)
    if xa.size == 0 or xb.size == 0:
        raise ValueError(msg)
    xa = _as_samples(xa, "bootstrap_diff_ci()", msg)
    xb = _as_samples(xb, "bootstrap_diff_ci()", msg)
    if n_resamples <= 0:
        raise ValueError("n_resamples must be positive")
    if not (0.0 < ci < 1.0):
        raise ValueError("ci must be between 0 and 1")

    diffs = np.empty(n_resamples, dtype=np.float64)
    per_chunk = max(1, 1_000_000 // max(xa.size, xb.size))
    done = 0
    while done < n_resamples:
        m = min(per_chunk, n_resamples - done)
        ia = rng.integers(0, xa.size, size=(m, xa.size))
        ib = rng.integers(0, xb.size, size=(m, xb.size))
        diffs[done:done + m] = (np.median(xa[ia], axis=1)
                                - np.median(xb[ib], axis=1))
        done += m
    tail = 0.5 * (1.0 - ci)
    lo, hi = np.quantile(diffs, [tail, 1.0 - tail])
    return float(lo), float(hi), float(np.median(xa) - np.median(xb))
