"""Measurement helpers: keep a run's stderr for the log, and reduce per-iteration times to statistics
(src/benchmark/monitor.py)."""

from __future__ import annotations

import contextlib
import io
import sys
from dataclasses import dataclass


class _Tee(io.TextIOBase):
    """Writes to a buffer and passes every write on to the stream it wraps, as it happens."""

    def __init__(self, stream):
        self.buf, self.stream = io.StringIO(), stream

    def write(self, text):
        self.buf.write(text)
        self.stream.write(text)
        self.stream.flush()
        return len(text)

    def getvalue(self):
        return self.buf.getvalue()


@contextlib.contextmanager
def capture():
    """Collects everything written to stderr inside the block (for the saved log) while still showing it as it is
    written (a long compile inside the block then shows its progress lines at once)."""
    tee = _Tee(sys.stderr)
    with contextlib.redirect_stderr(tee):
        yield tee


@dataclass
class TimingResults:
    mean_ms: float
    std_ms: float
    min_ms: float
    max_ms: float
    iterations: int
    q1_ms: float
    q3_ms: float
    iqr_ms: float
    outliers: int
    verified: bool | None = None
    ref_mean_ms: float | None = None
    speedup: float | None = None


def _quantile(sorted_times, q):
    """Linear interpolation between the closest ranks (numpy's default method)."""
    pos = q * (len(sorted_times) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(sorted_times) - 1)
    return sorted_times[lo] + (sorted_times[hi] - sorted_times[lo]) * (pos - lo)


def stats(times_ms, verified=None, ref_mean_ms=None) -> TimingResults:
    """Mean, population standard deviation, extremes, quartiles and Tukey outliers (samples outside
    [q1 - 1.5 IQR, q3 + 1.5 IQR]) of per-iteration times; ``speedup`` = reference mean / this mean."""
    if not times_ms:
        raise ValueError("no samples")
    t = sorted(float(x) for x in times_ms)
    n = len(t)
    mean = sum(t) / n
    std = (sum((x - mean) ** 2 for x in t) / n) ** 0.5
    q1, q3 = _quantile(t, 0.25), _quantile(t, 0.75)
    iqr = q3 - q1
    outliers = sum(1 for x in t if x < q1 - 1.5 * iqr or x > q3 + 1.5 * iqr)
    r = lambda v: round(v, 4)  # noqa: E731
    return TimingResults(r(mean), r(std), r(t[0]), r(t[-1]), n, r(q1), r(q3), r(iqr), outliers, verified,
                         ref_mean_ms, None if ref_mean_ms is None else round(ref_mean_ms / mean, 3))
