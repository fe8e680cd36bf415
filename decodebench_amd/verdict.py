"""Verdict: measured launch overhead against an analytic eliminable-byte time.

Two quantities decide whether a decode-chain fusion is worth writing:

* ``delta_launch = t_stream - t_graph`` -- measured; what graph replay (a
  hipGraph on ROCm, reached through ``torch.cuda.CUDAGraph``) already removes.
* ``B = eliminable_bytes / (total_bytes / t_graph)`` -- the time the
  eliminable intermediate bytes would take at the chain's average byte rate.
  This is a proportional estimate, not a bound: launch-, latency- or
  cache-dominated stages break its linearity assumption.

Semantics, validation messages and the rendered text follow
``src/decodebench/verdict.py:17-114`` of the reference; the rendered sentences
are kept word for word because they are the output format the reference's
tests and users match on (the phrase "CUDA Graphs" included).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

DEFAULT_BYTE_THRESHOLD = 0.01

LOW = "low-byte-opportunity"
MATERIAL = "material-byte-opportunity"


@dataclass(frozen=True)
class Verdict:
    t_stream: float           # us, median of stream-launch trials
    t_graph: float            # us, median of graph-replay trials
    delta_launch: float       # us, t_stream - t_graph (measured)
    b_bytes_est: float        # us, proportional time of the eliminable bytes
    achieved_bw: float        # bytes per us over the unfused chain
    total_bytes: int
    eliminable_bytes: int
    byte_threshold: float
    bound: str                # LOW or MATERIAL (analytic byte fraction)
    dominant: str             # "launch" or "bytes" (larger of the two terms)
    delta_launch_ci: Optional[tuple[float, float]] = None
    t_fused: Optional[float] = None
    residual_us: Optional[float] = None

    @property
    def b_ceiling(self) -> float:
        """Older name of :attr:`b_bytes_est`, kept for callers that use it."""
        return self.b_bytes_est

    def _launch_sentence(self) -> str:
        interval = ""
        straddles_zero = False
        if self.delta_launch_ci is not None:
            lo, hi = self.delta_launch_ci
            interval = f" (95% CI [{lo:.2f}, {hi:.2f}])"
            straddles_zero = lo <= 0.0 <= hi
        if straddles_zero:
            return (f"Measured launch saving {self.delta_launch:.2f} us{interval} "
                    "is statistically indistinguishable from zero (CI spans 0).")
        return (f"CUDA Graphs eliminate {self.delta_launch:.2f} us here{interval} "
                "(measured).")

    def render(self) -> str:
        dominant_text = ("launch overhead (measured)" if self.dominant == "launch"
                         else "eliminable bytes (estimated)")
        out = [
            self._launch_sentence(),
            f"Eliminable intermediate bytes correspond to ~{self.b_bytes_est:.2f} us "
            "at this workload's average byte throughput (analytic proportional "
            "estimate, NOT a strict bound).",
            f"Floor with graphs on (t_graph): {self.t_graph:.2f} us.",
            f"Dominant term: {dominant_text} (delta_launch "
            f"{self.delta_launch:.2f} us vs B {self.b_bytes_est:.2f} us).",
        ]
        if self.t_fused is not None and self.residual_us is not None:
            explained = self.delta_launch + self.b_bytes_est + self.residual_us
            out.append(f"Measured fused latency: {self.t_fused:.2f} us.")
            out.append(
                f"Decomposition: launch overhead {self.delta_launch:.2f} us + "
                f"eliminable bytes {self.b_bytes_est:.2f} us + unexplained "
                f"residual {self.residual_us:.2f} us = {explained:.2f} us "
                "(t_stream - t_fused).")
        if self.bound == LOW:
            advice = ("enable CUDA Graphs first; the declared byte fraction is "
                      "below the configured fusion threshold.")
        else:
            advice = ("the declared byte fraction clears the threshold; benchmark "
                      "a representative fused kernel before committing.")
        out.append(f"Verdict: {self.bound.upper()} -> {advice}")
        if self.bound == MATERIAL and self.dominant == "launch":
            out.append(
                "Caution: measured launch savings exceed the byte estimate; the "
                "material-byte-opportunity classification reflects the analytic "
                "byte fraction, not the empirically dominant source of gain.")
        return "\n".join(out)


def _finite(v: float) -> bool:
    return math.isfinite(v)


def compute_verdict(t_stream: float, t_graph: float, total_bytes: int,
                    eliminable_bytes: int,
                    byte_threshold: float = DEFAULT_BYTE_THRESHOLD,
                    delta_launch_ci: Optional[tuple[float, float]] = None,
                    t_fused: Optional[float] = None) -> Verdict:
    """Build a :class:`Verdict` from medians (us) and the chain's byte totals."""
    if not (_finite(t_stream) and _finite(t_graph)) or t_stream <= 0:
        raise ValueError(
            "t_stream and t_graph must be finite, and t_stream must be positive")
    if t_graph <= 0:
        raise ValueError("t_graph must be positive (us)")
    if t_fused is not None and not (_finite(t_fused) and t_fused > 0):
        raise ValueError("t_fused must be finite and positive (us) when provided")
    if total_bytes <= 0:
        raise ValueError("total_bytes must be positive")
    if eliminable_bytes < 0 or eliminable_bytes > total_bytes:
        raise ValueError("eliminable_bytes must be in [0, total_bytes]")
    if not _finite(byte_threshold) or byte_threshold < 0 or byte_threshold > 1:
        raise ValueError("byte_threshold must be finite and in [0, 1]")
    if delta_launch_ci is not None:
        lo, hi = delta_launch_ci
        if not (_finite(lo) and _finite(hi)) or hi < lo:
            raise ValueError("delta_launch_ci must contain finite ordered bounds")

    achieved_bw = total_bytes / t_graph
    b_est = eliminable_bytes / achieved_bw
    delta = t_stream - t_graph
    bound = MATERIAL if b_est >= byte_threshold * t_graph else LOW
    dominant = "launch" if delta >= b_est else "bytes"
    residual = None if t_fused is None else (t_graph - t_fused) - b_est
    return Verdict(t_stream=t_stream, t_graph=t_graph, delta_launch=delta,
                   b_bytes_est=b_est, achieved_bw=achieved_bw,
                   total_bytes=total_bytes, eliminable_bytes=eliminable_bytes,
                   byte_threshold=byte_threshold, bound=bound,
                   dominant=dominant, delta_launch_ci=delta_launch_ci,
                   t_fused=t_fused, residual_us=residual)
