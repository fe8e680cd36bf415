"""Report: raw per-trial timings plus byte traces -> verdict and CSV.

Follows ``src/decodebench/report.py:9-48`` of the reference: medians feed
``compute_verdict``, a bootstrap interval of ``delta_launch`` is attached, a
failed graph capture refuses to produce a verdict, and the CSV layout is
``name,variant,trial,us_per_invocation`` with stream rows, then graph rows,
then fused rows.
"""

from __future__ import annotations

import csv
from dataclasses import dataclass

from decodebench_amd.bytes_model import StageTrace, eliminable_bytes, total_bytes
from decodebench_amd.stats import bootstrap_diff_ci, summarize
from decodebench_amd.verdict import DEFAULT_BYTE_THRESHOLD, Verdict, compute_verdict


@dataclass
class Report:
    name: str
    stream_us: list[float]
    graph_us: list[float]
    traces: list[StageTrace]
    fused_us: list[float] | None = None
    byte_threshold: float = DEFAULT_BYTE_THRESHOLD
    graph_ok: bool = True
    graph_skip_reason: str = ""

    def verdict(self) -> Verdict:
        if not self.graph_ok:
            raise RuntimeError(
                f"CUDA graph capture failed for '{self.name}': "
                f"{self.graph_skip_reason}. Delta_launch is unknown for this "
                "chain; no verdict can be emitted.")
        t_stream = summarize(self.stream_us).median
        t_graph = summarize(self.graph_us).median
        lo, hi, _ = bootstrap_diff_ci(self.stream_us, self.graph_us)
        t_fused = (None if self.fused_us is None
                   else summarize(self.fused_us).median)
        return compute_verdict(
            t_stream=t_stream, t_graph=t_graph,
            total_bytes=total_bytes(self.traces),
            eliminable_bytes=eliminable_bytes(self.traces),
            byte_threshold=self.byte_threshold,
            delta_launch_ci=(lo, hi), t_fused=t_fused)

    def render(self) -> str:
        return self.verdict().render()

    def rows(self):
        """(name, variant, trial, us) tuples in CSV order."""
        groups = [("stream", self.stream_us), ("graph", self.graph_us)]
        if self.fused_us is not None:
            groups.append(("fused", self.fused_us))
        for variant, samples in groups:
            for i, us in enumerate(samples):
                yield self.name, variant, i, us

    def to_csv(self, path: str) -> None:
        with open(path, "w", newline="") as fh:
            writer = csv.writer(fh)
            writer.writerow(["name", "variant", "trial", "us_per_invocation"])
            writer.writerows(self.rows())
