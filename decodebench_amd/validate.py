"""Fail-closed validation report over this build's measurements.

The MI355X counterpart of the reference's analysis gate
(validation/analysis/compare.py:1-690): it joins the timing of the
decomposition configs (``bench.py``'s ``decomposition``: stream / graph /
fused trials of Sequence.profile) with the rocprofv3 counter summary
(``decodebench_amd.rocprof``: per-call kernel time τ and HBM bytes of the
fused call and of the unfused torch stage chain) and records structured
checks, from which the overall verdict is computed:

* **G0 completeness** -- every expected config has at least
  ``min_timing_samples`` usable trials per variant and counter data (bytes
  and τ) for both variants.  Missing data is a FAIL (WARN with
  ``allow_missing_counters``), never a skip.
* **G1 correctness** -- the fused output matched the unfused torch stages
  (bench.py's ``fused_check``, Sequence.profile's elementwise bar).
* **(a) decomposition** t_graph − t_fused = B + S, S the unexplained
  residual with a deterministic bootstrap 95% interval; gated by the sign
  agreement of the wall-clock gap and the kernel-time gap τ_u − τ_f, which
  is INDETERMINATE inside a 5 µs band (compare.py:238-250).
* **(b) bytes** -- F1/F2: the byte model's total within ±20% of the counter
  bytes of both variants.  F4: the eliminated delta (unfused − fused
  counter bytes) within ±``f4_delta_tol`` of the analytic delta
  (eliminable bytes minus the split partial records), only when that delta
  is ≥ 5% of the smaller total, else INDETERMINATE (compare.py:106-125,
  253-266).  The decode-layer rows are printed as diagnostics.
* **(c) Δ_launch** ≥ −max(0.5%·t_graph, 2 µs).
* **(H)** the reference's pre-registered v2 hypotheses: H1-v2 for F1/F2
  (fusion brings no wall-clock win and S ≤ max(1%·t_graph, 3 µs)), H2-v2 for
  F4 (t_fused < t_graph, S > 0, S > B).  They were registered for the
  reference's kernels on its GPU; ``hypotheses="report"`` (the default)
  records their outcome here without gating, ``"gate"`` gates on them as
  compare.py does.

INDETERMINATE adds no support (not a PASS) and does not gate (not a FAIL);
WARN makes the verdict INCOMPLETE.  The command exits non-zero on any FAIL
or WARN.

    python -m decodebench_amd.validate --bench bench.json \\
        --traffic profiles/traffic.json --kernel-trace profiles/kernel_trace_b1.json \\
        --output validation_report.md
"""

from __future__ import annotations

import argparse
import json
import math
import statistics
import sys
from pathlib import Path

import numpy as np

# config -> fusion family (F1/F2 byte and H1 rules, F4 delta and H2 rules,
# the decode layer as diagnostics)
EXPECTED = (("f1_cfg1", "f1"), ("f2_cfg2", "f2"), ("f4_L8192", "f4"),
            ("layer_cfg5", "layer"), ("layer_cfg5_fp8", "layer"))
VARIANTS = ("stream", "graph", "fused")
STATUSES = ("PASS", "FAIL", "WARN", "INDETERMINATE")


class Checks:
    """Structured check registry; the overall verdict comes from here."""

    def __init__(self):
        self.records: list[dict] = []

    def add(self, section: str, label: str, status: str, detail: str = "") -> str:
        if status not in STATUSES:
            raise ValueError(f"unknown status {status!r}")
        self.records.append({"section": section, "label": label, "status": status,
                             "detail": detail})
        return status

    def counts(self) -> dict:
        c = {s: 0 for s in STATUSES}
        for r in self.records:
            c[r["status"]] += 1
        return c

    def overall(self) -> str:
        c = self.counts()
        if c["FAIL"]:
            return "FAIL"
        return "INCOMPLETE" if c["WARN"] else "PASS"


def residual_term(t_graph: float, t_fused: float, b_est: float) -> float:
    """S = (t_graph − t_fused) − B: what the proportional byte estimate does
    not explain (positive when fusion saves more than the bytes it removes)."""
    return (t_graph - t_fused) - b_est


def residual_matches_model(t_graph: float, t_fused: float, b_est: float,
                           relative_tol: float = 0.02) -> tuple[bool, float]:
    """Two-sided: |S| ≤ relative_tol · t_graph."""
    s = residual_term(t_graph, t_fused, b_est)
    return abs(s) <= relative_tol * t_graph, s


def relative_delta_matches(measured: float, analytic: float, relative_tol: float) -> bool:
    """Two-sided: |measured − analytic| ≤ relative_tol · analytic."""
    if analytic <= 0 or relative_tol < 0:
        return False
    return abs(measured - analytic) <= relative_tol * analytic


def sign_corroborated(wall_gap: float, tau_gap: float, noise_us: float = 5.0) -> str:
    """PASS when both gaps are outside the noise band and agree in sign, FAIL
    when they disagree, INDETERMINATE when either is inside the band."""
    if abs(wall_gap) <= noise_us or abs(tau_gap) <= noise_us:
        return "INDETERMINATE"
    return "PASS" if (wall_gap > 0) == (tau_gap > 0) else "FAIL"


def f4_delta_detectable(analytic_delta: float, total_unfused: float, total_fused: float,
                        resolution_frac: float = 0.05) -> bool:
    """The F4 delta gate applies only when the analytic delta is at least
    ``resolution_frac`` of the smaller variant total."""
    smaller = min(total_unfused, total_fused)
    if smaller <= 0:
        return False
    return analytic_delta >= resolution_frac * smaller


def bootstrap_s_ci(graph: list[float], fused: list[float], elim_frac: float,
                   n_resamples: int = 10000, seed: int = 42,
                   alpha: float = 0.05) -> tuple[float, float] | None:
    """Percentile interval of S = t_graph·(1 − elim_frac) − t_fused over
    resamples of both medians (B is linear in t_graph, so S follows exactly).
    Deterministic for a given seed; within-run resampling uncertainty only."""
    if not graph or not fused:
        return None
    rng = np.random.default_rng(seed)
    g = np.asarray(graph, dtype=np.float64)
    f = np.asarray(fused, dtype=np.float64)
    gm = np.median(g[rng.integers(0, g.size, (n_resamples, g.size))], axis=1)
    fm = np.median(f[rng.integers(0, f.size, (n_resamples, f.size))], axis=1)
    s = np.sort(gm * (1.0 - elim_frac) - fm)
    lo = s[int((alpha / 2) * n_resamples)]
    hi = s[int((1 - alpha / 2) * n_resamples) - 1]
    return float(lo), float(hi)


def _usable(samples) -> list[float]:
    out = []
    for v in samples or []:
        try:
            x = float(v)
        except (TypeError, ValueError):
            continue
        if math.isfinite(x) and x > 0.001:
            out.append(x)
    return out


def _counter_cell(traffic: dict, label: str) -> tuple[float, float]:
    """(HBM bytes, τ µs) per call of a rocprof workload; zeros if missing."""
    w = traffic.get(label) or {}
    try:
        total = float(w.get("traffic_bytes") or 0.0)
        tau = float(w.get("call_us") or 0.0)
    except (TypeError, ValueError):
        return 0.0, 0.0
    if not (math.isfinite(total) and math.isfinite(tau)):
        return 0.0, 0.0
    return total, tau


def validate(bench: dict, traffic: dict, min_timing_samples: int = 30,
             f4_delta_tol: float = 0.5, allow_missing_counters: bool = False,
             hypotheses: str = "report") -> tuple[Checks, list[str]]:
    """Run every check; returns the registry and the report's lines."""
    if hypotheses not in ("report", "gate"):
        raise ValueError("hypotheses must be 'report' or 'gate'")
    decomp = bench.get("decomposition") or {}
    checks = Checks()
    rep = ["# DecodeBench validation report (MI355X)", ""]

    # ---- G0 ----
    rep += ["## Check (G0): data completeness", "",
            f"Every expected config needs >= {min_timing_samples} usable trials per variant "
            "and counter bytes and kernel time for the fused call and the unfused chain. "
            "A missing cell is a FAIL.", ""]
    med, samp = {}, {}
    for cfg, _ in EXPECTED:
        d = decomp.get(cfg) or {}
        ok_all = True
        for v in VARIANTS:
            vals = _usable((d.get("samples_us") or {}).get(v))
            label = f"{cfg}/{v}"
            if len(vals) < min_timing_samples:
                ok_all = False
                detail = f"{len(vals)} usable trials; require >= {min_timing_samples}"
                checks.add("G0", label, "FAIL", detail)
                rep.append(f"- {label}: **FAIL** ({detail})")
                continue
            med[(cfg, v)] = statistics.median(vals)
            samp[(cfg, v)] = vals
            checks.add("G0", label, "PASS", f"n={len(vals)}")
        for suffix, what in (("", "fused"), ("_unfused", "unfused")):
            total, tau = _counter_cell(traffic, cfg + suffix)
            label = f"counters {cfg}/{what}"
            if total > 0 and tau > 0:
                checks.add("G0", label, "PASS")
            else:
                missing = [m for m, bad in (("bytes", total <= 0), ("kernel time", tau <= 0))
                           if bad]
                status = "WARN" if allow_missing_counters else "FAIL"
                detail = "no " + " + ".join(missing)
                checks.add("G0", label, status, detail)
                rep.append(f"- {label}: **{status}** ({detail})")
        if ok_all:
            rep.append(f"- {cfg}: timing complete")
    rep.append("")

    def m(cfg, v):
        return med.get((cfg, v), 0.0)

    # ---- G1 ----
    rep += ["## Check (G1): fused output vs the unfused torch stages", "",
            "| Config | max abs | rel-L2 | Status |", "|---|---|---|---|"]
    for cfg, _ in EXPECTED:
        fc = (decomp.get(cfg) or {}).get("fused_check")
        if not fc:
            checks.add("G1", cfg, "FAIL", "no correctness record")
            rep.append(f"| {cfg} | — | — | FAIL (no record) |")
            continue
        st = checks.add("G1", cfg, "PASS" if fc.get("ok") else "FAIL",
                        f"max_abs={fc.get('max_abs')}")
        rep.append(f"| {cfg} | {fc.get('max_abs', float('nan')):.3e} | "
                   f"{fc.get('rel_l2', float('nan')):.3e} | {st} |")
    rep.append("")

    # ---- (a) ----
    rep += ["## Check (a): t_graph − t_fused = B + S, τ corroboration", "",
            "S is the unexplained residual (its 95% bootstrap interval resamples both "
            "medians, 10k draws, fixed seed). τ_u − τ_f is the per-call kernel-time gap "
            "from rocprofv3; it must agree in sign with the wall-clock gap outside a 5 µs "
            "band, inside which the check is INDETERMINATE.", "",
            "| Config | t_graph | t_fused | gap | B | S | S 95% CI | τ_u − τ_f | Status |",
            "|---|---|---|---|---|---|---|---|---|"]
    s_terms = {}
    for cfg, _ in EXPECTED:
        d = decomp.get(cfg) or {}
        tg, tf = m(cfg, "graph"), m(cfg, "fused")
        _, tau_u = _counter_cell(traffic, cfg + "_unfused")
        _, tau_f = _counter_cell(traffic, cfg)
        if not (tg > 0 and tf > 0 and tau_u > 0 and tau_f > 0):
            continue  # already a G0 failure
        total, elim = d.get("total_bytes") or 0, d.get("eliminable_bytes") or 0
        b_est = elim / (total / tg) if total > 0 else 0.0
        s_val = residual_term(tg, tf, b_est)
        s_terms[cfg] = (b_est, s_val)
        ci = bootstrap_s_ci(samp[(cfg, "graph")], samp[(cfg, "fused")],
                            elim / total if total > 0 else 0.0)
        gap, tau_gap = tg - tf, tau_u - tau_f
        st = checks.add("a", cfg, sign_corroborated(gap, tau_gap),
                        f"wall gap {gap:.2f} us vs tau gap {tau_gap:.2f} us")
        ci_txt = f"[{ci[0]:.2f}, {ci[1]:.2f}]" if ci else "n/a"
        rep.append(f"| {cfg} | {tg:.2f} | {tf:.2f} | {gap:.2f} | {b_est:.2f} | {s_val:.2f} | "
                   f"{ci_txt} | {tau_gap:.2f} | {st} |")
    rep.append("")

    # ---- (b) ----
    rep += ["## Check (b): analytic vs counter HBM bytes", "",
            "F1/F2: the byte model's total within ±20% of each variant's counter bytes. "
            f"F4: the eliminated delta within ±{f4_delta_tol:.0%} of the analytic delta "
            "(eliminable bytes minus the split partial records the fused call adds), only "
            "when that delta is >= 5% of the smaller total; otherwise INDETERMINATE. The "
            "decode-layer rows are diagnostics.", "",
            "| Config | Variant | Analytic (MB) | Counters (MB) | Ratio | Status |",
            "|---|---|---|---|---|---|"]
    for cfg, fam in EXPECTED:
        d = decomp.get(cfg) or {}
        analytic = float(d.get("total_bytes") or 0)
        tot = {v: _counter_cell(traffic, cfg + sfx)[0]
               for v, sfx in (("unfused", "_unfused"), ("fused", ""))}
        if fam == "f4":
            if tot["unfused"] > 0 and tot["fused"] > 0 and analytic > 0:
                a_delta = float(d.get("eliminable_bytes") or 0) - float(
                    d.get("fused_extra_bytes") or 0)
                m_delta = tot["unfused"] - tot["fused"]
                if f4_delta_detectable(a_delta, tot["unfused"], tot["fused"]):
                    ok = relative_delta_matches(m_delta, a_delta, f4_delta_tol)
                    st = checks.add("b", f"{cfg}/delta", "PASS" if ok else "FAIL",
                                    f"measured {m_delta / 1e6:.2f} MB vs analytic "
                                    f"{a_delta / 1e6:.2f} MB")
                else:
                    st = checks.add("b", f"{cfg}/delta", "INDETERMINATE",
                                    "analytic delta below 5% of the smaller total")
                rep.append(f"| {cfg} | delta (unfused − fused) | {a_delta / 1e6:.2f} | "
                           f"{m_delta / 1e6:.2f} | "
                           f"{m_delta / a_delta if a_delta else float('nan'):.2f} | {st} |")
            for v in ("unfused", "fused"):
                if tot[v] > 0:
                    rep.append(f"| {cfg} | {v} (diagnostic) | {analytic / 1e6:.2f} | "
                               f"{tot[v] / 1e6:.2f} | {analytic / tot[v]:.3f} | — |")
            continue
        for v in ("unfused", "fused"):
            if tot[v] <= 0 or analytic <= 0:
                continue  # already a G0 failure
            ratio = analytic / tot[v]
            if fam == "layer":
                rep.append(f"| {cfg} | {v} (diagnostic) | {analytic / 1e6:.2f} | "
                           f"{tot[v] / 1e6:.2f} | {ratio:.3f} | — |")
                continue
            st = checks.add("b", f"{cfg}/{v}", "PASS" if abs(ratio - 1.0) <= 0.20 else "FAIL",
                            f"ratio={ratio:.3f}")
            rep.append(f"| {cfg} | {v} | {analytic / 1e6:.2f} | {tot[v] / 1e6:.2f} | "
                       f"{ratio:.3f} | {st} |")
    rep.append("")

    # ---- (c) ----
    rep += ["## Check (c): graph replay at least as fast as stream launches", "",
            "Δ_launch = t_stream − t_graph ≥ −max(0.5%·t_graph, 2 µs).", "",
            "| Config | t_stream | t_graph | Δ_launch | Status |", "|---|---|---|---|---|"]
    for cfg, _ in EXPECTED:
        ts, tg = m(cfg, "stream"), m(cfg, "graph")
        if not (ts > 0 and tg > 0):
            continue
        dl = ts - tg
        floor = max(0.005 * tg, 2.0)
        st = checks.add("c", cfg, "PASS" if dl >= -floor else "FAIL",
                        f"delta {dl:.2f} us (noise floor {floor:.2f} us)")
        rep.append(f"| {cfg} | {ts:.2f} | {tg:.2f} | {dl:.2f} | {st} |")
    rep.append("")

    # ---- (H) ----
    rep += [f"## Check (H): the reference's v2 hypotheses ({hypotheses})", "",
            "H1-v2 (F1/F2): t_fused ≥ t_graph − max(0.5%·t_graph, 2 µs) and "
            "S ≤ max(1%·t_graph, 3 µs). H2-v2 (F4): t_fused < t_graph, S > 0, S > B. "
            + ("Outcomes are recorded, not gated: the hypotheses were registered for the "
               "reference's kernels on its GPU." if hypotheses == "report" else
               "Gating, as in the reference."), "",
            "| Hypothesis | Config | gap | B | S | Outcome |", "|---|---|---|---|---|---|"]
    for cfg, fam in EXPECTED:
        if fam not in ("f1", "f2", "f4") or cfg not in s_terms:
            continue
        tg, tf = m(cfg, "graph"), m(cfg, "fused")
        b_est, s_val = s_terms[cfg]
        if fam == "f4":
            hyp = "H2-v2"
            conds = {"t_fused<t_graph": tf < tg, "S>0": s_val > 0, "S>B": s_val > b_est}
        else:
            hyp = "H1-v2"
            conds = {"no fused win": tf >= tg - max(0.005 * tg, 2.0),
                     "S<=tol": s_val <= max(0.01 * tg, 3.0)}
        held = all(conds.values())
        failed = [k for k, v in conds.items() if not v]
        detail = "all conditions hold" if held else "failed: " + ", ".join(failed)
        if hypotheses == "gate":
            outcome = checks.add("H", f"{hyp}/{cfg}", "PASS" if held else "FAIL", detail)
        else:
            outcome = "supported" if held else f"refuted ({', '.join(failed)})"
        rep.append(f"| {hyp} | {cfg} | {tg - tf:.2f} | {b_est:.2f} | {s_val:.2f} | "
                   f"{outcome} |")
    rep.append("")

    # ---- summary ----
    c = checks.counts()
    rep += ["---", "", "## Summary", "",
            f"- PASS: {c['PASS']}",
            f"- INDETERMINATE: {c['INDETERMINATE']} (no claim either way; neither a pass "
            "nor a gate)",
            f"- WARN: {c['WARN']} (never a pass)",
            f"- FAIL: {c['FAIL']}",
            f"- **Overall: {checks.overall()}**"]
    if c["FAIL"]:
        rep += ["", "### Failing checks"]
        rep += [f"- [{r['section']}] {r['label']}: {r['detail']}"
                for r in checks.records if r["status"] == "FAIL"]
    return checks, rep


def _load_json(path: str) -> dict:
    try:
        text = Path(path).read_text()
    except OSError:
        return {}
    try:
        return json.loads(text)
    except ValueError:
        pass
    # bench.py's stdout captured with its log lines: the last JSON line
    for line in reversed(text.strip().splitlines()):
        if line.strip().startswith("{"):
            try:
                return json.loads(line)
            except ValueError:
                continue
    return {}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="DecodeBench validation report (fail-closed)")
    ap.add_argument("--bench", required=True, help="bench.py output (JSON line)")
    ap.add_argument("--traffic", required=True,
                    help="decodebench_amd.rocprof --json summary with the unfused rows")
    ap.add_argument("--kernel-trace", default=None,
                    help="decodebench_amd.rocprof --json summary of a --kernel-trace run; its "
                         "per-call kernel time fills in workloads the traffic summary has no "
                         "time for")
    ap.add_argument("--output", default="validation_report.md")
    ap.add_argument("--min-timing-samples", type=int, default=30)
    ap.add_argument("--f4-delta-tol", type=float, default=0.5)
    ap.add_argument("--allow-missing-counters", action="store_true",
                    help="missing counter data is a WARN instead of a FAIL (dev runs only)")
    ap.add_argument("--hypotheses", choices=("report", "gate"), default="report")
    args = ap.parse_args(argv)
    if not 0 <= args.f4_delta_tol < 1:
        ap.error("--f4-delta-tol must be in [0, 1)")
    if args.min_timing_samples <= 0:
        ap.error("--min-timing-samples must be positive")
    bench = _load_json(args.bench)
    traffic = _load_json(args.traffic).get("workloads", {})
    if args.kernel_trace:
        for label, w in _load_json(args.kernel_trace).get("workloads", {}).items():
            cell = traffic.setdefault(label, {})
            if cell.get("call_us") is None and w.get("call_us") is not None:
                cell["call_us"] = w["call_us"]
    checks, rep = validate(bench, traffic, args.min_timing_samples, args.f4_delta_tol,
                           args.allow_missing_counters, args.hypotheses)
    text = "\n".join(rep) + "\n"
    out = Path(args.output)
    if out.parent != Path(""):
        out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(text)
    print(text)
    print(f"Report written to {out}")
    c = checks.counts()
    return 0 if c["FAIL"] == 0 and c["WARN"] == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
