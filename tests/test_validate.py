"""The fail-closed validation report (decodebench_amd.validate).

The first tests restate what the reference pins for its analysis gate
(tests/test_validation_analysis.py:20-114 over
validation/analysis/compare.py and parse_ncu.py): two-sided residual and
delta gates, sign corroboration with a 5 us indeterminate band, the F4
detectability floor, WARN never passing, INDETERMINATE neither passing nor
gating, a deterministic bootstrap interval bracketing its point estimate, and
failing closed on empty inputs.  The rest run the report on synthetic
bench/rocprof data.
"""

import json
import statistics
import subprocess
import sys

import pytest

from decodebench_amd import validate as V


def test_residual_gate_is_two_sided():
    assert V.residual_matches_model(100.0, 99.0, 1.0)[0]
    assert not V.residual_matches_model(100.0, 80.0, 1.0)[0]
    assert not V.residual_matches_model(100.0, 120.0, 1.0)[0]


def test_residual_term_sign_convention():
    assert V.residual_term(384.0, 318.0, 11.6) > 0
    assert V.residual_term(220.0, 253.0, 0.03) < 0


def test_sign_corroboration_requires_agreement_outside_noise():
    assert V.sign_corroborated(66.0, 136.0) == "PASS"
    assert V.sign_corroborated(-102.0, -154.0) == "PASS"
    assert V.sign_corroborated(66.0, -136.0) == "FAIL"
    assert V.sign_corroborated(-14.0, -2.0) == "INDETERMINATE"
    assert V.sign_corroborated(3.0, -136.0) == "INDETERMINATE"
    assert V.sign_corroborated(2.0, 1.0) == "INDETERMINATE"


def test_f4_delta_detectability_floor():
    assert not V.f4_delta_detectable(1.0e6, 97.4e6, 90.4e6)
    assert V.f4_delta_detectable(6.0e6, 97.4e6, 90.4e6)
    assert not V.f4_delta_detectable(6.0e6, 0.0, 90.4e6)


def test_delta_gate_is_two_sided():
    assert V.relative_delta_matches(1.2, 1.0, 0.5)
    assert not V.relative_delta_matches(2.0, 1.0, 0.5)
    assert not V.relative_delta_matches(0.4, 1.0, 0.5)


def test_warnings_are_not_a_valid_pass():
    checks = V.Checks()
    checks.add("dev", "missing", "WARN")
    assert checks.overall() == "INCOMPLETE"


def test_bootstrap_s_ci_deterministic_and_brackets_point_estimate():
    graph = [100.0 + 0.1 * i for i in range(30)]
    fused = [90.0 + 0.1 * i for i in range(30)]
    ci1 = V.bootstrap_s_ci(graph, fused, elim_frac=0.03)
    ci2 = V.bootstrap_s_ci(graph, fused, elim_frac=0.03)
    assert ci1 == ci2
    lo, hi = ci1
    point = statistics.median(graph) * 0.97 - statistics.median(fused)
    assert lo <= point <= hi
    assert V.bootstrap_s_ci([], fused, 0.03) is None


def test_indeterminate_neither_passes_nor_gates():
    checks = V.Checks()
    checks.add("a", "tie-cell", "INDETERMINATE")
    checks.add("b", "real-pass", "PASS")
    c = checks.counts()
    assert c["INDETERMINATE"] == 1 and c["PASS"] == 1
    assert checks.overall() == "PASS"


def test_fails_closed_on_empty_inputs(tmp_path):
    bench, traffic, report = tmp_path / "b.json", tmp_path / "t.json", tmp_path / "r.md"
    bench.write_text("{}\n")
    traffic.write_text(json.dumps({"workloads": {}}))
    proc = subprocess.run([sys.executable, "-m", "decodebench_amd.validate", "--bench",
                           str(bench), "--traffic", str(traffic), "--output", str(report)],
                          text=True, capture_output=True)
    assert proc.returncode != 0
    assert "Overall: FAIL" in report.read_text()


# ------------------------------------------------------------ synthetic run
def _cell(stream, graph, fused, total, elim, extra=0):
    jitter = [0.01 * (i % 5) for i in range(30)]
    return {"total_bytes": total, "eliminable_bytes": elim, "fused_extra_bytes": extra,
            "fused_check": {"ok": True, "max_abs": 1e-3, "rel_l2": 1e-4},
            "samples_us": {"stream": [stream + j for j in jitter],
                           "graph": [graph + j for j in jitter],
                           "fused": [fused + j for j in jitter]}}


def _synthetic():
    bench = {"decomposition": {
        "f1_cfg1": _cell(56.0, 40.0, 9.0, 33_600_000, 16_384),
        "f2_cfg2": _cell(54.0, 55.0, 35.7, 235_000_000, 114_688),
        "f4_L8192": _cell(73.0, 72.0, 12.8, 37_800_000, 4_200_000, extra=1_064_960),
        "layer_cfg5": _cell(277.0, 226.0, 83.8, 474_000_000, 4_480_000),
        "layer_cfg5_fp8": _cell(864.0, 860.0, 58.1, 256_000_000, 4_480_000)}}
    traffic = {
        "f1_cfg1": {"traffic_bytes": 33_800_000, "call_us": 7.7},
        "f1_cfg1_unfused": {"traffic_bytes": 34_000_000, "call_us": 30.0},
        "f2_cfg2": {"traffic_bytes": 235_100_000, "call_us": 36.6},
        "f2_cfg2_unfused": {"traffic_bytes": 236_000_000, "call_us": 50.0},
        "f4_L8192": {"traffic_bytes": 34_300_000, "call_us": 13.2},
        "f4_L8192_unfused": {"traffic_bytes": 37_500_000, "call_us": 60.0},
        "layer_cfg5": {"traffic_bytes": 471_000_000, "call_us": 88.5},
        "layer_cfg5_unfused": {"traffic_bytes": 480_000_000, "call_us": 200.0},
        "layer_cfg5_fp8": {"traffic_bytes": 254_000_000, "call_us": 59.8},
        "layer_cfg5_fp8_unfused": {"traffic_bytes": 900_000_000, "call_us": 800.0}}
    return bench, traffic


def test_complete_synthetic_run_passes_and_records_hypotheses():
    bench, traffic = _synthetic()
    checks, rep = V.validate(bench, traffic)
    text = "\n".join(rep)
    assert checks.overall() == "PASS", [r for r in checks.records if r["status"] != "PASS"]
    # F4: analytic delta 4.2 - 1.06 MB vs measured 3.2 MB, within 50%
    assert any(r["label"] == "f4_L8192/delta" and r["status"] == "PASS"
               for r in checks.records)
    # the fused kernels win: H1-v2 is refuted for F1/F2, recorded without gating
    assert "| H1-v2 | f1_cfg1 |" in text and "refuted" in text
    assert "| H2-v2 | f4_L8192 |" in text
    # layer byte rows are diagnostics, never gated (fp8 unfused dequantises)
    assert not any(r["section"] == "b" and r["label"].startswith("layer")
                   for r in checks.records)


def test_hypotheses_gate_like_the_reference():
    bench, traffic = _synthetic()
    checks, _ = V.validate(bench, traffic, hypotheses="gate")
    failed = {r["label"] for r in checks.records if r["status"] == "FAIL"}
    assert failed == {"H1-v2/f1_cfg1", "H1-v2/f2_cfg2"}
    assert checks.overall() == "FAIL"


def test_missing_and_disagreeing_data_fail():
    bench, traffic = _synthetic()
    del traffic["f2_cfg2_unfused"]
    bench["decomposition"]["f1_cfg1"]["samples_us"]["fused"] = [9.0] * 10
    bench["decomposition"]["f4_L8192"]["fused_check"]["ok"] = False
    checks, _ = V.validate(bench, traffic)
    failed = {(r["section"], r["label"]) for r in checks.records if r["status"] == "FAIL"}
    assert ("G0", "f1_cfg1/fused") in failed
    assert ("G0", "counters f2_cfg2/unfused") in failed
    assert ("G1", "f4_L8192") in failed
    checks, _ = V.validate(bench, traffic, allow_missing_counters=True)
    assert ("G0", "counters f2_cfg2/unfused") not in {
        (r["section"], r["label"]) for r in checks.records if r["status"] == "FAIL"}
    # wall and kernel-time gaps of opposite sign
    bench, traffic = _synthetic()
    traffic["f4_L8192_unfused"]["call_us"] = 2.0
    checks, _ = V.validate(bench, traffic)
    assert any(r["section"] == "a" and r["label"] == "f4_L8192" and r["status"] == "FAIL"
               for r in checks.records)
    # graph replay slower than the stream beyond the noise floor
    bench, traffic = _synthetic()
    bench["decomposition"]["f2_cfg2"]["samples_us"]["graph"] = [60.0] * 30
    checks, _ = V.validate(bench, traffic)
    assert any(r["section"] == "c" and r["label"] == "f2_cfg2" and r["status"] == "FAIL"
               for r in checks.records)
