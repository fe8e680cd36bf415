"""Host API (byte model, verdict, report, stats, bindings, timing arguments).

The expected numbers and message fragments are the reference's own test
values: tests/test_bytes_model.py:3-38, tests/test_cost_model.py:4-50,
tests/test_verdict.py:4-84, tests/test_report.py:7-82, tests/test_stats.py:5-42,
tests/test_sequence_bindings.py:6-60 and tests/test_timing_inputs.py:8-22 of
the reference repository.  The cost-model numbers are reproduced through
StageTrace lists of the same unfused pipelines (model/cost_model.py:18-45).
"""

import csv
import math
import os

import numpy as np
import pytest

from decodebench_amd.bytes_model import StageTrace, eliminable_bytes, total_bytes
from decodebench_amd.report import Report
from decodebench_amd.sequence import Sequence
from decodebench_amd.stats import bootstrap_diff_ci, summarize
from decodebench_amd.timing import (cache_defeat_replicas, n_weight_replicas,
                                    time_callable)
from decodebench_amd.verdict import compute_verdict

F1_4096 = [
    StageTrace("rmsnorm", reads=[8192, 8192], write=8192, is_final=False),
    StageTrace("gemv", reads=[33554432, 8192], write=8192, is_final=True),
]


# ----------------------------------------------------------- bytes model
def test_bytes_model_golden_f1():
    assert total_bytes(F1_4096) == 33595392
    assert eliminable_bytes(F1_4096) == 16384


def test_single_final_stage():
    t = [StageTrace("gemv", reads=[33554432, 8192], write=8192, is_final=True)]
    assert total_bytes(t) == 33570816
    assert eliminable_bytes(t) == 0


def test_fanout_counts_one_read_per_consumer():
    t = [StageTrace("producer", reads=[64], write=128, consumers=2),
         StageTrace("final", reads=[128, 128], write=32, is_final=True, consumers=0)]
    assert total_bytes(t) == 480
    assert eliminable_bytes(t) == 384


def test_invalid_trace_metadata():
    with pytest.raises(ValueError, match="non-negative"):
        StageTrace("bad", reads=[-1], write=1)
    with pytest.raises(ValueError, match="consumers"):
        StageTrace("bad", reads=[], write=1, consumers=-1)
    with pytest.raises(ValueError, match="at least one consumer"):
        StageTrace("dead", reads=[], write=1, consumers=0)


def _cost_traces(d, b=1, l=1024, hd=128):
    ff = {2048: 8192, 4096: 11008}[d]
    h = d // hd
    f1 = [StageTrace("rmsnorm", [2 * b * d, 2 * d], 2 * b * d),
          StageTrace("gemv", [2 * d * d, 2 * b * d], 2 * b * d, is_final=True)]
    f2 = [StageTrace("gate", [2 * b * d, 2 * ff * d], 2 * b * ff),
          StageTrace("up", [2 * b * d, 2 * ff * d], 2 * b * ff),
          StageTrace("swiglu", [2 * b * ff, 2 * b * ff], 2 * b * ff, is_final=True)]
    f4 = [StageTrace("scores", [2 * b * d, 2 * b * h * l * hd], 4 * b * h * l),
          StageTrace("softmax", [4 * b * h * l], 4 * b * h * l),
          StageTrace("weighted_v", [4 * b * h * l, 2 * b * h * l * hd], 2 * b * d,
                     is_final=True)]
    return {"F1": f1, "F2": f2, "F4": f4}


@pytest.mark.parametrize("d,expect", [
    (4096, {"F1": (33595392, 16384, 0.000488, "low"),
            "F2": (180481536, 88064, 0.000488, "low"),
            "F4": (17317888, 524288, 0.030274, "material")}),
    (2048, {"F1": (8409088, 8192, 0.000974, "low"),
            "F2": (67198976, 65536, 0.000975, "low"),
            "F4": (8658944, 262144, 0.030274, "material")}),
])
def test_cost_model_numbers(d, expect):
    for name, traces in _cost_traces(d).items():
        tot, elim = total_bytes(traces), eliminable_bytes(traces)
        ratio = elim / tot
        e_tot, e_elim, e_ratio, e_label = expect[name]
        assert (tot, elim) == (e_tot, e_elim)
        assert round(ratio, 6) == e_ratio
        label = "material" if ratio >= 0.01 else "low"
        assert label == e_label


# ---------------------------------------------------------------- verdict
def test_verdict_low_byte_opportunity():
    v = compute_verdict(t_stream=20.0, t_graph=16.0, total_bytes=33595392,
                        eliminable_bytes=16384, byte_threshold=0.01)
    assert v.bound == "low-byte-opportunity"
    assert v.delta_launch == 4.0
    assert abs(v.b_bytes_est - (16384 / (33595392 / 16.0))) < 1e-6
    assert v.b_ceiling == v.b_bytes_est
    assert v.dominant == "launch"
    r = v.render()
    assert "CUDA Graphs eliminate 4.00 us here" in r
    assert "Eliminable intermediate bytes correspond to" in r
    assert "NOT a strict bound" in r
    assert "Verdict: LOW-BYTE-OPPORTUNITY" in r


def test_verdict_threshold_respected():
    v = compute_verdict(t_stream=20, t_graph=16, total_bytes=1000000,
                        eliminable_bytes=30000, byte_threshold=0.01)
    assert v.bound == "material-byte-opportunity"
    v = compute_verdict(t_stream=20, t_graph=16, total_bytes=1000000,
                        eliminable_bytes=30000, byte_threshold=0.05)
    assert v.bound == "low-byte-opportunity"


def test_verdict_f4_ratio_regression():
    v = compute_verdict(t_stream=20.0, t_graph=16.0, total_bytes=17317888,
                        eliminable_bytes=524288, byte_threshold=0.01)
    assert v.bound == "material-byte-opportunity"
    assert v.dominant == "launch"
    assert "Caution: measured launch savings exceed the byte estimate" in v.render()


def test_verdict_invalid_inputs():
    with pytest.raises(ValueError, match="t_graph must be positive"):
        compute_verdict(t_stream=10.0, t_graph=0.0, total_bytes=100, eliminable_bytes=10)
    with pytest.raises(ValueError, match="t_fused must be finite and positive"):
        compute_verdict(t_stream=10.0, t_graph=8.0, total_bytes=100, eliminable_bytes=10,
                        t_fused=-1.0)
    with pytest.raises(ValueError, match="must be finite"):
        compute_verdict(t_stream=float("nan"), t_graph=8.0, total_bytes=100,
                        eliminable_bytes=10)
    with pytest.raises(ValueError, match="byte_threshold"):
        compute_verdict(t_stream=10.0, t_graph=8.0, total_bytes=100, eliminable_bytes=10,
                        byte_threshold=-0.1)
    with pytest.raises(ValueError, match="ordered bounds"):
        compute_verdict(t_stream=10.0, t_graph=8.0, total_bytes=100, eliminable_bytes=10,
                        delta_launch_ci=(2.0, 1.0))
    with pytest.raises(ValueError, match="eliminable_bytes"):
        compute_verdict(t_stream=10.0, t_graph=8.0, total_bytes=100, eliminable_bytes=101)


def test_verdict_with_fused():
    v = compute_verdict(t_stream=20.0, t_graph=16.0, total_bytes=33595392,
                        eliminable_bytes=16384, byte_threshold=0.01, t_fused=12.0)
    assert abs(v.residual_us - 3.9922) < 1e-3
    r = v.render()
    assert "Measured fused latency: 12.00 us" in r
    assert "Decomposition:" in r
    assert "unexplained residual 3.99 us" in r


def test_verdict_ci_spanning_zero_is_reported():
    v = compute_verdict(t_stream=10.0, t_graph=9.9, total_bytes=100, eliminable_bytes=1,
                        delta_launch_ci=(-0.5, 0.7))
    assert "statistically indistinguishable from zero" in v.render()


# ----------------------------------------------------------------- report
def test_report_success(tmp_path):
    rep = Report(name="test_f1", stream_us=[20.0] * 30, graph_us=[16.0] * 30,
                 traces=F1_4096, byte_threshold=0.01)
    v = rep.verdict()
    assert v.bound == "low-byte-opportunity"
    assert v.delta_launch_ci is not None
    path = tmp_path / "r.csv"
    rep.to_csv(str(path))
    assert os.path.exists(path)
    rows = list(csv.reader(open(path)))
    assert rows[0] == ["name", "variant", "trial", "us_per_invocation"]
    assert len(rows) == 61
    assert rows[1] == ["test_f1", "stream", "0", "20.0"]
    assert rows[31] == ["test_f1", "graph", "0", "16.0"]


def test_report_with_fused(tmp_path):
    rep = Report(name="test_f1", stream_us=[20.0] * 30, graph_us=[16.0] * 30,
                 traces=F1_4096, fused_us=[12.0] * 30, byte_threshold=0.01)
    v = rep.verdict()
    assert v.t_fused == 12.0
    assert v.residual_us is not None
    path = tmp_path / "r.csv"
    rep.to_csv(str(path))
    rows = list(csv.reader(open(path)))
    assert len(rows) == 91
    assert rows[61] == ["test_f1", "fused", "0", "12.0"]


def test_report_capture_failure():
    rep = Report(name="test_fail", stream_us=[20.0], graph_us=[], traces=[],
                 graph_ok=False, graph_skip_reason="Host sync detected")
    with pytest.raises(RuntimeError, match="capture failed for 'test_fail': Host sync detected"):
        rep.verdict()


# ------------------------------------------------------------------ stats
def test_summarize():
    s = summarize([10, 12, 11, 13, 100])
    assert (s.median, s.p25, s.p75, s.iqr, s.n) == (12.0, 11.0, 13.0, 2.0, 5)
    with pytest.raises(ValueError, match="requires at least one sample"):
        summarize([])
    with pytest.raises(ValueError, match="finite"):
        summarize([1.0, np.nan])
    with pytest.raises(ValueError, match="one-dimensional"):
        summarize([[1.0, 2.0]])


def test_bootstrap_diff_ci():
    rng = np.random.default_rng(42)
    a = rng.normal(100, 2, 200)
    b = rng.normal(90, 2, 200)
    lo, hi, point = bootstrap_diff_ci(a, b, n_resamples=1000, seed=42)
    assert lo > 0 and lo < point < hi
    a2 = rng.normal(100, 2, 200)
    lo2, hi2, _ = bootstrap_diff_ci(a, a2, n_resamples=1000, seed=42)
    assert lo2 < 0 < hi2
    with pytest.raises(ValueError, match="requires non-empty samples"):
        bootstrap_diff_ci([], [1.0])
    with pytest.raises(ValueError, match="finite"):
        bootstrap_diff_ci([np.inf], [1.0])
    with pytest.raises(ValueError, match="n_resamples"):
        bootstrap_diff_ci([1.0], [1.0], n_resamples=0)
    with pytest.raises(ValueError, match="ci must"):
        bootstrap_diff_ci([1.0], [1.0], ci=1.0)
    with pytest.raises(ValueError, match="one-dimensional"):
        bootstrap_diff_ci([[1.0]], [1.0])


def test_bootstrap_constant_samples_are_exact():
    lo, hi, point = bootstrap_diff_ci([5.0] * 7, [2.0] * 9, n_resamples=50)
    assert lo == hi == point == 3.0


# --------------------------------------------------------------- bindings
def test_named_fanin_and_fanout_consumer_counts():
    seq = Sequence("dag")

    @seq.stage
    def source(x):
        return x

    @seq.stage
    def left(source):
        return source

    @seq.stage
    def right(source):
        return source

    @seq.stage
    def merge(left, right):
        return left

    assert seq._dependency_consumer_counts({"x": object()}) == {
        "source": 2, "left": 1, "right": 1}


def test_unconsumed_output_fails_before_execution():
    seq = Sequence("bad")

    @seq.stage
    def first(x):
        return x

    @seq.stage
    def second(x):
        return x

    with pytest.raises(ValueError, match="first.*never consumed"):
        seq._dependency_consumer_counts({"x": object()})


def test_missing_binding_is_a_key_error():
    seq = Sequence("missing")

    @seq.stage
    def only(x, y):
        return x

    with pytest.raises(KeyError, match="parameter 'y' not found"):
        seq._dependency_consumer_counts({"x": object()})


def test_unsupported_signature_and_duplicate_names_fail_registration():
    seq = Sequence("signatures")
    with pytest.raises(TypeError, match="plain positional"):
        @seq.stage
        def bad(*args):
            return args

    def same(x):
        return x

    seq.stage(same)
    with pytest.raises(ValueError, match="duplicate stage"):
        seq.stage(same)


def test_bind_args_precedence():
    seq = Sequence("prec")

    @seq.stage
    def a(x):
        return x

    @seq.stage
    def b(prev, a, w):
        return prev

    st = seq._stages[1]
    args = seq._bind_args(st, 1, "PREV", {"w": "W", "a": "INPUT_A"}, {"a": "OUT_A"})
    # stage output beats the inputs dict; first param falls back to previous
    assert args == ["PREV", "OUT_A", "W"]


def test_empty_sequence_rejected():
    with pytest.raises(ValueError, match="no stages"):
        Sequence("empty")._run_once({})


# ------------------------------------------------------------------ timing
def test_replica_sizing_validation():
    assert n_weight_replicas(1024, l2_bytes=48 * 1024 * 1024) == 8
    assert n_weight_replicas(10 ** 9, l2_bytes=4 * 1024 * 1024) == 4
    with pytest.raises(ValueError, match="weight_bytes"):
        n_weight_replicas(0, l2_bytes=1024)
    with pytest.raises(ValueError, match="l2_bytes"):
        n_weight_replicas(1024, l2_bytes=-1)


def test_cache_defeat_replicas_cover_twice_the_caches():
    cache = 288 * 1024 * 1024
    for nbytes in (33_554_432, 50_331_648, 234_881_024, 134_217_728):
        n = cache_defeat_replicas(nbytes, cache=cache)
        assert n * nbytes >= 2 * cache
        assert (n - 1) * nbytes < 2 * cache or n == 2


def test_timing_arguments_fail_before_torch_is_needed():
    with pytest.raises(ValueError, match="trials"):
        time_callable(lambda: None, trials=0)
    with pytest.raises(ValueError, match="target_ms"):
        time_callable(lambda: None, target_ms=math.nan)
    with pytest.raises(ValueError, match="warmup"):
        time_callable(lambda: None, warmup=-1)


# ------------------------------------------------------- profile schedule
def test_rotation_plan_splits_trials_and_rotates_variants():
    """The reference's measurement procedure (sequence.py:276-291): up to
    three rounds, the remainder to the first rounds, round r starting at
    variant r, full warmup only in the first round."""
    from decodebench_amd.sequence import _rotation_plan

    plan = _rotation_plan(["stream", "graph", "fused"], 7, 50)
    assert plan == [("stream", 3, 50), ("graph", 3, 50), ("fused", 3, 50),
                    ("graph", 2, 5), ("fused", 2, 5), ("stream", 2, 5),
                    ("fused", 2, 5), ("stream", 2, 5), ("graph", 2, 5)]
    two = _rotation_plan(["stream", "graph"], 30, 3)
    assert [n for _, n, _ in two] == [10] * 6
    assert [v for v, _, _ in two] == ["stream", "graph", "graph", "stream", "stream", "graph"]
    assert [w for _, _, w in two] == [3] * 6                 # min(3, 5) after round 0
    assert _rotation_plan(["stream", "graph"], 2, 9) == [
        ("stream", 1, 9), ("graph", 1, 9), ("graph", 1, 5), ("stream", 1, 5)]
    for trials in range(1, 12):
        plan = _rotation_plan(["a", "b", "c"], trials, 7)
        for v in "abc":
            assert sum(n for name, n, _ in plan if name == v) == trials


class _FakeGraph:
    def __init__(self, body, ok=True):
        self.body, self.ok, self.reason = body, ok, None if ok else "capture refused"

    def replay(self):
        self.body()


def _profile_with_fakes(monkeypatch, ok=True, fused=None, n_replicas=3):
    """profile() on the CPU: captures and timing replaced by recorders."""
    import torch

    from decodebench_amd import graph, timing

    captured, timed = [], []

    def fake_capture(fn, pool=None):
        captured.append(pool)
        return _FakeGraph(fn, ok=ok or len(captured) < 2)

    def fake_time(body, trials, target_ms, warmup):
        for _ in range(trials):
            body()
        timed.append((body, trials, warmup))
        return [float(len(timed))] * trials

    monkeypatch.setattr(graph, "try_capture", fake_capture)
    monkeypatch.setattr(timing, "time_callable", fake_time)
    monkeypatch.setattr(torch.cuda, "graph_pool_handle", lambda: "pool")
    seen = []
    seq = Sequence("fake")

    @seq.stage
    def double(x):
        seen.append(int(x[0]))
        return x * 2

    replicas = [{"x": torch.full((4,), float(i))} for i in range(n_replicas)]
    rep = seq.profile(replicas[0], trials=7, warmup=4, input_replicas=replicas, fused=fused)
    return rep, captured, timed, seen


def test_profile_rotates_replicas_and_variants(monkeypatch):
    fused_seen = []

    def fused(inp):
        fused_seen.append(int(inp["x"][0]))
        return inp["x"] * 2

    rep, captured, timed, seen = _profile_with_fakes(monkeypatch, fused=fused)
    assert captured == ["pool"] * 3                      # one graph per replica, one pool
    assert [(t, w) for _, t, w in timed] == [(3, 4)] * 3 + [(2, 4)] * 6
    assert len(rep.stream_us) == len(rep.graph_us) == len(rep.fused_us) == 7
    # trace (replica 0), the fused check (replica 0), then every timed call
    # walks the replicas in order: stream and graph share the stage body.
    assert seen[:2] == [0, 0] and fused_seen[0] == 0
    assert fused_seen[1:] == [i % 3 for i in range(7)]


def test_profile_without_graphs_reports_stream_times(monkeypatch):
    rep, captured, timed, seen = _profile_with_fakes(monkeypatch, ok=False)
    assert len(captured) == 2                            # stops at the failing capture
    assert [(t, w) for _, t, w in timed] == [(7, 4)]
    assert rep.graph_ok is False and rep.graph_skip_reason == "capture refused"
    assert rep.stream_us == rep.graph_us
