"""The host API on the GPU: the behaviour the reference's end-to-end tests pin
(tests/test_gpu_e2e.py:13-205), run against this build's ``Sequence``,
``try_capture``, ``time_callable`` and demos on ROCm.

Byte accounting of a traced stage, fan-out consumer counts, rejection of
aliased, strided and closure-captured tensors, replica validation, hipGraph
capture/replay and a capture that fails on a host synchronisation, the
hidden-allocation warning, event timing, the three demo verdicts, and
``profile(fused=...)`` with a matching and a mismatching fused callable.
"""

import pytest

torch = pytest.importorskip("torch")

from decodebench_amd.demos.llama_decode import build_demo  # noqa: E402
from decodebench_amd.graph import try_capture  # noqa: E402
from decodebench_amd.sequence import Sequence  # noqa: E402
from decodebench_amd.timing import n_weight_replicas, time_callable  # noqa: E402

pytestmark = pytest.mark.gpu


def test_small_weights_still_get_the_minimum_replicas():
    assert n_weight_replicas(2048, l2_bytes=64 << 20) >= 4


def test_trace_counts_the_stage_inputs_and_output():
    d = 512
    x = torch.randn(1, d, device="cuda").half()
    g = torch.randn(d, device="cuda").half()
    seq = Sequence("one_stage")

    @seq.stage
    def scale(x, g):
        return x * g

    (t,) = seq.trace({"x": x, "g": g})
    assert t.name == "scale"
    assert t.reads == [x.nbytes, g.nbytes] and t.write == x.nbytes


def test_trace_fanout_and_rejected_tensor_forms():
    x = torch.randn(32, device="cuda")
    seq = Sequence("diamond")

    @seq.stage
    def src(x):
        return x.clone()

    @seq.stage
    def a(src):
        return src * 2

    @seq.stage
    def b(src):
        return src - 1

    @seq.stage
    def join(a, b):
        return a * b

    assert seq.trace({"x": x})[0].consumers == 2

    inplace = Sequence("inplace")

    @inplace.stage
    def bump(x):
        return x.mul_(3)

    with pytest.raises(ValueError, match="aliases"):
        inplace.trace({"x": x.clone()})

    strided = Sequence("strided")

    @strided.stage
    def cp(x):
        return x.clone()

    with pytest.raises(ValueError, match="non-contiguous"):
        strided.trace({"x": torch.ones(8, 4, device="cuda").t()})

    w = torch.ones(32, device="cuda")
    closure = Sequence("closure")

    @closure.stage
    def uses_w(x):
        return x + w

    with pytest.raises(ValueError, match="captures tensor"):
        closure.trace({"x": x})


def test_replicas_must_match_replica_zero():
    with pytest.raises(ValueError, match="does not match replica 0"):
        Sequence._validate_replicas([{"x": torch.ones(4, device="cuda")},
                                     {"x": torch.ones(5, device="cuda")}])


def test_graph_capture_replays_with_new_inputs():
    x = torch.randn(1, 128, device="cuda").half()
    y = torch.zeros(1, 128, device="cuda").half()

    def body():
        y.copy_(x * 3.0)

    cap = try_capture(body)
    assert cap.ok and cap._graph is not None
    x.fill_(2.0)
    cap.replay()
    torch.cuda.synchronize()
    assert torch.all(y == 6.0)


def test_graph_capture_failure_is_reported_not_raised():
    x = torch.tensor([3.0], device="cuda")

    def body():
        float(x.item())  # a host synchronisation cannot be captured

    cap = try_capture(body)
    assert cap.ok is False and cap.reason
    with pytest.raises(RuntimeError, match="cannot replay: capture failed"):
        cap.replay()
    # the device RNG is usable again after the failed capture
    assert torch.randn(4, device="cuda").shape == (4,)


def test_hidden_stage_allocation_warns():
    seq = Sequence("hidden_alloc")

    @seq.stage
    def big_temp(x):
        scratch = torch.empty(200_000, device="cuda")  # 0.8 MB, not the output
        scratch.fill_(1.0)
        return x.clone()

    with pytest.warns(UserWarning, match="allocated .* MB internally; byte model undercounts"):
        seq.trace({"x": torch.randn(16, device="cuda").half()})


def test_time_callable_returns_positive_per_call_times():
    c = torch.zeros(1, dtype=torch.int32, device="cuda")
    times = time_callable(lambda: c.add_(1), trials=8, target_ms=4, warmup=3)
    assert len(times) == 8 and all(t > 0 for t in times)


@pytest.mark.parametrize("name,bound", [("f1", "low-byte-opportunity"),
                                        ("f2", "low-byte-opportunity"),
                                        ("f4", "material-byte-opportunity")])
def test_demo_verdict_bounds(name, bound):
    seq, inputs, replicas = build_demo(name, dim=4096, batch=1)
    rep = seq.profile(inputs, trials=6, warmup=5, input_replicas=replicas)
    assert rep.graph_ok
    assert rep.verdict().bound == bound


def test_profile_times_a_matching_fused_callable():
    d = 256
    x = torch.randn(1, d, device="cuda").half()
    g = torch.randn(d, device="cuda").half()
    seq = Sequence("two_stages")

    @seq.stage
    def mul(x, g):
        return (x * g).contiguous()

    @seq.stage
    def add(mul):
        return mul + 0.5

    rep = seq.profile({"x": x, "g": g}, trials=5, target_ms=2.0, warmup=3,
                      fused=lambda inp: inp["x"] * inp["g"] + 0.5)
    assert len(rep.stream_us) == len(rep.graph_us) == len(rep.fused_us) == 5
    v = rep.verdict()
    assert v.t_fused is not None and v.t_fused > 0


def test_profile_rejects_a_wrong_fused_callable():
    x = torch.randn(1, 128, device="cuda").half()
    seq = Sequence("wrong_fused")

    @seq.stage
    def triple(x):
        return x * 3.0

    with pytest.raises(ValueError, match="fused"):
        seq.profile({"x": x}, trials=3, target_ms=2.0, warmup=2,
                    fused=lambda inp: inp["x"] * 2.0)
