"""Pins the CPU oracle before it is trusted as the parity checker.

Sources of truth, in order:
  * known answers of the reference's C++ tests
    (validation/src/tests/test_reference.cpp:32-158), restated as literals;
  * the reference's own cpu_reference.cpp compiled into oracle/_ref (its
    known-answer binary must pass, and its functions must agree with the
    oracle on random inputs);
  * numpy.float16 / torch.float8_e4m3fn conversions, exhaustively;
  * closed forms and invariants that a plausible mistake breaks: GQA equals
    MHA with repeated KV heads, any split count equals one split, uniform
    scores average V, L = 1 returns the V row, RMSNorm scale invariance and
    an eps-sensitive closed form, fp8 dequantise-then-GEMV equals
    GEMV-then-scale;
  * planted mistakes (wrong GQA head map, wrong eps, missing scale, zero
    output) that each of those checks must reject.
The torch-stage restatement (oracle/stages.py) is then cross-checked against
the C oracle at fp16 tolerance.
"""

import json
import math
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import cref

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module", autouse=True)
def _built():
    cref.build(ref=True)
    cref.load()


def rng(seed=0):
    return np.random.default_rng(seed)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


# ------------------------------------------------------------ conversions
def test_h2f_every_fp16_value():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = cref.h2f(bits.view(np.float16))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_every_value_and_midpoint():
    bits = np.arange(0, 0x7C00, dtype=np.uint16)             # finite positives
    vals = bits.view(np.float16).astype(np.float64)
    nxt = np.append(vals[1:], 65536.0)
    mids = ((vals + nxt) / 2).astype(np.float32)             # exact in fp32
    probes = np.concatenate([vals.astype(np.float32), mids,
                             np.nextafter(mids, np.float32(0)),
                             np.nextafter(mids, np.float32(np.inf))])
    probes = np.concatenate([probes, -probes, [np.inf, -np.inf, 1e9, -1e9, 0.0]])
    probes = probes.astype(np.float32)
    with np.errstate(over="ignore"):
        want = probes.astype(np.float16)
    got = cref.f2h(probes)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


# ------------------------------------------- reference known answers (C++)
def test_reference_known_answer_binary_passes():
    if not cref.REF_TEST.exists():
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    out = subprocess.run([str(cref.REF_TEST)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout
    assert "All tests PASSED" in out.stdout


def test_known_answers_rmsnorm_gemv_silu_swiglu():
    lib = cref.load()
    x = np.array([1, 2, 3, 4], np.float32)
    out = np.empty(4, np.float32)
    lib.orc_rmsnorm_f32(x, np.ones(4, np.float32), out, 4, 1e-6)
    rms = math.sqrt(7.5 + 1e-6)
    assert np.allclose(out, x / rms, atol=1e-5, rtol=0)

    y = np.empty(2, np.float32)
    lib.orc_gemv_f32(np.array([1, 2, 3, 4], np.float32), np.ones(2, np.float32), y, 2, 2)
    assert np.allclose(y, [3.0, 7.0], atol=1e-5, rtol=0)

    assert abs(lib.orc_silu_f32(0.0)) < 1e-6
    assert abs(lib.orc_silu_f32(1.0) - 0.7310586) < 1e-6
    sw = np.empty(3, np.float32)
    lib.orc_swiglu_f32(np.array([0, 1, 2], np.float32), np.ones(3, np.float32), sw, 3)
    assert np.allclose(sw, [0.0, 0.7310586, lib.orc_silu_f32(2.0)], atol=1e-5, rtol=0)


def test_known_answers_softmax_attention():
    lib = cref.load()
    s = np.array([0, 1, 2, 0, 0, 0], np.float32)
    p = np.empty(6, np.float32)
    lib.orc_softmax_f32(s, p, 2, 3)
    e = np.exp([0.0, 1.0, 2.0])
    assert np.allclose(p[:3], e / e.sum(), atol=1e-6, rtol=0)
    assert np.allclose(p[3:], 1 / 3, atol=1e-6, rtol=0)

    q = np.array([1, 0], np.float32)
    K = np.array([1, 0, 0, 1], np.float32)
    V = np.array([2, 0, 0, 3], np.float32)
    o = np.empty(2, np.float32)
    lib.orc_attention_f32(q, K, V, o, 1, 2, 2)
    ee = math.e
    assert np.allclose(o, [2 * ee / (ee + 1), 3 / (ee + 1)], atol=1e-5, rtol=0)


def test_oracle_agrees_with_compiled_reference():
    ref = cref.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    lib = cref.load()
    r = rng(1)
    for d in (8, 96, 4096):
        x = r.standard_normal(d).astype(np.float32)
        g = (1 + 0.1 * r.standard_normal(d)).astype(np.float32)
        a, b = np.empty(d, np.float32), np.empty(d, np.float32)
        ref.ref_rmsnorm(x, g, a, d, 1e-6)
        lib.orc_rmsnorm_f32(x, g, b, d, 1e-6)
        assert np.allclose(a, b, rtol=1e-5, atol=1e-6)
    W = r.standard_normal((64, 256)).astype(np.float32)
    xv = r.standard_normal(256).astype(np.float32)
    a, b = np.empty(64, np.float32), np.empty(64, np.float32)
    ref.ref_gemv(W.ravel(), xv, a, 64, 256)
    lib.orc_gemv_f32(W.ravel(), xv, b, 64, 256)
    assert np.allclose(a, b, rtol=1e-4, atol=1e-4)
    for v in (-8.0, -1.5, 0.0, 0.3, 5.0):
        assert abs(ref.ref_silu(v) - lib.orc_silu_f32(v)) < 1e-6
    H, L, D = 3, 37, 16
    q = r.standard_normal(H * D).astype(np.float32)
    K = r.standard_normal(H * L * D).astype(np.float32)
    V = r.standard_normal(H * L * D).astype(np.float32)
    a, b = np.empty(H * D, np.float32), np.empty(H * D, np.float32)
    ref.ref_attention(q, K, V, a, H, L, D)
    lib.orc_attention_f32(q, K, V, b, H, L, D)
    assert np.allclose(a, b, rtol=1e-4, atol=1e-5)
    s = r.standard_normal(4 * 50).astype(np.float32) * 5
    a, b = np.empty(200, np.float32), np.empty(200, np.float32)
    ref.ref_softmax(s, a, 4, 50)
    lib.orc_softmax_f32(s, b, 4, 50)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-7)


def test_unscaled_gqa_attention_matches_compiled_reference_mha():
    """orc_attention_f64 (fp16 in) with G = 1 and scale 1 is the reference's
    attention_ref on the same values."""
    ref = cref.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    r = rng(2)
    H, L, D = 4, 33, 128
    q = r.standard_normal((1, H, D)).astype(np.float16) * np.float16(0.2)
    K = r.standard_normal((1, H, L, D)).astype(np.float16) * np.float16(0.2)
    V = r.standard_normal((1, H, L, D)).astype(np.float16)
    ours = cref.attention(q, K, V, scale=1.0)
    out = np.empty(H * D, np.float32)
    ref.ref_attention(q.astype(np.float32).ravel(), K.astype(np.float32).ravel(),
                      V.astype(np.float32).ravel(), out, H, L, D)
    assert np.allclose(ours.ravel(), out, rtol=1e-4, atol=1e-5)


# ------------------------------------------------- RMSNorm / GEMV closed forms
def test_rmsnorm_f16_closed_form_and_eps_sensitivity():
    # tiny activations make eps matter: mean(x^2) = 1e-6 exactly at x = 1e-3
    K = 64
    x = np.full((1, K), 1e-3, np.float16)
    g = np.ones(K, np.float16)
    got = cref.rmsnorm(x, g, eps=1e-6).astype(np.float64)
    xv = float(np.float16(1e-3))
    want = xv / math.sqrt(xv * xv + 1e-6)
    assert np.allclose(got, want, rtol=1e-3)
    planted = cref.rmsnorm(x, g, eps=1e-5).astype(np.float64)   # reference CUDA eps
    assert not np.allclose(planted, want, rtol=1e-2)


def test_rmsnorm_scale_invariance_and_unit_rms():
    r = rng(3)
    x = r.standard_normal((3, 4096)).astype(np.float16)
    g = np.ones(4096, np.float16)
    # with eps = 0 a power-of-two scaling of x is exact end to end
    a = cref.rmsnorm(x, g, eps=0.0).astype(np.float64)
    b = cref.rmsnorm((x.astype(np.float32) * 8).astype(np.float16), g,
                     eps=0.0).astype(np.float64)
    assert np.array_equal(a, b)
    assert np.allclose(np.sqrt((cref.rmsnorm(x, g).astype(np.float64) ** 2).mean(-1)),
                       1.0, atol=2e-3)


def test_gemv_small_integers_exact():
    r = rng(4)
    x = r.integers(-3, 4, (2, 64)).astype(np.float16)
    W = r.integers(-3, 4, (40, 64)).astype(np.float16)
    want = x.astype(np.int64) @ W.astype(np.int64).T
    assert np.array_equal(cref.gemv_exact(x, W), want.astype(np.float64))
    assert np.array_equal(cref.gemv(x, W).astype(np.float64), want.astype(np.float64))


def test_gemv_matches_numpy_float64_and_catches_transpose():
    r = rng(5)
    x = r.standard_normal((3, 96)).astype(np.float16)
    W = r.standard_normal((96, 96)).astype(np.float16)
    want = x.astype(np.float64) @ W.astype(np.float64).T
    assert rel_l2(cref.gemv_exact(x, W), want) < 1e-12
    planted = x.astype(np.float64) @ W.astype(np.float64)      # W not transposed
    assert rel_l2(cref.gemv_exact(x, W), planted) > 0.1


def test_swiglu_closed_form():
    gate = np.array([0.0, 1.0, 2.0, -3.0], np.float16)
    upv = np.array([1.0, 1.0, 1.0, 2.0], np.float16)
    got = cref.swiglu(gate, upv).astype(np.float64)
    silu = gate.astype(np.float64) / (1 + np.exp(-gate.astype(np.float64)))
    assert np.allclose(got, silu * upv, rtol=1e-3, atol=0)


# --------------------------------------------------------------- attention
def _qkv(B, Hq, Hkv, L, D=128, seed=0, qs=1.0):
    r = rng(seed)
    q = (r.standard_normal((B, Hq, D)) * qs).astype(np.float16)
    K = r.standard_normal((B, Hkv, L, D)).astype(np.float16)
    V = r.standard_normal((B, Hkv, L, D)).astype(np.float16)
    return q, K, V


def test_gqa_equals_mha_with_repeated_kv():
    q, K, V = _qkv(2, 8, 2, 45, seed=6)
    gqa = cref.attention(q, K, V)
    mha = cref.attention(q, np.repeat(K, 4, axis=1), np.repeat(V, 4, axis=1))
    assert np.array_equal(gqa, mha)
    # planted mistake: head h reading KV head h % Hkv instead of h // G
    Kp = np.repeat(K, 4, axis=1)[:, [h % 2 for h in range(8)]]
    Vp = np.repeat(V, 4, axis=1)[:, [h % 2 for h in range(8)]]
    Kp = np.stack([K[:, h % 2] for h in range(8)], axis=1)
    Vp = np.stack([V[:, h % 2] for h in range(8)], axis=1)
    assert rel_l2(cref.attention(q, Kp, Vp), mha) > 0.1


@pytest.mark.parametrize("S", [1, 2, 3, 4, 16, 64, 100])
def test_splitkv_equals_single_split(S):
    q, K, V = _qkv(1, 8, 2, 77, seed=7)
    one = cref.attention(q, K, V)
    assert rel_l2(cref.attention_splitkv(q, K, V, S), one) < 1e-12


def test_uniform_scores_give_mean_of_v_and_l1_gives_row():
    _, K, V = _qkv(1, 4, 1, 50, seed=8)
    q0 = np.zeros((1, 4, 128), np.float16)
    o = cref.attention(q0, K, V)
    assert np.allclose(o[0, 0], V[0, 0].astype(np.float64).mean(0), atol=1e-12)
    q, K1, V1 = _qkv(1, 4, 2, 1, seed=9)
    assert np.allclose(cref.attention(q, K1, V1)[0, 1], V1[0, 0, 0].astype(np.float64))


def test_attention_scale_and_shift_invariance():
    q, K, V = _qkv(1, 2, 1, 30, seed=10, qs=0.3)
    base = cref.attention(q, K, V)
    # the scale is applied: doubling the scale equals doubling q
    q2 = (q.astype(np.float32) * 2).astype(np.float16)
    assert rel_l2(cref.attention(q2, K, V), cref.attention(q, K, V, scale=2 / math.sqrt(128))) < 1e-12
    # planted mistake: forgetting the scale changes the result
    assert rel_l2(cref.attention(q, K, V, scale=1.0), base) > 1e-2
    # adding the same vector c to every key shifts all scores by q.c: no change
    c = np.full(128, 0.5, np.float16)
    Ks = (K.astype(np.float32) + c).astype(np.float16)
    exact_shift = np.array_equal(Ks.astype(np.float32), K.astype(np.float32) + 0.5)
    if exact_shift:
        assert rel_l2(cref.attention(q, Ks, V), base) < 1e-10


def test_relative_l2_rejects_zero_output_at_long_context():
    """At L = 32768 |o| ~ 0.009, so atol 1e-2 alone would pass an all-zero
    output; the relative-L2 check used by the parity tests must not."""
    q, K, V = _qkv(1, 4, 1, 32768, seed=11)
    o = cref.attention(q, K, V)
    zeros = np.zeros_like(o)
    # the elementwise check is nearly vacuous: most zero entries pass it
    assert np.isclose(zeros, o, rtol=1e-2, atol=1e-2).mean() > 0.6
    assert rel_l2(zeros, o) > 0.5


# ------------------------------------------------------------------- fp8
def test_e4m3_decode_matches_torch():
    torch = pytest.importorskip("torch")
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = cref.e4m3_to_f32(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


def test_fp8_gemv_dequant_then_gemv_equals_gemv_then_scale():
    r = rng(12)
    x = r.standard_normal((2, 256)).astype(np.float16)
    Wq = r.integers(0, 256, (32, 256)).astype(np.uint8)
    Wq[(Wq & 0x7F) == 0x7F] = 0x10                       # no NaN codes
    scale = (r.random(32) + 0.5).astype(np.float32)
    deq = cref.e4m3_to_f32(Wq).astype(np.float64) * scale[:, None]
    want = x.astype(np.float64) @ deq.T
    assert rel_l2(cref.gemv_fp8_exact(x, Wq, scale), want) < 1e-12


def test_e4m3_row_quantiser_and_fp8_stage():
    """quantize_e4m3_rows maps each row's absmax onto 448 (3 mantissa bits:
    relative error <= 2^-4 on normal values); the torch fp8 stage equals the
    exact C oracle to fp16 rounding, and dropping the row scale is caught."""
    torch = pytest.importorskip("torch")
    from decodebench_amd.quant import dequantize_e4m3_rows, quantize_e4m3_rows
    from oracle import stages

    r = rng(14)
    W = (r.standard_normal((96, 512)) * 0.02).astype(np.float16)
    W[3] = 0
    Wq, s = quantize_e4m3_rows(torch.from_numpy(W))
    assert Wq.dtype == torch.float8_e4m3fn and s.dtype == torch.float32
    live = np.arange(96) != 3
    assert torch.all(Wq.float().abs().amax(1)[live] == 448.0)
    assert float(s[3]) == 1.0 and torch.all(Wq[3].float() == 0)
    deq = dequantize_e4m3_rows(Wq, s).numpy().astype(np.float64)
    w64 = W.astype(np.float64)
    normal = np.abs(w64) >= s.numpy()[:, None].astype(np.float64) * 2.0 ** -6
    assert np.all(np.abs(deq - w64)[normal] <= np.abs(w64[normal]) * 2.0 ** -4 * (1 + 1e-6))
    x = r.standard_normal((2, 512)).astype(np.float16)
    got = stages.gemv_fp8(torch.from_numpy(x), Wq, s).float().numpy()
    exact = cref.gemv_fp8_exact(x, Wq.view(torch.uint8).numpy(), s.numpy())
    assert rel_l2(got, exact) < 1e-3
    unscaled = (torch.from_numpy(x).float() @ Wq.float().T).numpy()
    assert rel_l2(unscaled, exact) > 0.5


# -------------------------------------------------- torch-stage restatement
def test_torch_stages_match_c_oracle():
    torch = pytest.importorskip("torch")
    from oracle import stages

    r = rng(13)
    x = r.standard_normal((2, 1024)).astype(np.float16)
    g = (1 + 0.1 * r.standard_normal(1024)).astype(np.float16)
    W = (r.standard_normal((384, 1024)) * 0.03).astype(np.float16)
    t = lambda a: torch.from_numpy(a)  # noqa: E731
    xh_t = stages.rmsnorm(t(x), t(g)).numpy()
    xh_c = cref.rmsnorm(x, g)
    # same rounding points: at most a one-ulp fp16 difference on rare ties
    diff = np.abs(xh_t.astype(np.float64) - xh_c.astype(np.float64))
    assert (diff > 0).mean() < 0.01
    assert np.allclose(xh_t, xh_c, rtol=1e-3, atol=1e-3)
    f1_t = stages.f1(t(x), t(g), t(W)).numpy().astype(np.float64)
    assert np.allclose(f1_t, cref.f1(x, g, W).astype(np.float64), rtol=1e-2, atol=1e-2)
    assert rel_l2(f1_t, cref.f1_exact(x, g, W)) < 2e-3

    Wg = (r.standard_normal((512, 1024)) * 0.02).astype(np.float16)
    Wu = (r.standard_normal((512, 1024)) * 0.02).astype(np.float16)
    f2_t = stages.f2(t(x), t(Wg), t(Wu)).numpy().astype(np.float64)
    assert np.allclose(f2_t, cref.f2(x, Wg, Wu).astype(np.float64), rtol=1e-2, atol=1e-2)
    assert rel_l2(f2_t, cref.f2_exact(x, Wg, Wu)) < 5e-3

    q, K, V = _qkv(2, 8, 2, 300, seed=14)
    f4_t = stages.f4(t(q), t(K), t(V)).numpy().astype(np.float64)
    exact = cref.attention(q, K, V)
    assert np.allclose(f4_t, exact, rtol=1e-2, atol=1e-2)
    assert rel_l2(f4_t, exact) < 1e-2


# ------------------------------------------------------- host statistics
def test_bootstrap_matches_reference_vectors():
    from decodebench_amd.stats import bootstrap_diff_ci, summarize

    data = json.loads((ROOT / "tests" / "golden" / "stats_vectors.json").read_text())
    for c in data["cases"]:
        lo, hi, point = bootstrap_diff_ci(c["a"], c["b"], n_resamples=c["n_resamples"],
                                          ci=c["ci"], seed=c["seed"])
        assert (lo, hi, point) == (c["lo"], c["hi"], c["point"])
        s = summarize(c["a"])
        assert [s.median, s.p25, s.p75, s.n] == c["summary_a"]
