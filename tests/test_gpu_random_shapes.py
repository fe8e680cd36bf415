"""Seeded random shapes through the C ABI against the CPU oracle.

The hand-picked parity cases cover the decode shapes and known edges; these
draw the rest of the contract at random: every GEMV mode (plain, F1, F2,
RMSNorm→F2) in fp16 and e4m3 weights with batches that land on both the
VALU and the MFMA kernel (K ∈ {2048, 4096} is weighted up so the MFMA path
is hit), ragged K and N, one weight matrix at 17..48 rows (the MFMA kernel's
32-row passes), plain GEMV with K a multiple of 2048 above 4096 at 3..48
rows (the long-row MFMA kernel), and F4 over random batch, head grouping, KV length and
split count.  The draws are fixed by the seed, so every run tests the
same cases; each prints its case before it runs.  DB_RANDOM_SHAPES=<n> and
DB_RANDOM_SEED=<s> draw a larger or different set for a one-off sweep (the
F4 count is half the GEMV count).  Bars as in the parity
tests: rtol/atol 1e-2 against the torch stages on the CPU and a relative-L2
bound against the exact oracle.
"""

import math
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from decodebench_amd import ops  # noqa: E402
from decodebench_amd.quant import quantize_e4m3_rows  # noqa: E402
from oracle import cref, stages  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-2
MAC_BUDGET = 24_000_000  # B*N*K per case: keeps the CPU reference to about a second
N_GEMV = int(os.environ.get("DB_RANDOM_SHAPES", "48"))
SEED = int(os.environ.get("DB_RANDOM_SEED", "20261201"))


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def randn(gen, shape, std=1.0, mean=0.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * std + mean).half()


def check(got, stage_ref, exact, bound, what):
    got = got.float().cpu().numpy().astype(np.float64)
    ref = stage_ref.float().numpy().astype(np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    bad = ~np.isclose(got, ref, rtol=TOL, atol=TOL)
    assert not bad.any(), f"{what}: {bad.sum()} elements outside 1e-2, max abs " \
                          f"{np.abs(got - ref).max():.3e}"
    err = rel_l2(got, exact)
    assert err <= bound, f"{what}: rel-L2 {err:.3e} > {bound}"


def _gemv_cases(n=N_GEMV, seed=SEED):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        mode = ("plain", "f1", "f2", "f2n")[rng.integers(4)]
        dtype = "fp8" if rng.random() < 0.5 else "f16"
        step = 16 if dtype == "fp8" else 8
        B = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 33]))
        if rng.random() < 0.4:
            K = int(rng.choice([2048, 4096]))
        else:
            K = step * int(rng.integers(1, 6000 // step + 1))
        N = int(rng.integers(1, 3000))
        if B * N * K > MAC_BUDGET:
            continue
        cases.append((mode, dtype, B, K, N, int(rng.integers(1 << 30))))
    return cases


def _pass32_cases(n=max(16, N_GEMV // 3), seed=SEED + 2):
    """One weight matrix at 17..48 rows with K in {2048, 4096}: the 32-row
    passes that hold rows 16..31 of x in LDS (and a second pass above 32)."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        mode = ("plain", "f1")[rng.integers(2)]
        dtype = "fp8" if rng.random() < 0.5 else "f16"
        B = int(rng.choice([17, 20, 24, 25, 31, 32, 33, 40, 48]))
        K = int(rng.choice([2048, 4096]))
        N = int(rng.integers(1, 6145))
        if B * N * K > 8 * MAC_BUDGET:
            continue
        cases.append((mode, dtype, B, K, N, int(rng.integers(1 << 30))))
    return cases


def _long_cases(n=max(16, N_GEMV // 3), seed=SEED + 3):
    """Plain GEMV at 3..48 rows with K a multiple of 2048 above 4096: the
    long-row MFMA kernel that streams x in K chunks (one pass up to 32 rows)."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        dtype = "fp8" if rng.random() < 0.5 else "f16"
        B = int(rng.choice([3, 5, 8, 9, 16, 17, 24, 32, 33, 48]))
        K = 2048 * int(rng.integers(3, 15))
        N = int(rng.integers(1, 4097))
        if B * N * K > 8 * MAC_BUDGET:
            continue
        cases.append(("plain", dtype, B, K, N, int(rng.integers(1 << 30))))
    return cases


def _f4_cases(n=N_GEMV // 2, seed=SEED + 1):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        B = int(rng.integers(1, 5))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 4, 8]))
        L = int(rng.integers(1, 6000))
        S = None if rng.random() < 0.4 else int(rng.integers(1, 65))
        cases.append((B, Hkv * G, Hkv, L, S, int(rng.integers(1 << 30))))
    return cases


@pytest.fixture(scope="module", autouse=True)
def _lib():
    ops.load_library()
    cref.load()


@pytest.mark.parametrize("mode,dtype,B,K,N,seed", _gemv_cases() + _pass32_cases() + _long_cases())
def test_random_gemv_shapes(mode, dtype, B, K, N, seed):
    print(f"[rand-gemv] {mode} {dtype} B={B} K={K} N={N} seed={seed}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    x = randn(gen, (B, K))
    g = randn(gen, (K,), std=0.1, mean=1.0)
    W = randn(gen, (N, K), std=1.0 / math.sqrt(K))
    W2 = randn(gen, (N, K), std=1.0 / math.sqrt(K))
    xd, gd = x.cuda(), g.cuda()
    norm = mode in ("f1", "f2n")
    xin = stages.rmsnorm(x, g) if norm else x
    xin_np = cref.rmsnorm(x.numpy(), g.numpy()) if norm else x.numpy()
    if dtype == "fp8":
        Wq, s = quantize_e4m3_rows(W)
        W2q, s2 = quantize_e4m3_rows(W2)
        bits, bits2 = Wq.view(torch.uint8).numpy(), W2q.view(torch.uint8).numpy()
        if mode in ("plain", "f1"):
            y = (ops.gemv(xd, Wq.cuda(), w_scale=s.cuda()) if mode == "plain" else
                 ops.f1_rmsnorm_gemv(xd, gd, Wq.cuda(), w_scale=s.cuda()))
            ref = stages.gemv_fp8(xin, Wq, s)
            exact, bound = cref.gemv_fp8_exact(xin_np, bits, s.numpy()), 2e-3
        else:
            y = (ops.f2_gateup_swiglu(xd, Wq.cuda(), W2q.cuda(), s.cuda(), s2.cuda())
                 if mode == "f2" else
                 ops.f2_rmsnorm_gateup_swiglu(xd, gd, Wq.cuda(), W2q.cuda(), sg=s.cuda(),
                                              su=s2.cuda()))
            ref = stages.f2_fp8(xin, Wq, s, W2q, s2)
            exact = cref.f2_fp8_exact(xin_np, bits, s.numpy(), bits2, s2.numpy())
            bound = 5e-3
    else:
        if mode in ("plain", "f1"):
            y = (ops.gemv(xd, W.cuda()) if mode == "plain" else
                 ops.f1_rmsnorm_gemv(xd, gd, W.cuda()))
            ref = stages.gemv(xin, W)
            exact, bound = cref.gemv_exact(xin_np, W.numpy()), 2e-3
        else:
            y = (ops.f2_gateup_swiglu(xd, W.cuda(), W2.cuda()) if mode == "f2" else
                 ops.f2_rmsnorm_gateup_swiglu(xd, gd, W.cuda(), W2.cuda()))
            ref = stages.f2(xin, W, W2)
            exact, bound = cref.f2_exact(xin_np, W.numpy(), W2.numpy()), 5e-3
    torch.cuda.synchronize()
    assert y.shape == (B, N)
    check(y, ref, exact, bound, f"{mode} {dtype} B={B} K={K} N={N}")


@pytest.mark.parametrize("B,Hq,Hkv,L,S,seed", _f4_cases())
def test_random_f4_shapes(B, Hq, Hkv, L, S, seed):
    print(f"[rand-f4] B={B} Hq={Hq} Hkv={Hkv} L={L} S={S} seed={seed}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    q = randn(gen, (B, Hq, 128))
    K = randn(gen, (B, Hkv, L, 128))
    V = randn(gen, (B, Hkv, L, 128))
    o = ops.f4_flashdecode(q.cuda(), K.cuda(), V.cuda(), n_splits=S)
    torch.cuda.synchronize()
    assert o.shape == (B, Hq, 128)
    exact = cref.attention(q.numpy(), K.numpy(), V.numpy())
    check(o, stages.f4(q, K, V), exact, 5e-3, f"f4 B={B} Hq={Hq} Hkv={Hkv} L={L} S={S}")
