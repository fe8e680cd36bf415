"""C ABI checks that need no GPU.

* libdecodebench_hip.so loads and exports every function declared in
  include/*.h (the drop-in surface and the tuning hooks);
* every contract violation returns DB_ERR_INVALID with a message before any
  HIP call (so these run on a GPU-less host);
* the Python wrappers turn those codes into ValueError / NotImplementedError.
"""

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


@pytest.fixture(scope="module")
def lib():
    from decodebench_amd import build, ops

    if not ops.LIB_PATH.exists():
        build.build(verbose=False)
    return ops.load_library()


def declared_functions():
    text = "\n".join(h.read_text() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(db_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for want in ("db_abi_version", "db_last_error", "db_f1_rmsnorm_gemv",
                 "db_f2_gateup_swiglu", "db_f2_rmsnorm_gateup_swiglu", "db_gemv",
                 "db_f4_splitkv",
                 "db_f4_workspace_bytes", "db_f4_default_splits", "db_device_cu_count",
                 "db_f4_splitkv_noalloc", "db_tune", "db_tune_get"):
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.db_abi_version() == 1


P = 0x10000  # a fake, 16-byte aligned device address: never dereferenced


def last(lib):
    return lib.db_last_error().decode()


def test_f1_contract_errors(lib):
    f = lib.db_f1_rmsnorm_gemv
    assert f(None, P, P, None, P, 1, 4096, 4096, 1e-6, 0, None) == -1
    assert "null" in last(lib)
    assert f(P, P, P, None, P, 1, 4100, 4096, 1e-6, 0, None) == -1
    assert "multiple of 8" in last(lib)
    assert f(P, P, P, None, P, 0, 4096, 4096, 1e-6, 0, None) == -1
    assert f(P, P, P + 2, None, P, 1, 4096, 4096, 1e-6, 0, None) == -1
    assert "aligned" in last(lib)
    assert f(P, P, P, None, P, 1, 4096, 4096, -1.0, 0, None) == -1
    assert "eps" in last(lib)
    assert f(P, P, P, None, P, 1, 4096, 4096, 1e-6, 7, None) == -1
    assert "dtype" in last(lib)
    assert f(P, P, P, None, P, 1, 1 << 20, 4096, 1e-6, 0, None) == -1
    assert "LDS" in last(lib)


def test_f2_and_gemv_contract_errors(lib):
    assert lib.db_f2_gateup_swiglu(P, P, None, None, None, P, 1, 4096, 14336, 0, None) == -1
    assert lib.db_f2_gateup_swiglu(P, P, P, C.c_void_p(P), None, P, 1, 4096, 14336, 0,
                                   None) == -1
    assert "no scale" in last(lib)
    assert lib.db_gemv(P, P, None, P, 1, 12, 16, 0, None) == -1


def test_f2_rmsnorm_contract_errors(lib):
    f = lib.db_f2_rmsnorm_gateup_swiglu
    assert f(P, None, P, P, None, None, P, 1, 4096, 14336, 1e-6, 0, None) == -1
    assert "gain" in last(lib)
    assert f(P, P, P, None, None, None, P, 1, 4096, 14336, 1e-6, 0, None) == -1
    assert "null" in last(lib)
    assert f(P, P, P, P, None, None, P, 1, 4096, 14336, float("nan"), 0, None) == -1
    assert "eps" in last(lib)
    assert f(P, P + 8, P, P, None, None, P, 1, 4096, 14336, 1e-6, 0, None) == -1
    assert "aligned" in last(lib)


def test_fp8_weight_contract_errors(lib):
    """fp8 e4m3 weights: K % 16, a scale vector per matrix, 4-byte aligned
    scales.  (No call here passes the contract: that would reach the GPU.)"""
    S = C.c_void_p(P)
    f1 = lib.db_f1_rmsnorm_gemv
    assert f1(P, P, P, None, P, 1, 4096, 4096, 1e-6, 1, None) == -1
    assert "scale" in last(lib)
    assert f1(P, P, P, S, P, 1, 4104, 4096, 1e-6, 1, None) == -1
    assert "multiple of 16" in last(lib)
    assert f1(P, P, P, C.c_void_p(P + 2), P, 1, 4096, 4096, 1e-6, 1, None) == -1
    assert "4-byte" in last(lib)
    f2 = lib.db_f2_gateup_swiglu
    assert f2(P, P, P, S, None, P, 1, 4096, 14336, 1, None) == -1
    assert "scale" in last(lib)
    assert lib.db_gemv(P, P, None, P, 1, 4096, 4096, 1, None) == -1
    assert "scale" in last(lib)
    assert lib.db_f2_rmsnorm_gateup_swiglu(P, P, P, P, S, None, P, 1, 4096, 14336, 1e-6, 1,
                                           None) == -1


def test_f4_contract_errors(lib):
    f = lib.db_f4_splitkv
    ok = dict(B=1, Hq=32, Hkv=8, L=1024, D=128, S=4)

    def call(ws=P, ws_bytes=1 << 30, **kw):
        a = {**ok, **kw}
        return f(P, P, P, P, ws, ws_bytes, a["B"], a["Hq"], a["Hkv"], a["L"], a["D"], a["S"],
                 0.088, None)

    assert call(D=64) == -1 and "128" in last(lib)
    assert call(Hq=30) == -1 and "multiple" in last(lib)
    assert call(Hq=48, Hkv=4) == -1 and "G=12" in last(lib)
    assert call(L=0) == -1
    assert call(S=0) == -1 and call(S=257) == -1
    assert call(ws=None) == -1 and "workspace" in last(lib)
    assert call(ws_bytes=16) == -1 and "required" in last(lib)
    assert f(None, P, P, P, P, 1 << 30, 1, 32, 8, 1024, 128, 4, 0.1, None) == -1


def test_f4_noalloc_contract_errors(lib):
    """The allocation-free F4 entry point checks the same contract, and
    rejects split counts whose partial records exceed its scratch array,
    before any HIP call."""
    f = lib.db_f4_splitkv_noalloc

    def call(B=1, Hq=32, Hkv=8, L=1024, D=128, S=4, q=P):
        return f(q, P, P, P, B, Hq, Hkv, L, D, S, 0.088, None)

    assert call(q=None) == -1 and "null" in last(lib)
    assert call(D=64) == -1 and "128" in last(lib)
    assert call(Hq=48, Hkv=4) == -1 and "G=12" in last(lib)
    assert call(S=0) == -1 and call(S=257) == -1
    scratch = 4 << 20
    # B=8, Hkv=8, G=8, 256 splits: 64 pairs x 256 x 8 heads x 128 x 4 B = 64 MiB of partials
    assert lib.db_f4_workspace_bytes(8, 64, 8, 1 << 16, 128, 256) > scratch
    assert call(B=8, Hq=64, Hkv=8, L=1 << 16, S=256) == -1
    assert "scratch" in last(lib) and str(scratch) in last(lib)
    # S is capped at the tile count first: 256 splits of 16 keys need one split
    assert lib.db_f4_workspace_bytes(8, 64, 8, 16, 128, 1) == 0


def test_f4_workspace_and_split_policy(lib):
    assert lib.db_f4_workspace_bytes(1, 32, 8, 8192, 128, 1) == 0
    ws = lib.db_f4_workspace_bytes(1, 32, 8, 8192, 128, 64)
    assert ws >= 8 * 256 + 8 * 64 * 4 * 130 * 4    # ticket lines; o, m, l per (pair, split, head)
    s = lib.db_f4_default_splits(1, 8, 8192, 256)
    assert 1 <= s <= 256
    assert lib.db_f4_default_splits(1, 8, 16, 256) == 1       # one tile -> one split
    assert lib.db_f4_default_splits(8, 8, 32768, 256) >= 1


def test_tune_keys(lib):
    assert lib.db_tune(b"nope", 1) == -1
    assert lib.db_tune(b"f4_blocks_per_cu", 0) == -1
    assert lib.db_tune(b"f4_waves", 5) == -1
    assert lib.db_tune(b"f4_merge", 3) == -1
    assert lib.db_tune(b"f4_misplace", -1) == -1
    assert lib.db_tune(b"f4_depth", 3) == -1
    assert lib.db_tune(b"f4_depth", 0) == 0
    assert lib.db_tune(b"f4_launch", 3) == -1
    assert lib.db_tune(b"f4_launch", 0) == 0
    assert lib.db_tune(b"f4_waves", 16) == -1
    assert lib.db_tune(b"gemv_long_kc", 3) == -1
    assert lib.db_tune(b"gemv_long_gpw", 3) == -1
    assert lib.db_tune(b"gemv_long_kc", 0) == 0
    assert lib.db_tune(b"gemv_long_gpw", 0) == 0
    assert lib.db_tune(b"gemv_long_stage", 3) == -1
    assert lib.db_tune(b"gemv_long_stage", 0) == 0
    assert lib.db_tune(b"gemv_pair_min_batch", 1) == -1
    assert lib.db_tune(b"gemv_pair_min_batch", 0) == 0
    assert lib.db_tune(b"gemv_long_gpw", 7) == -1
    assert lib.db_tune(b"gemv_pair_tiles", 0) == -1
    assert lib.db_tune(b"gemv_pass_grid", 12) == -1
    assert lib.db_tune(b"gemv_pass_grid", -8) == -1
    assert lib.db_tune(b"gemv_pass_grid", 0) == 0
    assert lib.db_tune(b"gemv_xb", 2) == -1
    assert lib.db_tune(b"gemv_xb", 0) == 0
    assert lib.db_tune(b"f4_merge", 2) == 0
    assert lib.db_tune(b"f4_merge", 0) == 0
    assert lib.db_tune(b"f4_blocks_per_cu", 2) == 0
    assert lib.db_tune(b"f4_blocks_per_cu", 1) == 0   # back to the default


def test_tune_get_reads_this_threads_knobs(lib):
    import threading

    v = C.c_int(-1)
    assert lib.db_tune_get(b"nope", C.byref(v)) == -1 and "unknown" in last(lib)
    assert lib.db_tune_get(b"f4_min_tiles", None) == -1
    assert lib.db_tune_get(b"f4_min_tiles", C.byref(v)) == 0 and v.value == 8
    # a rejected value changes nothing
    assert lib.db_tune(b"f4_min_tiles", 0) == -1
    assert lib.db_tune_get(b"f4_min_tiles", C.byref(v)) == 0 and v.value == 8
    # gemv_waves_per_cu stores non-positive values as 0 (the default)
    assert lib.db_tune(b"gemv_waves_per_cu", -3) == 0
    assert lib.db_tune_get(b"gemv_waves_per_cu", C.byref(v)) == 0 and v.value == 0
    seen = {}
    try:
        assert lib.db_tune(b"f4_merge", 2) == 0

        def other():
            w = C.c_int(-1)
            seen["rc"] = lib.db_tune_get(b"f4_merge", C.byref(w))
            seen["value"] = w.value
            seen["set"] = lib.db_tune(b"f4_min_tiles", 3)

        t = threading.Thread(target=other)
        t.start()
        t.join()
        assert seen == {"rc": 0, "value": 0, "set": 0}   # a new thread starts from defaults
        assert lib.db_tune_get(b"f4_merge", C.byref(v)) == 0 and v.value == 2
        assert lib.db_tune_get(b"f4_min_tiles", C.byref(v)) == 0 and v.value == 8
    finally:
        assert lib.db_tune(b"f4_merge", 0) == 0


def test_python_wrappers_check_fp8_scales():
    torch = pytest.importorskip("torch")
    from decodebench_amd import ops

    x = torch.zeros(1, 64, dtype=torch.float16)
    Wq = torch.zeros(8, 64, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError):
        ops.gemv(x, Wq)  # CPU tensors and no scale: rejected before any launch


def test_python_wrappers_raise_on_cpu_tensors():
    torch = pytest.importorskip("torch")
    from decodebench_amd import ops

    x = torch.zeros(1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        ops.f1_rmsnorm_gemv(x, torch.zeros(64, dtype=torch.float16),
                            torch.zeros(8, 64, dtype=torch.float16))


def test_python_wrappers_reject_mixed_devices():
    torch = pytest.importorskip("torch")
    from decodebench_amd import ops

    a = torch.zeros(4)
    ops._same_device((a, "x"), (torch.zeros(2), "W"))  # one device: accepted
    with pytest.raises(ValueError, match="W is on meta"):
        ops._same_device((a, "x"), (torch.zeros(2, device="meta"), "W"))
