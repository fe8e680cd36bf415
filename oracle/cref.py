"""ctypes/numpy wrapper over oracle/cref.c (TEST INFRASTRUCTURE ONLY).

fp16 arrays are passed as numpy ``float16`` (their bits are read as uint16);
results come back as numpy arrays.  ``load()`` builds liboracle.so with the
committed Makefile when it is missing.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libcpu_reference.so"
REF_TEST = HERE / "_ref" / "test_reference"

_lib = None
_ref = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i, _f, _d, _sz = C.c_int, C.c_float, C.c_double, C.c_size_t


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if ref and Path("/root/reference/validation/src/reference/cpu_reference.cpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build(ref=False)
    lib = C.CDLL(str(LIB))
    sig = {
        "orc_h2f": (_f, [C.c_uint16]),
        "orc_f2h": (C.c_uint16, [_f]),
        "orc_h2f_array": (None, [_u16p, _f32p, _sz]),
        "orc_f2h_array": (None, [_f32p, _u16p, _sz]),
        "orc_rmsnorm_f32": (None, [_f32p, _f32p, _f32p, _i, _f]),
        "orc_gemv_f32": (None, [_f32p, _f32p, _f32p, _i, _i]),
        "orc_silu_f32": (_f, [_f]),
        "orc_swiglu_f32": (None, [_f32p, _f32p, _f32p, _i]),
        "orc_softmax_f32": (None, [_f32p, _f32p, _i, _i]),
        "orc_attention_f32": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i]),
        "orc_rmsnorm_f16": (None, [_u16p, _u16p, _u16p, _i, _i, _f]),
        "orc_gemv_f64": (None, [_u16p, _u16p, _f64p, _i, _i, _i]),
        "orc_gemv_f16": (None, [_u16p, _u16p, _u16p, _i, _i, _i]),
        "orc_swiglu_f16": (None, [_u16p, _u16p, _u16p, _sz]),
        "orc_attention_f64": (None, [_u16p, _u16p, _u16p, _f64p, _i, _i, _i, _i, _i, _d]),
        "orc_attention_splitkv_f64": (None, [_u16p, _u16p, _u16p, _f64p, _i, _i, _i, _i,
                                             _i, _d, _i]),
        "orc_e4m3_to_f32": (_f, [C.c_uint8]),
        "orc_gemv_fp8_f64": (None, [_u16p, _u8p, _f32p, _f64p, _i, _i, _i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def load_ref():
    """The reference's compiled cpu_reference.cpp (None when not built)."""
    global _ref
    if _ref is not None:
        return _ref
    if not REF_LIB.exists():
        return None
    lib = C.CDLL(str(REF_LIB))
    for name, args, res in [
        ("ref_rmsnorm", [_f32p, _f32p, _f32p, _i, _f], None),
        ("ref_gemv", [_f32p, _f32p, _f32p, _i, _i], None),
        ("ref_silu", [_f], _f),
        ("ref_swiglu", [_f32p, _f32p, _f32p, _i], None),
        ("ref_softmax", [_f32p, _f32p, _i, _i], None),
        ("ref_attention", [_f32p, _f32p, _f32p, _f32p, _i, _i, _i], None),
    ]:
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _ref = lib
    return lib


# ----------------------------------------------------------------- helpers
def _h(a) -> np.ndarray:
    """float16 array -> contiguous uint16 view."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float16))
    return a.view(np.uint16)


def _as_f16(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16)


def f2h(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, dtype=np.uint16)
    load().orc_f2h_array(x.ravel(), out.ravel(), x.size)
    return _as_f16(out)


def h2f(x) -> np.ndarray:
    bits = _h(x)
    out = np.empty(bits.shape, dtype=np.float32)
    load().orc_h2f_array(bits.ravel(), out.ravel(), bits.size)
    return out


# -------------------------------------------------- torch-stage semantics
def rmsnorm(x, g, eps: float = 1e-6) -> np.ndarray:
    """fp16 [B,K] -> fp16 [B,K] with the torch stage's rounding points."""
    x = np.atleast_2d(x)
    B, K = x.shape
    out = np.empty((B, K), dtype=np.uint16)
    load().orc_rmsnorm_f16(_h(x), _h(g), out, B, K, eps)
    return _as_f16(out)


def gemv_exact(x, W) -> np.ndarray:
    """x [B,K] . W[N,K]^T in double."""
    x = np.atleast_2d(x)
    B, K = x.shape
    N = W.shape[0]
    out = np.empty((B, N), dtype=np.float64)
    load().orc_gemv_f64(_h(x), _h(W), out, B, K, N)
    return out


def gemv(x, W) -> np.ndarray:
    """fp16 output of a double-accumulated GEMV (the F.linear stage)."""
    x = np.atleast_2d(x)
    B, K = x.shape
    N = W.shape[0]
    out = np.empty((B, N), dtype=np.uint16)
    load().orc_gemv_f16(_h(x), _h(W), out, B, K, N)
    return _as_f16(out)


def swiglu(gate, up) -> np.ndarray:
    g = _h(gate)
    out = np.empty(g.shape, dtype=np.uint16)
    load().orc_swiglu_f16(g.ravel(), _h(up).ravel(), out.ravel(), g.size)
    return _as_f16(out)


def f1(x, g, W, eps: float = 1e-6) -> np.ndarray:
    """F1 chain: rmsnorm then gemv, fp16 out."""
    return gemv(rmsnorm(x, g, eps), W)


def f1_exact(x, g, W, eps: float = 1e-6) -> np.ndarray:
    """F1 with the fp16-rounded normalised activation and an exact GEMV."""
    return gemv_exact(rmsnorm(x, g, eps), W)


def f2(x, Wg, Wu) -> np.ndarray:
    """F2 chain: gate, up (fp16 each), silu(gate)*up, fp16 out."""
    return swiglu(gemv(x, Wg), gemv(x, Wu))


def f2_exact(x, Wg, Wu) -> np.ndarray:
    """silu(x Wg^T) * (x Wu^T) with no intermediate rounding (double)."""
    g = gemv_exact(x, Wg)
    u = gemv_exact(x, Wu)
    return g / (1.0 + np.exp(-g)) * u


def attention(q, K, V, scale: float | None = None) -> np.ndarray:
    """Exact GQA decode attention: q [B,Hq,D], K/V [B,Hkv,L,D] -> double."""
    B, Hq, D = q.shape
    Hkv, L = K.shape[1], K.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.empty((B, Hq, D), dtype=np.float64)
    load().orc_attention_f64(_h(q), _h(K), _h(V), out, B, Hq, Hkv, L, D, float(scale))
    return out


def attention_splitkv(q, K, V, S: int, scale: float | None = None) -> np.ndarray:
    B, Hq, D = q.shape
    Hkv, L = K.shape[1], K.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.empty((B, Hq, D), dtype=np.float64)
    load().orc_attention_splitkv_f64(_h(q), _h(K), _h(V), out, B, Hq, Hkv, L, D,
                                     float(scale), int(S))
    return out


def e4m3_to_f32(codes) -> np.ndarray:
    lib = load()
    return np.array([lib.orc_e4m3_to_f32(int(c)) for c in np.asarray(codes).ravel()],
                    dtype=np.float32).reshape(np.shape(codes))


def gemv_fp8_exact(x, Wq, scale) -> np.ndarray:
    x = np.atleast_2d(x)
    B, K = x.shape
    N = Wq.shape[0]
    out = np.empty((B, N), dtype=np.float64)
    load().orc_gemv_fp8_f64(_h(x), np.ascontiguousarray(Wq, dtype=np.uint8),
                            np.ascontiguousarray(scale, dtype=np.float32), out, B, K, N)
    return out


def f1_fp8_exact(x, g, Wq, scale, eps: float = 1e-6) -> np.ndarray:
    """fp8 F1: the fp16-rounded normalised activation, then an exact fp8 GEMV."""
    return gemv_fp8_exact(rmsnorm(x, g, eps), Wq, scale)


def f2_fp8_exact(x, Wgq, sg, Wuq, su) -> np.ndarray:
    """silu(g) * u of the exact fp8 gate and up projections (double)."""
    g = gemv_fp8_exact(x, Wgq, sg)
    u = gemv_fp8_exact(x, Wuq, su)
    return g / (1.0 + np.exp(-g)) * u
