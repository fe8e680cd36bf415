"""Fused decode ops backed by libdecodebench_hip.so (HIP, gfx950).

Each op takes torch tensors on the GPU, allocates its output with
``torch.empty`` and launches one kernel on ``torch.cuda.current_stream()``
through the C ABI declared in ``include/decodebench_hip.h``.  No op allocates
inside the library, synchronises, or reads device memory on the host, so the
ops work as ``Sequence`` stages, inside a ``profile(fused=...)`` callable, and
under ``torch.cuda.graph`` capture.

This follows the plug-in pattern of the reference's custom-kernel example
(examples/custom_kernel/bindings.cpp:13-30: output from ``empty_like``, launch
on the current stream) with ctypes over a C ABI instead of a torch extension.

There is no fallback: if the HIP library is missing or cannot be loaded the
ops raise ``RuntimeError`` naming the build command.
"""

from __future__ import annotations

import ctypes as C
import math
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libdecodebench_hip.so"

DB_OK = 0
DB_ERR_INVALID = -1
DB_ERR_UNSUPPORTED = -2
DTYPE_F16 = 0
DTYPE_FP8_E4M3 = 1

_lock = threading.Lock()
_lib = None
_cu_cache: dict[int, int] = {}
_ws_cache: dict[tuple, object] = {}
_captured_ws: dict[tuple, object] = {}  # workspaces made under graph capture (kept alive)

_p = C.c_void_p
_i = C.c_int


def load_library():
    """Load the HIP library (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  -- torch's libamdhip64 must be loaded first

        if not LIB_PATH.exists():
            raise RuntimeError(
                f"HIP library {LIB_PATH} is not built; run "
                "`python -m decodebench_amd.build` (hipcc, gfx950)")
        lib = C.CDLL(str(LIB_PATH))
        protos = {
            "db_abi_version": (_i, []),
            "db_last_error": (C.c_char_p, []),
            "db_device_cu_count": (_i, [C.POINTER(_i)]),
            "db_f1_rmsnorm_gemv": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, C.c_float, _i, _p]),
            "db_f2_gateup_swiglu": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
            "db_f2_rmsnorm_gateup_swiglu": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i,
                                                 C.c_float, _i, _p]),
            "db_gemv": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p]),
            "db_f4_default_splits": (_i, [_i, _i, _i, _i]),
            "db_f4_workspace_bytes": (C.c_size_t, [_i, _i, _i, _i, _i, _i]),
            "db_f4_splitkv": (_i, [_p, _p, _p, _p, _p, C.c_size_t, _i, _i, _i, _i, _i, _i,
                                   C.c_float, _p]),
            "db_f4_splitkv_noalloc": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, C.c_float,
                                           _p]),
            "db_stream_read": (_i, [_p, C.c_size_t, _i, C.c_uint, _p, _p]),
            "db_stream_capture_id": (_i, [_p, C.POINTER(C.c_ulonglong)]),
            "db_tune": (_i, [C.c_char_p, _i]),
            "db_tune_get": (_i, [C.c_char_p, C.POINTER(_i)]),
            "db_f4_launch_info": (_i, [_i, _i, _i, _i, _i, C.POINTER(_i), C.POINTER(_i)]),
            "db_null_kernel": (_i, [_p]),
        }
        for name, (res, args) in protos.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.db_abi_version() != 1:
            raise RuntimeError("libdecodebench_hip.so ABI version mismatch")
        _lib = lib
        return lib


def _check(rc: int, what: str) -> None:
    if rc == DB_OK:
        return
    msg = load_library().db_last_error().decode(errors="replace")
    if rc == DB_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if rc == DB_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (HIP error {rc}): {msg}")


def _same_device(*named) -> None:
    """All tensors of one call must live on one GPU."""
    dev = named[0][0].device
    for t, name in named[1:]:
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev} like {named[0][1]}")


_torch = None
_raw_stream = None


def _torch_mod():
    """torch, imported once, and the fastest handle to the current stream."""
    global _torch, _raw_stream
    if _torch is None:
        import torch

        raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        _raw_stream = raw if raw is not None else (
            lambda idx: torch.cuda.current_stream(idx).cuda_stream)
        _torch = torch
    return _torch


def _gpu_tensors(*items) -> int:
    """Check ``(tensor, name, dtype or None)`` items in one pass: a torch
    tensor on a GPU, of that dtype, contiguous, all on one GPU.  Returns the
    GPU's index.  Every check is a C-level attribute read, so the hot call
    stays cheap."""
    torch = _torch or _torch_mod()
    idx, first = -1, None
    for t, name, dt in items:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU device (got {t.device})")
        if dt is not None and t.dtype != dt:
            raise TypeError(f"{name} must be {dt} (got {t.dtype})")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        d = t.get_device()
        if first is None:
            idx, first = d, name
        elif d != idx:
            raise ValueError(f"{name} is on cuda:{d}, expected cuda:{idx} like {first}")
    return idx


def _launch(fn, idx: int, what: str, *args) -> None:
    """``fn(*args, stream)`` on GPU ``idx`` (made current if it is not) and
    its current stream; a non-zero status raises."""
    torch = _torch
    if torch.cuda.current_device() == idx:
        rc = fn(*args, _raw_stream(idx))
    else:
        with torch.cuda.device(idx):
            rc = fn(*args, _raw_stream(idx))
    if rc:
        _check(rc, what)


def _output(shape, idx: int, out, name: str = "out"):
    """A new fp16 tensor of ``shape`` on GPU ``idx``, or ``out`` checked."""
    torch = _torch
    if out is None:
        return torch.empty(shape, dtype=torch.float16, device=torch.device("cuda", idx))
    _gpu_tensors((out, name, torch.float16))
    if out.get_device() != idx:
        raise ValueError(f"{name} is on cuda:{out.get_device()}, expected cuda:{idx}")
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(out.shape)})")
    return out


def cu_count(device=None) -> int:
    """Compute units of a GPU (index, torch.device or None for the current one)."""
    if isinstance(device, int) and device in _cu_cache:
        return _cu_cache[device]
    torch = _torch or _torch_mod()
    if isinstance(device, int):
        idx = device
    else:
        dev = torch.device("cuda" if device is None else device)
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cu_cache:
        _cu_cache[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cu_cache[idx]


def null_kernel(device=None) -> None:
    """Launch the library's empty kernel on the current stream (the
    launch-overhead probe of ``decodebench_amd.calibrate``)."""
    import torch

    dev = torch.device("cuda" if device is None else device)
    with torch.cuda.device(dev):
        rc = load_library().db_null_kernel(torch.cuda.current_stream(dev).cuda_stream)
    _check(rc, "db_null_kernel")


def stream_read(src, kb_per_wave: int = 8, sink=None) -> None:
    """Launch the read-only streaming probe over all of ``src`` (a contiguous
    GPU tensor of a whole number of ``kb_per_wave`` KB) on the current stream.

    ``src`` should hold zeros: the probe stores to ``sink`` only when the
    folded data equals its (non-zero) magic value, so it then writes
    nothing.  ``sink`` (int32, >= nbytes/16 elements) is allocated when not
    given; pass one to keep the call allocation-free (graph capture)."""
    import torch

    idx = _gpu_tensors((src, "src", None))
    nbytes = src.numel() * src.element_size()
    if sink is None:
        sink = _torch.empty(max(1, nbytes // 16), dtype=_torch.int32, device=src.device)
    _launch((_lib or load_library()).db_stream_read, idx, "db_stream_read", src.data_ptr(),
            nbytes, int(kb_per_wave), 0x9E3779B9, sink.data_ptr())


def tune(key: str, value: int) -> None:
    """Set a launch-geometry knob of the library (for tuning sweeps).  The
    library keeps one set of knobs per host thread: the value applies to
    the launches this thread makes."""
    _check(load_library().db_tune(key.encode(), int(value)), "db_tune")


def f4_launch_info(B: int, Hq: int, Hkv: int, L: int, S: int) -> tuple[int, int]:
    """(splits, launches) of an F4 call of this shape on the current device:
    launches is 1 when the split merge runs in the same launch (or there is
    one split), 2 when it takes a second launch."""
    s, n = C.c_int(0), C.c_int(0)
    _check(load_library().db_f4_launch_info(B, Hq, Hkv, L, S, C.byref(s), C.byref(n)),
           "db_f4_launch_info")
    return s.value, n.value


def tuned(key: str) -> int:
    """This thread's current value of a launch-geometry knob."""
    v = C.c_int(0)
    _check(load_library().db_tune_get(key.encode(), C.byref(v)), "db_tune_get")
    return v.value


def _weights(W, w_scale, name: str, N: int, K: int):
    """(dtype code, scale pointer, items to check) for an fp16 or e4m3 weight
    matrix."""
    torch = _torch or _torch_mod()
    if W.dtype == torch.float16:
        if w_scale is not None:
            raise ValueError(f"{name}: fp16 weights take no scale")
        return DTYPE_F16, None, ()
    if W.dtype in (torch.float8_e4m3fn, torch.uint8):
        if w_scale is None:
            raise ValueError(f"{name}: fp8 weights need a per-row fp32 scale")
        if not isinstance(w_scale, torch.Tensor) or tuple(w_scale.shape) != (N,):
            raise ValueError(f"{name} scale must be a tensor of shape ({N},)")
        return DTYPE_FP8_E4M3, w_scale.data_ptr(), ((w_scale, f"{name} scale", torch.float32),)
    raise TypeError(f"{name}: unsupported weight dtype {W.dtype}")


def _as_2d(x, name: str):
    if x.dim() == 1:
        return x.unsqueeze(0), True
    if x.dim() != 2:
        raise ValueError(f"{name} must be [K] or [B, K] (got {tuple(x.shape)})")
    return x, False


def f1_rmsnorm_gemv(x, g, W, eps: float = 1e-6, w_scale=None, out=None):
    """F1: ``F.linear(rmsnorm(x, g, eps), W)`` in one kernel.

    x [B,K] (or [K]) fp16, g [K] fp16, W [N,K] fp16 (or e4m3 + w_scale [N]).
    Returns [B,N] fp16 (or [N] for a 1-D x), written to ``out`` if given."""
    torch = _torch or _torch_mod()
    x2, squeeze = _as_2d(x, "x")
    B, K = x2.shape
    if W.dim() != 2 or W.shape[1] != K or g.shape != (K,):
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, g {tuple(g.shape)}, "
                         f"W {tuple(W.shape)}")
    N = W.shape[0]
    dt, sp, sc = _weights(W, w_scale, "W", N, K)
    idx = _gpu_tensors((x, "x", torch.float16), (g, "g", torch.float16), (W, "W", None), *sc)
    y = _output((B, N), idx, out)
    _launch((_lib or load_library()).db_f1_rmsnorm_gemv, idx, "db_f1_rmsnorm_gemv",
            x2.data_ptr(), g.data_ptr(), W.data_ptr(), sp, y.data_ptr(), B, K, N,
            float(eps), dt)
    return y[0] if squeeze else y


def f2_gateup_swiglu(x, Wg, Wu, sg=None, su=None, out=None):
    """F2: ``silu(F.linear(x, Wg)) * F.linear(x, Wu)`` in one kernel.

    x [B,K] (or [K]) fp16, Wg/Wu [N,K] fp16 (or e4m3 + per-row scales)."""
    torch = _torch or _torch_mod()
    x2, squeeze = _as_2d(x, "x")
    B, K = x2.shape
    if Wg.dim() != 2 or Wg.shape != Wu.shape or Wg.shape[1] != K or Wg.dtype != Wu.dtype:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, Wg {tuple(Wg.shape)}, "
                         f"Wu {tuple(Wu.shape)}")
    N = Wg.shape[0]
    dt, sgp, sgc = _weights(Wg, sg, "Wg", N, K)
    _, sup, suc = _weights(Wu, su, "Wu", N, K)
    idx = _gpu_tensors((x, "x", torch.float16), (Wg, "Wg", None), (Wu, "Wu", None), *sgc, *suc)
    y = _output((B, N), idx, out)
    _launch((_lib or load_library()).db_f2_gateup_swiglu, idx, "db_f2_gateup_swiglu",
            x2.data_ptr(), Wg.data_ptr(), Wu.data_ptr(), sgp, sup, y.data_ptr(), B, K, N, dt)
    return y[0] if squeeze else y


def f2_rmsnorm_gateup_swiglu(x, g, Wg, Wu, eps: float = 1e-6, sg=None, su=None, out=None):
    """RMSNorm -> F2 in one kernel: ``f2_gateup_swiglu(rmsnorm(x, g, eps), Wg, Wu)``
    with the normalised activations kept on chip (the post-attention half
    of the decode-layer chain).

    x [B,K] (or [K]) fp16, g [K] fp16, Wg/Wu [N,K] fp16 (or e4m3 + per-row
    scales).  Returns [B,N] fp16 (or [N])."""
    torch = _torch or _torch_mod()
    x2, squeeze = _as_2d(x, "x")
    B, K = x2.shape
    if (Wg.dim() != 2 or Wg.shape != Wu.shape or Wg.shape[1] != K or Wg.dtype != Wu.dtype
            or g.shape != (K,)):
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, g {tuple(g.shape)}, "
                         f"Wg {tuple(Wg.shape)}, Wu {tuple(Wu.shape)}")
    N = Wg.shape[0]
    dt, sgp, sgc = _weights(Wg, sg, "Wg", N, K)
    _, sup, suc = _weights(Wu, su, "Wu", N, K)
    idx = _gpu_tensors((x, "x", torch.float16), (g, "g", torch.float16), (Wg, "Wg", None),
                       (Wu, "Wu", None), *sgc, *suc)
    y = _output((B, N), idx, out)
    _launch((_lib or load_library()).db_f2_rmsnorm_gateup_swiglu, idx,
            "db_f2_rmsnorm_gateup_swiglu", x2.data_ptr(), g.data_ptr(), Wg.data_ptr(),
            Wu.data_ptr(), sgp, sup, y.data_ptr(), B, K, N, float(eps), dt)
    return y[0] if squeeze else y


def gemv(x, W, w_scale=None, out=None):
    """Plain projection ``F.linear(x, W)`` (fp16 out, fp32 accumulation)."""
    torch = _torch or _torch_mod()
    x2, squeeze = _as_2d(x, "x")
    B, K = x2.shape
    if W.dim() != 2 or W.shape[1] != K:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, W {tuple(W.shape)}")
    N = W.shape[0]
    dt, sp, sc = _weights(W, w_scale, "W", N, K)
    idx = _gpu_tensors((x, "x", torch.float16), (W, "W", None), *sc)
    y = _output((B, N), idx, out)
    _launch((_lib or load_library()).db_gemv, idx, "db_gemv",
            x2.data_ptr(), W.data_ptr(), sp, y.data_ptr(), B, K, N, dt)
    return y[0] if squeeze else y


def f4_default_splits(B: int, Hkv: int, L: int, device=None) -> int:
    return int(load_library().db_f4_default_splits(B, Hkv, L, cu_count(device)))


def f4_workspace(B: int, Hq: int, Hkv: int, L: int, D: int, S: int, device):
    """Workspace for db_f4_splitkv (None when S = 1), zero-filled when it is
    made: the split tickets of the in-launch merge must start at zero, and
    every call leaves them at zero again.

    Outside graph capture it is cached per size, device and current stream,
    so one buffer serves every later call of that size on that stream, whose
    calls run in order.  Calls on different streams get different buffers,
    so they may overlap.  torch draws streams from a fixed pool per device,
    so the cache stays bounded.

    Under graph capture each capture (each hipGraph being recorded) gets a
    workspace of its own from the graph's memory pool, shared by the calls
    of that size it records (they run in stream order on replay), never the
    cached one: graphs captured on torch's one capture stream would
    otherwise share it, and replaying two of them at once on different
    streams would mix their partial records.  Its zero fill is recorded
    into the graph ahead of the first F4 call of the capture, so a graph
    replays one small fill kernel besides its F4 launches.  Those
    workspaces stay referenced until :func:`release_captured_workspaces`,
    so the pool never hands their memory to another graph while one that
    uses it can still be replayed."""
    import torch

    nbytes = int(load_library().db_f4_workspace_bytes(B, Hq, Hkv, L, D, S))
    if nbytes == 0:
        return None
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(idx).cuda_stream
    if torch.cuda.is_current_stream_capturing():
        cid = C.c_ulonglong(0)
        _check(load_library().db_stream_capture_id(stream, C.byref(cid)),
               "db_stream_capture_id")
        key = (idx, stream, cid.value, nbytes)
        cache = _captured_ws
    else:
        key = (idx, stream, nbytes)
        cache = _ws_cache
    ws = cache.get(key)
    if ws is None:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        cache[key] = ws
    return ws


def release_captured_workspaces() -> int:
    """Drop the references to the F4 workspaces made under graph capture;
    call it once every graph that recorded F4 calls has been destroyed.
    Returns how many were released."""
    n = len(_captured_ws)
    _captured_ws.clear()
    return n


def f4_flashdecode(q, K, V, scale: float | None = None, n_splits: int | None = None,
                   workspace=None, out=None):
    """F4: split-KV GQA decode attention with the log-sum-exp merge.

    q [B,Hq,D], K/V [B,Hkv,L,D] fp16 (D = 128); query head h reads KV head
    h // (Hq // Hkv).  ``scale`` defaults to 1/sqrt(D); ``n_splits`` defaults
    to the library's CU-count-based choice.  Returns [B,Hq,D] fp16."""
    torch = _torch or _torch_mod()
    if q.dim() != 3 or K.dim() != 4 or K.shape != V.shape:
        raise ValueError(f"expected q [B,Hq,D] and K, V [B,Hkv,L,D]; got q {tuple(q.shape)}, "
                         f"K {tuple(K.shape)}, V {tuple(V.shape)}")
    B, Hq, D = q.shape
    Bk, Hkv, L, Dk = K.shape
    if Bk != B or Dk != D:
        raise ValueError(f"q {tuple(q.shape)} and K {tuple(K.shape)} disagree on B or D")
    f16 = torch.float16
    idx = _gpu_tensors((q, "q", f16), (K, "K", f16), (V, "V", f16),
                       *(((workspace, "workspace", None),) if workspace is not None else ()))
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    lib = _lib or load_library()
    S = int(lib.db_f4_default_splits(B, Hkv, L, cu_count(idx))) if n_splits is None \
        else int(n_splits)
    if workspace is None:
        workspace = f4_workspace(B, Hq, Hkv, L, D, S, idx)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    o = _output((B, Hq, D), idx, out)
    _launch(lib.db_f4_splitkv, idx, "db_f4_splitkv", q.data_ptr(), K.data_ptr(), V.data_ptr(),
            o.data_ptr(), ws_ptr, ws_bytes, B, Hq, Hkv, L, D, S, scale)
    return o


def f4_flashdecode_noalloc(q, K, V, scale: float | None = None, n_splits: int | None = None,
                           out=None):
    """F4 through ``db_f4_splitkv_noalloc``: the same kernels as
    :func:`f4_flashdecode`, with the split partials in a library-owned
    device array (``DB_F4_SCRATCH_BYTES`` per GPU) instead of a workspace,
    so the library allocates nothing.  Pass ``out`` ([B,Hq,D] fp16,
    contiguous) to allocate nothing on the Python side either.

    Every call on one GPU shares that array: calls that overlap in time on
    one GPU (concurrent streams or concurrently replayed graphs) race.  Make
    the first call on a device outside graph capture (it looks up the
    array's device address)."""
    torch = _torch or _torch_mod()
    if q.dim() != 3 or K.dim() != 4 or K.shape != V.shape:
        raise ValueError(f"expected q [B,Hq,D] and K, V [B,Hkv,L,D]; got q {tuple(q.shape)}, "
                         f"K {tuple(K.shape)}, V {tuple(V.shape)}")
    B, Hq, D = q.shape
    Bk, Hkv, L, Dk = K.shape
    if Bk != B or Dk != D:
        raise ValueError(f"q {tuple(q.shape)} and K {tuple(K.shape)} disagree on B or D")
    f16 = torch.float16
    idx = _gpu_tensors((q, "q", f16), (K, "K", f16), (V, "V", f16))
    out = _output((B, Hq, D), idx, out)
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    lib = _lib or load_library()
    S = int(lib.db_f4_default_splits(B, Hkv, L, cu_count(idx))) if n_splits is None \
        else int(n_splits)
    _launch(lib.db_f4_splitkv_noalloc, idx, "db_f4_splitkv_noalloc", q.data_ptr(), K.data_ptr(),
            V.data_ptr(), out.data_ptr(), B, Hq, Hkv, L, D, S, scale)
    return out
