"""The allocation-free F4 entry point against the workspace one, on the GPU.

``db_f4_splitkv_noalloc`` keeps its split partials in a library-owned device
array instead of a caller workspace and always merges them in a second
launch.  It runs the same kernels as ``db_f4_splitkv`` with its merge in a
second launch (``f4_merge`` = 2), so on the same inputs and split count the
two outputs must be bit-identical; against the default in-launch merge of
``db_f4_splitkv`` they agree to fp32 summation order.  Two calls in a row,
the second smaller, show that whatever the first call left in the array
does not leak into the second.  Both calls go through the C ABI (ctypes), as
a caller that cannot allocate would make them.
"""

import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from decodebench_amd import ops  # noqa: E402
from oracle import cref  # noqa: E402

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, L, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, 128, generator=gen).half().cuda()
    K = torch.randn(B, Hkv, L, 128, generator=gen).half().cuda()
    V = torch.randn(B, Hkv, L, 128, generator=gen).half().cuda()
    return q, K, V


def _noalloc_call(q, K, V, S, out):
    lib = ops.load_library()
    B, Hq, D = q.shape
    Hkv, L = K.shape[1], K.shape[2]
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.db_f4_splitkv_noalloc(q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(),
                                   B, Hq, Hkv, L, D, S, 1.0 / math.sqrt(D), stream)
    assert rc == 0, lib.db_last_error().decode()


# (B, Hq, Hkv, L, S): the second case of each pair is the smaller input
SEQUENCES = [
    ((4, 32, 8, 8192, None), (1, 32, 8, 1024, None)),
    ((1, 32, 8, 32768, None), (2, 16, 2, 700, 16)),
]


def _two_launch(q, K, V, S):
    """db_f4_splitkv with its split merge in a second launch."""
    try:
        ops.tune("f4_merge", 2)
        return ops.f4_flashdecode(q, K, V, n_splits=S)
    finally:
        ops.tune("f4_merge", 0)


def _rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("first,second", SEQUENCES)
def test_noalloc_matches_workspace_entry_point(first, second):
    for i, (B, Hq, Hkv, L, S) in enumerate((first, second)):
        print(f"[noalloc] call {i}: B={B} Hq={Hq} Hkv={Hkv} L={L} S={S}", flush=True)
        q, K, V = _inputs(B, Hq, Hkv, L, 7100 + 13 * i + L + B)
        S_eff = ops.f4_default_splits(B, Hkv, L, q.device) if S is None else S
        want = _two_launch(q, K, V, S_eff)
        default = ops.f4_flashdecode(q, K, V, n_splits=S_eff)
        got = torch.full_like(want, float("nan"))
        _noalloc_call(q, K, V, S_eff, got)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (
            f"call {i}: noalloc differs from db_f4_splitkv "
            f"(max abs {float((got.float() - want.float()).abs().max()):.3e})")
        assert _rel(got, default) < 1e-3
        if L <= 1024:
            exact = cref.attention(q.cpu().numpy(), K.cpu().numpy(), V.cpu().numpy())
            err = np.linalg.norm(got.float().cpu().numpy() - exact) / np.linalg.norm(exact)
            assert err <= 5e-3, f"call {i}: rel-L2 {err:.3e} against the exact oracle"


def _free_device_bytes():
    free, _ = torch.cuda.mem_get_info()
    return free


def test_noalloc_python_op_with_out_allocates_nothing_in_the_library():
    """After a warm-up call, a call into the caller's ``out`` changes neither
    torch's allocated bytes nor the device's free memory (hipMemGetInfo), and
    writes exactly ``out``."""
    q, K, V = _inputs(1, 32, 8, 4096, 7301)
    out = torch.empty(1, 32, 128, dtype=torch.float16, device="cuda")
    ops.f4_flashdecode_noalloc(q, K, V, out=out)       # warm-up: symbol lookup
    torch.cuda.synchronize()
    alloc0, free0 = torch.cuda.memory_allocated(), _free_device_bytes()
    res = ops.f4_flashdecode_noalloc(q, K, V, out=out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc0
    assert _free_device_bytes() == free0
    assert res.data_ptr() == out.data_ptr()
    want = _two_launch(q, K, V, ops.f4_default_splits(1, 8, 4096, q.device))
    torch.cuda.synchronize()
    assert torch.equal(res, want)


def test_noalloc_ignores_the_merge_knobs_and_a_dirty_scratch_array():
    """The allocation-free entry point always merges in a second launch, so
    neither f4_merge nor f4_misplace changes its output, and records another
    shape left in the scratch array do not leak into a later call."""
    q, K, V = _inputs(2, 32, 8, 2048, 7401)
    S = ops.f4_default_splits(2, 8, 2048, q.device)
    want = _two_launch(q, K, V, S)
    big = _inputs(8, 64, 8, 4096, 7402)                  # fills the array with other records
    scratch_out = torch.empty(8, 64, 128, dtype=torch.float16, device="cuda")
    _noalloc_call(*big, ops.f4_default_splits(8, 8, 4096, q.device), scratch_out)
    outs = []
    try:
        for merge, misplace in ((1, 0), (0, 1), (2, 3)):
            ops.tune("f4_merge", merge)
            ops.tune("f4_misplace", misplace)
            got = torch.full_like(want, float("nan"))
            _noalloc_call(q, K, V, S, got)
            outs.append(got)
    finally:
        ops.tune("f4_merge", 0)
        ops.tune("f4_misplace", 0)
    torch.cuda.synchronize()
    for got in outs:
        assert torch.equal(got, want)
