"""The ctypes stub INTEGRATION.md tells a maintainer of the reference to add
(its section 2), run exactly as printed there.

The stub is the reference-side binding of the C ABI: what a maintainer
drops into the reference as ``src/decodebench/hip_fused.py`` in place of the
torch extension of examples/custom_kernel/bindings.cpp:13-30.  These tests
take its code block out of INTEGRATION.md, point its ``CDLL`` at the library
built here and execute it as a module, then hold its f1, f2 and f4 to the
same oracle bars as the parity tests, and replay two captured F4 graphs
concurrently (each capture must get its own workspace).
"""

import math
import re
import types
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
STUB_PATH = "/path/to/decodebench_amd/lib/libdecodebench_hip.so"
STUB_HEADING = "## 2. The ctypes stub the reference would add"


def stub_source() -> str:
    text = DOC.read_text()
    sec = text[text.index(STUB_HEADING):]
    m = re.search(r"```python\n(.*?)```", sec, flags=re.S)
    assert m, "INTEGRATION.md section 2 has no python block"
    return m.group(1)


def test_stub_is_python_and_binds_declared_symbols():
    """The stub compiles, loads the library from the path the doc names, and
    every library function it sets up is declared in include/*.h."""
    src = stub_source()
    compile(src, "hip_fused.py", "exec")
    assert STUB_PATH in src
    used = set(re.findall(r"_lib\.(db_\w+)", src))
    headers = "\n".join(h.read_text() for h in (ROOT / "include").glob("*.h"))
    declared = set(re.findall(r"\b(db_\w+)\s*\(", re.sub(r"/\*.*?\*/", "", headers, flags=re.S)))
    assert used and used <= declared, used - declared


torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def stub():
    from decodebench_amd import ops

    ops.load_library()                      # builds nothing; raises if the library is missing
    mod = types.ModuleType("hip_fused")
    exec(compile(stub_source().replace(STUB_PATH, str(ops.LIB_PATH)), "hip_fused.py", "exec"),
         mod.__dict__)
    return mod


def _randn(gen, shape, std=1.0, mean=0.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * std + mean).half()


def _rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _check(got, stage_ref, exact, rel_bound, what):
    g = got.float().cpu().numpy().astype(np.float64)
    r = stage_ref.float().numpy().astype(np.float64)
    assert np.isclose(g, r, rtol=1e-2, atol=1e-2).all(), f"{what}: outside rtol/atol 1e-2"
    assert _rel_l2(g, exact) <= rel_bound, f"{what}: rel-L2 {_rel_l2(g, exact):.2e}"


@pytest.mark.gpu
@pytest.mark.parametrize("fp8", [False, True])
def test_stub_f1_matches_the_oracle(stub, fp8):
    from decodebench_amd.quant import quantize_e4m3_rows
    from oracle import cref, stages

    print(f"[stub] f1 fp8={fp8}", flush=True)
    gen = torch.Generator().manual_seed(8101 + fp8)
    x = _randn(gen, (1, 4096))
    g = _randn(gen, (4096,), std=0.1, mean=1.0)
    W = _randn(gen, (4096, 4096), std=1 / 64)
    if fp8:
        Wq, s = quantize_e4m3_rows(W)
        y = stub.f1(x.cuda(), g.cuda(), Wq.cuda(), scale=s.cuda())
        torch.cuda.synchronize()
        ref = stages.f1_fp8(x, g, Wq, s)
        exact = cref.f1_fp8_exact(x.numpy(), g.numpy(), Wq.view(torch.uint8).numpy(), s.numpy())
    else:
        y = stub.f1(x.cuda(), g.cuda(), W.cuda())
        torch.cuda.synchronize()
        ref = stages.f1(x, g, W)
        exact = cref.f1_exact(x.numpy(), g.numpy(), W.numpy())
    _check(y, ref, exact, 2e-3, f"stub f1 fp8={fp8}")


@pytest.mark.gpu
def test_stub_f2_matches_the_oracle(stub):
    from oracle import cref, stages

    print("[stub] f2", flush=True)
    gen = torch.Generator().manual_seed(8201)
    x = _randn(gen, (1, 4096))
    Wg = _randn(gen, (2048, 4096), std=0.02)
    Wu = _randn(gen, (2048, 4096), std=0.02)
    y = stub.f2(x.cuda(), Wg.cuda(), Wu.cuda())
    torch.cuda.synchronize()
    _check(y, stages.f2(x, Wg, Wu), cref.f2_exact(x.numpy(), Wg.numpy(), Wu.numpy()), 2e-3,
           "stub f2")


def _f4_inputs(B, L, seed):
    gen = torch.Generator().manual_seed(seed)
    return (_randn(gen, (B, 32, 128)), _randn(gen, (B, 8, L, 128)), _randn(gen, (B, 8, L, 128)))


@pytest.mark.gpu
@pytest.mark.parametrize("B,L", [(1, 8192), (2, 1000), (1, 16)])
def test_stub_f4_matches_the_oracle(stub, B, L):
    from oracle import cref

    print(f"[stub] f4 B={B} L={L}", flush=True)
    q, K, V = _f4_inputs(B, L, 8300 + B + L)
    o = stub.f4(q.cuda(), K.cuda(), V.cuda())
    again = stub.f4(q.cuda(), K.cuda(), V.cuda())    # the cached workspace, reused
    torch.cuda.synchronize()
    assert torch.equal(o, again)
    exact = cref.attention(q.numpy(), K.numpy(), V.numpy())
    assert _rel_l2(o.float().cpu().numpy(), exact) <= 5e-3


@pytest.mark.gpu
def test_stub_f4_graphs_replayed_concurrently(stub):
    """Two graphs captured on torch's one capture stream, each recording
    stub F4 calls, replayed at the same time on two streams: each capture has
    its own workspace, so every replay gives the eager results."""
    print("[stub] f4 graphs", flush=True)
    inputs = [tuple(t.cuda() for t in _f4_inputs(1, 8192, 8400 + i)) for i in range(2)]
    want = [stub.f4(*d) for d in inputs]
    torch.cuda.synchronize()
    graphs, outs = [], []
    for d in inputs:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            o = [stub.f4(*d) for _ in range(4)]
        graphs.append(g)
        outs.append(o)
    assert len(stub._captured) == 2                  # one workspace per capture
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(6):
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for g, s in zip(graphs, streams):
            with torch.cuda.stream(s):
                g.replay()
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for i in range(2):
            for o in outs[i]:
                assert torch.equal(o, want[i]), f"graph {i}, replay {rep}"
    del graphs
    torch.cuda.synchronize()
    stub.release_captured()
    assert not stub._captured
    # the scale argument, as the reference stage passes it (1/sqrt(D) by default)
    q, K, V = inputs[0]
    assert torch.equal(stub.f4(q, K, V, scale=1.0 / math.sqrt(128)), want[0])
