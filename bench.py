"""Benchmark of the fused decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Prints ONE JSON line.  The headline workload is the benchmark's config 2 at batch 1:
F2 = gate/up GEMV + SwiGLU, x[1,4096] fp16, Wg/Wu[14336,4096] fp16 ~N(0,0.02).
A step is one fused launch over a fresh weight replica; the replicas rotate
through a working set larger than twice the on-die caches (8 x 4 MB L2 plus
the 256 MB Infinity Cache), so every step streams its weights from HBM.

  value          algorithmic bytes / (timed region / K), GB/s
  roofline       the F2 kernel against the 8 TB/s HBM3E peak; its average
                 launch duration is the same event-timed region on the
                 stream the kernel runs on (torch's current stream)
  roofline_by_kernel  F1 (configs 1 and 3), F2 and F4 (L = 8192, 32768) at
                 batch 1 against the 8 TB/s peak, from the kernels table, with
                 the committed rocprofv3 kernel-trace medians beside them
  kernels        F1 (config 1 and the QKV shape of config 3), F2 and F4
                 (config 4 at L = 1024 / 8192 / 32768) with their batch and
                 split sweeps, the fp8 e4m3-weight F1/F2 and the config-5
                 decode layer (fp16 and fp8), each timed as back-to-back
                 calls replayed from a hipGraph
  decomposition  Sequence.profile of the unfused torch stages (stream and
                 graph) against the fused kernels: Delta_launch and B, for
                 F1, F2, F4 and the decode layer (fp16 and fp8 weights),
                 with the per-trial samples and a fused-vs-unfused output
                 check that decodebench_amd.validate reads
  cpu_baseline   the torch CPU restatement of the reference stages
                 (oracle/stages.py) on this host's cores: F2 at full size
                 (the headline), with F1 (config 1) and F4 (L = 8192) rows

``--gpus N`` with N > 1 exits with an error: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import contextlib
import json
import math
import os
import platform
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense fp16 MFMA, MI355X
METRIC = ("fused kernel µs + HBM GB/s (% of ~8 TB/s) for F1/F2/F4 at bs=1; "
          "Δ_launch vs B")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--quick", action="store_true",
                    help="headline only: skip the per-kernel table, the "
                         "decomposition and the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bound on the CPU baseline sample")
    ap.add_argument("--trials", type=int, default=30,
                    help="trials per variant in the decomposition (the validation report "
                         "needs >= 30)")
    ap.add_argument("--profile-pass", metavar="MANIFEST",
                    help="run the workload for rocprofv3 instead: calibration copies, then "
                         "every fused workload and the decomposition configs' unfused stage "
                         "chains eagerly, each between two delimiter kernels; write the launch "
                         "manifest to MANIFEST and exit")
    ap.add_argument("--graph", action="store_true",
                    help="with --profile-pass: replay each fused workload's calls from one "
                         "hipGraph (back-to-back launches for the kernel trace)")
    ap.add_argument("--isolated", action="store_true",
                    help="with --profile-pass: synchronise after every fused call, so each "
                         "launch runs alone (its kernel-trace duration is execution time)")
    ap.add_argument("--calls", type=int, default=24,
                    help="with --profile-pass: calls per workload segment")
    ap.add_argument("--sweep-only", metavar="REGEX",
                    help="per-kernel table restricted to matching workloads; skips the "
                         "decomposition and the CPU baseline")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="rocprofv3 traffic summary (decodebench_amd.rocprof) for roofline.traffic")
    ap.add_argument("--kernel-trace", default=os.path.join(ROOT, "profiles",
                                                           "kernel_trace_b1.json"),
                    help="rocprofv3 graph-replay kernel-trace summary for roofline_by_kernel")
    ap.add_argument("--kernel-trace-isolated",
                    default=os.path.join(ROOT, "profiles", "kernel_trace_isolated_b1.json"),
                    help="rocprofv3 kernel-trace summary of isolated launches (one call, then a "
                         "sync) for roofline_by_kernel")
    return ap.parse_args(argv)


# ----------------------------------------------------------------- timing
def time_steps(case, steps: int, warmup: int, settle_ms: float = 20.0):
    """Eager launches, one per step, replica i % n; returns seconds.

    Before the ``warmup`` steps the GPU is kept busy with about ``settle_ms``
    of the same launches (untimed, not counted as steps), so that a short
    timed region (the driver's 20 steps are 0.7 ms) does not start while the
    clocks are still ramping up from the parity check."""
    import torch

    reps = case.replicas
    n = len(reps)
    t0 = time.perf_counter()
    i = 0
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        case.fused(reps[i % n])
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    for i in range(warmup):
        case.fused(reps[i % n])
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        case.fused(reps[i % n])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


def time_graph_launches(case, min_launches: int = 96, replays: int = 20):
    """Per-launch microseconds of the fused kernel, back-to-back in a graph.

    One graph holds whole rotations over the replicas, so the host never
    throttles the launch rate; returns the median over ``replays``."""
    import torch

    reps = case.replicas
    n = len(reps)
    per_graph = n * max(1, math.ceil(min_launches / n))
    for r in reps:                       # allocations (F4 workspace) happen here
        case.fused(r)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n):
            case.fused(reps[i])
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            case.fused(reps[i % n])
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    samples = []
    for _ in range(replays):
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        samples.append(e0.elapsed_time(e1) * 1e3 / per_graph)
    samples.sort()
    del graph
    torch.cuda.synchronize()
    from decodebench_amd import ops

    ops.release_captured_workspaces()
    return samples[len(samples) // 2], per_graph


CHECK_REL_L2 = 1e-2
# The decode-layer chain compounds twelve fp16 rounding points; two correct
# implementations of it differ by up to 1.6e-2 elementwise, so it is held to
# the parity tests' chain tolerance (each of its kernels meets 1e-2 alone).
CHECK_TOL = {"layer": 2e-2}


def check_case(case) -> float:
    """Fused output vs the unfused torch stages on the GPU: rtol/atol 1e-2
    elementwise (2e-2 for the decode-layer chain), and relative L2 <= 1e-2,
    which an all-zero output fails also where |o| is below atol (F4 at long
    KV lengths)."""
    import torch

    ref = case.seq._replay_body(case.inputs).float()
    out = case.fused(case.inputs).float()
    torch.cuda.synchronize()
    err = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
    tol = CHECK_TOL.get(case.name, 1e-2)
    if not torch.allclose(out, ref, rtol=tol, atol=tol) or not err <= CHECK_REL_L2:
        raise RuntimeError(f"{case.name}: fused output differs from the torch stages "
                           f"(max abs {float((out - ref).abs().max()):.3e}, rel-L2 {err:.3e})")
    return err


def fused_check(case) -> dict:
    """The fused output against the unfused torch stages on the same inputs,
    with Sequence.profile's elementwise bar (abs < 5e-2 or rel < 2e-2)."""
    import torch

    from decodebench_amd.sequence import _FUSED_ABS_TOL, _FUSED_REL_TOL

    ref = case.seq._replay_body(case.replicas[0]).float()
    out = case.fused(case.replicas[0]).float()
    err = (out - ref).abs()
    rel = err / ref.abs().clamp_min(1e-12)
    ok = bool(((err < _FUSED_ABS_TOL) | (rel < _FUSED_REL_TOL)).all())
    torch.cuda.synchronize()
    return {"ok": ok, "max_abs": float(err.max()),
            "rel_l2": float((out - ref).norm() / ref.norm().clamp_min(1e-30))}


def kernel_row(case, us: float) -> dict:
    gbs = case.algorithmic_bytes / (us * 1e-6) / 1e9
    tflops = case.flops / (us * 1e-6) / 1e12
    return {"us": round(us, 3), "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "TFLOP/s": round(tflops, 2), "frac_mfma_f16": round(tflops / MFMA_F16_PEAK_TFLOPS, 5),
            "algorithmic_bytes": case.algorithmic_bytes, "flops": case.flops,
            "replicas": len(case.replicas), "shape": case.shape}


def sweep_workloads():
    """Benchmark configs 1-4 with their batch, KV-length and split sweeps."""
    out = [("f1_cfg1", dict(name="f1", batch=1))]
    for B in (1, 4, 8, 16, 32):
        out.append((f"f1_qkv_cfg3" + ("" if B == 1 else f"_B{B}"), dict(name="f1_qkv", batch=B)))
    for B in (1, 4, 16):
        out.append((f"f2_cfg2" + ("" if B == 1 else f"_B{B}"), dict(name="f2", batch=B)))
    for L in (1024, 8192, 32768):
        for B in (1, 4, 8):
            out.append((f"f4_L{L}" + ("" if B == 1 else f"_B{B}"), dict(name="f4", L=L, batch=B)))
    for S in (1, 4, 16, 64):
        out.append((f"f4_L8192_S{S}", dict(name="f4", L=8192, batch=1, n_splits=S)))
    # F4 with its split merge in a second launch, the form the reference times
    # (f4_partial_kernel + f4_reduce_kernel): the fallback when a call cannot
    # merge in its first launch
    for L in (8192, 32768):
        out.append((f"f4_L{L}_2launch", dict(name="f4", L=L, batch=1, tune={"f4_merge": 2})))
    # each half of that pair alone, back to back (db_tune f4_launch): the split
    # kernel, then the merge (reading whatever records its workspace holds, so
    # no parity check); their times add up to the pair's
    for L in (8192, 32768):
        for half, only in (("split", 1), ("merge", 2)):
            out.append((f"f4_L{L}_2launch_{half}",
                        dict(name="f4", L=L, batch=1, tune={"f4_merge": 2, "f4_launch": only},
                             check=False)))
    # fp8 e4m3 weights (per-row scales) at batch 1, and the config-5 layer
    out += [("f1_cfg1_fp8", dict(name="f1", batch=1, dtype="fp8")),
            ("f1_qkv_cfg3_fp8", dict(name="f1_qkv", batch=1, dtype="fp8")),
            ("f2_cfg2_fp8", dict(name="f2", batch=1, dtype="fp8"))]
    out += [(f"f1_qkv_cfg3_fp8_B{B}", dict(name="f1_qkv", batch=B, dtype="fp8"))
            for B in (4, 8, 16, 32)]
    out += [(f"f2_cfg2_fp8_B{B}", dict(name="f2", batch=B, dtype="fp8")) for B in (4, 16)]
    out += [
            ("layer_cfg5", dict(name="layer", batch=1, L=8192)),
            ("layer_cfg5_fp8", dict(name="layer", batch=1, L=8192, dtype="fp8"))]
    return out


# ------------------------------------------------------------ profile pass
PROFILE_WORKLOADS = (("f1_cfg1", dict(name="f1")), ("f1_qkv_cfg3", dict(name="f1_qkv")),
                     ("f2_cfg2", dict(name="f2")), ("f4_L1024", dict(name="f4", L=1024)),
                     ("f4_L8192", dict(name="f4", L=8192)), ("f4_L32768", dict(name="f4", L=32768)),
                     ("f4_L8192_2launch", dict(name="f4", L=8192, tune={"f4_merge": 2})),
                     ("f4_L32768_2launch", dict(name="f4", L=32768, tune={"f4_merge": 2})),
                     ("f4_L8192_2launch_split",
                      dict(name="f4", L=8192, tune={"f4_merge": 2, "f4_launch": 1}, check=False)),
                     ("f4_L8192_2launch_merge",
                      dict(name="f4", L=8192, tune={"f4_merge": 2, "f4_launch": 2}, check=False)),
                     ("f4_L32768_2launch_split",
                      dict(name="f4", L=32768, tune={"f4_merge": 2, "f4_launch": 1}, check=False)),
                     ("f4_L32768_2launch_merge",
                      dict(name="f4", L=32768, tune={"f4_merge": 2, "f4_launch": 2}, check=False)),
                     ("f1_cfg1_fp8", dict(name="f1", dtype="fp8")),
                     ("f1_qkv_cfg3_fp8", dict(name="f1_qkv", dtype="fp8")),
                     ("f2_cfg2_fp8", dict(name="f2", dtype="fp8")),
                     ("layer_cfg5", dict(name="layer", L=8192)),
                     ("layer_cfg5_fp8", dict(name="layer", L=8192, dtype="fp8")),
                     ("f1_qkv_cfg3_B16", dict(name="f1_qkv", batch=16)),
                     ("f1_qkv_cfg3_B32", dict(name="f1_qkv", batch=32)),
                     ("f2_cfg2_B16", dict(name="f2", batch=16)),
                     ("f2_cfg2_fp8_B16", dict(name="f2", batch=16, dtype="fp8")))

# The decomposition configs: Sequence.profile of the torch stages against
# the fused call; their unfused stage chains are also profiled (τ_u and the
# unfused bytes of decodebench_amd.validate).
DECOMP_WORKLOADS = (("f1_cfg1", dict(name="f1")), ("f2_cfg2", dict(name="f2")),
                    ("f4_L8192", dict(name="f4", L=8192)),
                    ("layer_cfg5", dict(name="layer", L=8192)),
                    ("layer_cfg5_fp8", dict(name="layer", L=8192, dtype="fp8")))


@contextlib.contextmanager
def knobs(kw: dict):
    """Apply a workload's launch-geometry knobs (kw["tune"]) for the calls
    made inside, and restore the previous values after."""
    from decodebench_amd import ops

    tune = kw.get("tune") or {}
    old = {k: ops.tuned(k) for k in tune}
    try:
        for k, v in tune.items():
            ops.tune(k, v)
        yield
    finally:
        for k, v in old.items():
            ops.tune(k, v)


def case_args(kw: dict) -> dict:
    """build_config arguments of a workload (its knobs and check flag removed)."""
    return {k: v for k, v in kw.items() if k not in ("tune", "check")}


def f4_launches(L: int, n_splits=None, batch: int = 1) -> int:
    """Launches of one F4 call as the library plans it on this device: 1 (one
    split, or the split merge in the same launch) or 2 (merge in a second
    launch)."""
    from decodebench_amd import ops
    from decodebench_amd.demos.llama_decode import LAYER

    S = ops.f4_default_splits(batch, LAYER["Hkv"], L) if n_splits is None else n_splits
    return ops.f4_launch_info(batch, LAYER["Hq"], LAYER["Hkv"], L, S)[1]


def kernels_per_call(kw: dict) -> int:
    """Kernel launches of one fused call (F4 is one or two, see f4_launches;
    the decode layer is F1, F4, O GEMV, RMSNorm+F2 and the down GEMV)."""
    B = kw.get("batch", 1)
    if kw["name"] == "f4":
        return f4_launches(kw.get("L", 8192), kw.get("n_splits"), B)
    if kw["name"] == "layer":
        return 4 + f4_launches(kw.get("L", 8192), None, B)
    return 1


def f4_partial_bytes(kw: dict, batch: int = 1) -> int:
    """HBM bytes a fused F4 call adds over a single-pass kernel: the split
    partial records (o, m, l per head and split, fp32).  Merged in the same
    launch they are read back from the XCD's L2, so only their write-back
    reaches HBM; merged by a second launch they are also read back from
    memory."""
    from decodebench_amd import ops
    from decodebench_amd.demos.llama_decode import LAYER

    if kw["name"] not in ("f4", "layer"):
        return 0
    Hq, Hkv, D = LAYER["Hq"], LAYER["Hkv"], LAYER["D"]
    L = kw.get("L", 8192)
    S = ops.f4_default_splits(batch, Hkv, L)
    if S <= 1:
        return 0
    passes = f4_launches(L, None, batch)   # 1: write only, 2: write and read
    return passes * batch * Hq * S * (D + 2) * 4


def profile_pass(manifest_path: str, calls: int = 24, warmup: int = 4,
                 graph: bool = False, isolated: bool = False) -> int:
    """Launch sequence for decodebench_amd.rocprof: calibration kernels first
    (``copy_calls`` device copies of ``copy_bytes``, which read and write that
    many bytes, then ``read_calls`` launches of the read-only streaming probe
    over ``read_bytes``), then each workload's calls over cache-defeating
    replicas, between two launches of the library's empty kernel (the segment
    delimiters).  The fused calls of every profile workload come first, then
    the unfused torch stage chains of the decomposition configs.

    Eager (default): the calls are launched one by one, with two warm-up
    calls before each segment, outside its delimiters.  ``graph=True``: the
    fused calls of a workload are captured into one hipGraph, replayed once
    as warm-up, and then replayed between the delimiters, so the kernel
    trace shows back-to-back launches with no host gaps (the unfused chains
    stay eager).  ``isolated=True``: every fused call is followed by a
    device synchronisation, so each launch runs alone on an idle GPU and the
    kernel trace gives its execution time apart from any launch boundary
    (the reference's single-launch timing, bench_variant.cu:441-469)."""
    import torch

    from decodebench_amd import ops
    from decodebench_amd.bytes_model import eliminable_bytes, total_bytes
    from decodebench_amd.demos.llama_decode import build_config

    def segment(body, n, sync=False):
        for i in range(2):
            body(n - 1 - i)  # warm-up, on replicas the first calls do not use first
        torch.cuda.synchronize()
        ops.null_kernel()
        for i in range(calls):
            body(i)
            if sync:
                torch.cuda.synchronize()
        ops.null_kernel()
        torch.cuda.synchronize()

    def graph_segment(case):
        reps = case.replicas
        n = len(reps)
        for r in reps:                  # first calls (workspaces) outside the capture
            case.fused(r)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(calls):
                case.fused(reps[i % n])
        g.replay()                      # warm-up replay
        torch.cuda.synchronize()
        ops.null_kernel()
        g.replay()
        ops.null_kernel()
        torch.cuda.synchronize()
        del g
        ops.release_captured_workspaces()

    ops.load_library()
    copy_bytes, copy_calls = 512 << 20, 3
    src = torch.empty(copy_bytes, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(copy_calls):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    read_bytes, read_calls, read_kb = 512 << 20, 3, 4
    zeros = torch.zeros(read_bytes, dtype=torch.uint8, device="cuda")
    sink = torch.empty(read_bytes // 16, dtype=torch.int32, device="cuda")
    for _ in range(read_calls):
        ops.stream_read(zeros, read_kb, sink)
    torch.cuda.synchronize()
    del zeros, sink
    workloads = []
    for label, kw in PROFILE_WORKLOADS:
        case = build_config(gen_device="cuda", **{"batch": 1, **case_args(kw)})
        n = len(case.replicas)
        with knobs(kw):
            if graph:
                graph_segment(case)
            else:
                segment(lambda i: case.fused(case.replicas[i % n]), n, sync=isolated)
            per_call = kernels_per_call(kw)
        workloads.append({"label": label, "kind": "fused", "calls": calls, "warmup": warmup,
                          "kernels_per_call": per_call,
                          "algorithmic_bytes": case.algorithmic_bytes})
        log(f"profile pass: {label} x {calls}" + (" (graph)" if graph else "")
            + (" (isolated)" if isolated else ""))
        del case
        torch.cuda.empty_cache()
    for label, kw in DECOMP_WORKLOADS:
        case = build_config(gen_device="cuda", **{"batch": 1, **kw})
        traces = case.seq.trace(case.inputs)
        n = len(case.replicas)
        # the stage chain as Sequence.profile's stream variant runs it
        segment(lambda i: case.seq._replay_body(case.replicas[i % n]), n)
        workloads.append({"label": f"{label}_unfused", "kind": "unfused", "calls": calls,
                          "warmup": warmup, "kernels_per_call": None,
                          "algorithmic_bytes": total_bytes(traces),
                          "eliminable_bytes": eliminable_bytes(traces)})
        log(f"profile pass: {label}_unfused x {calls}")
        del case
        torch.cuda.empty_cache()
    with open(manifest_path, "w") as f:
        json.dump({"copy_bytes": copy_bytes, "copy_calls": copy_calls,
                   "read_bytes": read_bytes, "read_calls": read_calls, "read_kb_per_wave": read_kb,
                   "mode": "graph" if graph else ("isolated" if isolated else "eager"),
                   "delimiter": "null_kernel", "workloads": workloads}, f, indent=1)
    return 0


# The batch-1 kernels the metric names (F1 at configs 1 and 3, F2, F4), with the
# kernel names of their launches.
ROOFLINE_KERNELS = (("f1_cfg1", "gemv_kernel<1,...> (F1 RMSNorm mode)"),
                    ("f1_qkv_cfg3", "gemv_kernel<1,...> (F1 RMSNorm mode)"),
                    ("f2_cfg2", "gemv_kernel<2,...> (F2 SwiGLU mode)"),
                    ("f4_L8192", "f4_kernel<4,8,...> (split merge in the same launch)"),
                    ("f4_L32768", "f4_kernel<4,8,...> (split merge in the same launch)"))


def two_launch_parts(kernels: dict) -> dict:
    """The two-launch F4 pair against its halves timed alone back to back:
    split kernel + merge (µs per launch) and their sum next to the pair's
    time per call."""
    out = {}
    for L in (8192, 32768):
        pair, split, merge = (kernels.get(f"f4_L{L}_2launch{sfx}")
                              for sfx in ("", "_split", "_merge"))
        if pair and split and merge:
            total = split["us"] + merge["us"]
            out[f"L{L}"] = {"split_us": split["us"], "merge_us": merge["us"],
                            "sum_us": round(total, 3), "pair_us": pair["us"],
                            "sum_minus_pair_us": round(total - pair["us"], 3)}
    return out


def load_kernel_trace(path: str) -> dict:
    try:
        with open(path) as f:
            return json.load(f).get("workloads", {})
    except (OSError, ValueError):
        return {}


def roofline_by_kernel(kernels: dict, traffic: dict, trace: dict, isolated: dict | None = None) -> dict:
    """Per batch-1 kernel: algorithmic bytes / its average launch time
    against 8 TB/s.  ``us`` is this run's event-timed average over
    back-to-back launches replayed from a hipGraph; ``rocprof_us`` is the
    committed rocprofv3 kernel-trace median of the same calls replayed the
    same way (profiles/kernel_trace_b1.md, profiler overhead included), a
    launch-to-launch figure; ``rocprof_isolated_us`` the median duration of
    single launches on an idle GPU (profiles/kernel_trace_isolated_b1.md),
    the kernel's own execution time; ``traffic`` the committed read bytes by
    request size + WRITE_SIZE per call."""
    out = {}
    for name, kernel in ROOFLINE_KERNELS:
        k = kernels.get(name)
        if not k:
            continue
        achieved = k["GB/s"]
        row = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
               "frac": round(achieved / HBM_PEAK_GBS, 4), "us": k["us"],
               "algorithmic_bytes": k["algorithmic_bytes"], "kernel": kernel,
               "traffic": traffic.get(name, {}).get("traffic_bytes"),
               "bar_70pct_us": round(k["algorithmic_bytes"] / (0.7 * HBM_PEAK_GBS * 1e3), 3)}
        t = trace.get(name, {})
        if "call_us" in t:
            row["rocprof_us"] = round(t["call_us"], 3)
            row["rocprof_kernel_us"] = {kk.split("::")[-1]: round(v, 3)
                                        for kk, v in t.get("kernel_us", {}).items()}
        ti = (isolated or {}).get(name, {})
        if "call_us" in ti:
            row["rocprof_isolated_us"] = round(ti["call_us"], 3)
        out[name] = row
    return out


def load_traffic(path: str) -> dict:
    try:
        with open(path) as f:
            return json.load(f).get("workloads", {})
    except (OSError, ValueError):
        return {}


# ------------------------------------------------------------ CPU baseline
def _cpu_model() -> str:
    name = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return name


def cpu_threads() -> int:
    """Threads for the CPU baseline: every CPU this process may run on, capped
    by OMP_NUM_THREADS when the host sets it (the GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _time_cpu(fn, reps: list, seconds: float) -> tuple[float, int]:
    """Median seconds per call of fn(*reps[i % n]) over about ``seconds``."""
    fn(*reps[0])  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        args = reps[len(times) % len(reps)]
        t0 = time.perf_counter()
        fn(*args)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(seconds: float) -> dict:
    """The torch CPU restatement of the reference stages (oracle/stages.py),
    time-bounded, on this host's cores: F2 (config 2, B = 1, the headline
    workload; ``seconds``), and beside it F1 (config 1) and F4 (config 4,
    L = 8192), a third of ``seconds`` each.  Calls rotate over replicas of the
    large operands (F2: 3, 705 MB) so the sample is not served from a large
    host L3."""
    import torch

    from oracle import stages

    threads = cpu_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(42)
    K, N = 4096, 14336
    x = torch.randn(1, K, generator=gen).half()
    Wg = (torch.randn(N, K, generator=gen) * 0.02).half()
    Wu = (torch.randn(N, K, generator=gen) * 0.02).half()
    f2_reps = [(x, Wg, Wu)] + [(x, Wg.clone(), Wu.clone()) for _ in range(2)]
    f2_bytes = 2 * N * K * 2 + (K + N) * 2
    med, calls = _time_cpu(stages.f2, f2_reps, seconds)
    del f2_reps, Wg, Wu
    out = {"value": round(f2_bytes / med / 1e9, 2), "unit": "GB/s", "cores": threads,
           "kind": "port",
           "sample": (f"F2 B=1 Wg/Wu[14336,4096] fp16 via oracle/stages.py (torch CPU, "
                      f"{threads} threads), {calls} calls over 3 weight replicas in "
                      f"~{seconds:.0f} s, median {med * 1e6:.0f} us/call"),
           "us_per_call": round(med * 1e6, 1), "cpu_model": _cpu_model(),
           "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}

    rows = {}
    W = (torch.randn(4096, K, generator=gen) / 64).half()
    g = (torch.randn(K, generator=gen) * 0.1 + 1).half()
    f1_reps = [(x, g, W)] + [(x, g, W.clone()) for _ in range(7)]
    med, calls = _time_cpu(stages.f1, f1_reps, seconds / 3)
    nb = 4096 * K * 2 + K * 2 + (K + 4096) * 2
    rows["f1_cfg1"] = {"us_per_call": round(med * 1e6, 1), "GB/s": round(nb / med / 1e9, 2),
                       "calls": calls, "replicas": len(f1_reps)}
    del f1_reps, W
    L = 8192
    q = torch.randn(1, 32, 128, generator=gen).half()
    f4_reps = [(q, torch.randn(1, 8, L, 128, generator=gen).half(),
                torch.randn(1, 8, L, 128, generator=gen).half()) for _ in range(4)]
    med, calls = _time_cpu(lambda q_, k_, v_: stages.f4(q_, k_, v_), f4_reps, seconds / 3)
    nb = 2 * 8 * L * 128 * 2 + 2 * 32 * 128 * 2
    rows["f4_L8192"] = {"us_per_call": round(med * 1e6, 1), "GB/s": round(nb / med / 1e9, 2),
                        "calls": calls, "replicas": len(f4_reps)}
    out["rows"] = rows
    return out


# -------------------------------------------------------------------- main
def main(argv=None) -> int:
    args = parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the fused decode kernels run "
              "on a single MI355X; no multi-GPU path exists). Run with --gpus 1.",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch

    from decodebench_amd import ops
    from decodebench_amd.demos.llama_decode import build_config

    if args.profile_pass:
        return profile_pass(args.profile_pass, calls=args.calls, graph=args.graph,
                            isolated=args.isolated)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    ops.load_library()
    dev_name = torch.cuda.get_device_name(0)
    log(f"device {dev_name}, {ops.cu_count()} CUs")

    traffic = load_traffic(args.traffic)

    # ---- headline: F2, config 2, batch 1 --------------------------------
    head = build_config("f2", batch=1)
    err = check_case(head)
    log(f"f2 parity vs torch stages ok (rel-L2 {err:.2e}); {len(head.replicas)} replicas")
    secs = time_steps(head, args.steps, args.warmup)
    us = secs * 1e6 / args.steps
    gbs = head.algorithmic_bytes * args.steps / secs / 1e9
    log(f"f2 headline: {us:.2f} us/step, {gbs:.1f} GB/s")

    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded torch.Generator(42), fp32 -> fp16)",
        "config": {"workload": "F2 gate/up GEMV + SwiGLU fused, batch 1, x[1,4096], "
                               "Wg/Wu[14336,4096] fp16 (benchmark configs[1])",
                   "batch": 1, "K": 4096, "N": 14336,
                   "weight_replicas": len(head.replicas), "device": dev_name},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("f2_cfg2", {}).get("traffic_bytes"),
                     "traffic_source": (os.path.relpath(args.traffic, ROOT)
                                        if "f2_cfg2" in traffic else None),
                     "kernel": "gemv_kernel<2,...> (F2 SwiGLU mode)",
                     "algorithmic_bytes_per_launch": head.algorithmic_bytes,
                     "avg_launch_us": round(us, 3)},
    }
    del head
    torch.cuda.empty_cache()

    if not args.quick:
        # ---- per-kernel table (graph-replayed back-to-back launches) -----
        kernels = {}
        for name, kw in sweep_workloads():
            if args.sweep_only and not re.search(args.sweep_only, name):
                continue
            case = build_config(gen_device="cuda", **case_args(kw))
            with knobs(kw):
                if kw.get("check", True):
                    check_case(case)
                us_k, launches = time_graph_launches(case)
            kernels[name] = kernel_row(case, us_k)
            kernels[name]["launches_per_graph"] = launches
            kernels[name]["traffic_bytes"] = traffic.get(name, {}).get("traffic_bytes")
            log(f"{name}: {us_k:.2f} us, {kernels[name]['GB/s']:.0f} GB/s, "
                f"{kernels[name]['TFLOP/s']:.1f} TFLOP/s")
            del case
            torch.cuda.empty_cache()
        out["kernels"] = kernels
        parts = two_launch_parts(kernels)
        if parts:
            out["f4_two_launch_parts"] = parts
        out["roofline_by_kernel"] = roofline_by_kernel(
            kernels, traffic, load_kernel_trace(args.kernel_trace),
            load_kernel_trace(args.kernel_trace_isolated))

    if not args.quick and not args.sweep_only:
        # ---- Delta_launch vs B: unfused stream / graph vs fused ----------
        decomp = {}
        for name, kw in DECOMP_WORKLOADS:
            case = build_config(batch=1, gen_device="cuda", **kw)
            rep = case.seq.profile(case.inputs, trials=args.trials, target_ms=10.0,
                                   warmup=10, input_replicas=case.replicas,
                                   fused=case.fused)
            v = rep.verdict()
            # the fused call replayed back to back from a graph, as the unfused
            # chain's t_graph is: the residual against it holds no host time
            t_fused_graph, _ = time_graph_launches(case, replays=10)
            decomp[name] = {
                "t_stream_us": round(v.t_stream, 3), "t_graph_us": round(v.t_graph, 3),
                "t_fused_us": round(v.t_fused, 3), "delta_launch_us": round(v.delta_launch, 3),
                "delta_launch_ci": [round(c, 3) for c in v.delta_launch_ci],
                "B_us": round(v.b_bytes_est, 3), "residual_us": round(v.residual_us, 3),
                "t_fused_graph_us": round(t_fused_graph, 3),
                "residual_graph_us": round(v.t_graph - t_fused_graph - v.b_bytes_est, 3),
                "bound": v.bound, "dominant": v.dominant,
                "total_bytes": v.total_bytes, "eliminable_bytes": v.eliminable_bytes,
                "fused_extra_bytes": f4_partial_bytes(kw),
                "fused_check": fused_check(case),
                "samples_us": {k: [round(t, 3) for t in getattr(rep, f"{k}_us")]
                               for k in ("stream", "graph", "fused")}}
            log(f"{name}: stream {v.t_stream:.2f} graph {v.t_graph:.2f} fused "
                f"{v.t_fused:.2f} (graph {t_fused_graph:.2f}) us; dL {v.delta_launch:.2f} "
                f"B {v.b_bytes_est:.3f}")
            del case, rep
            torch.cuda.empty_cache()
        out["decomposition"] = decomp

        # ---- CPU baseline ------------------------------------------------
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        cb = out["cpu_baseline"]
        log(f"cpu baseline: F2 {cb['value']} GB/s on {cb['cores']} threads; "
            + "; ".join(f"{k} {v['us_per_call']} us" for k, v in cb["rows"].items()))
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
