"""Sequence: a decode chain of stages, traced for bytes and profiled for time.

A stage is a plain function whose parameters are bound by name: a parameter
named after an earlier stage receives that stage's output, otherwise a key of
the inputs dict, otherwise (first parameter of a later stage only) the
previous stage's output.  ``trace`` runs the chain once and records each
stage's read and write bytes; ``profile`` times the chain as eager stream
launches, as graph replay, and optionally a fused replacement, in rotated
rounds on rotating input replicas.

The public behaviour -- registration rules, binding precedence, static DAG
validation with consumer counts, the tensor checks in a traced run, the
``profile`` keyword arguments, the fused-output check and the replica checks
-- follows ``src/decodebench/sequence.py:20-365`` of the reference, including
the exception types and the message fragments callers match on.

The fused variant is where this package's HIP kernels plug in: the callables
in ``decodebench_amd.ops`` take tensors, allocate their output with torch and
launch on torch's current stream, so they can be used as stages and inside a
``fused=`` lambda, and they are safe to capture into a graph.
"""

from __future__ import annotations

import functools
import inspect
import itertools
import warnings
from dataclasses import dataclass
from typing import Any, Callable

from decodebench_amd.bytes_model import StageTrace
from decodebench_amd.verdict import DEFAULT_BYTE_THRESHOLD

# A stage that grows allocated device memory by more than this beyond its
# declared output triggers a warning (the byte model cannot see it).
_HIDDEN_ALLOC_WARN_MB = 0.1

# Fused-output agreement: an element fails only if it misses both bounds.
_FUSED_ABS_TOL = 5e-2
_FUSED_REL_TOL = 2e-2

_PLAIN_KINDS = (inspect.Parameter.POSITIONAL_ONLY,
                inspect.Parameter.POSITIONAL_OR_KEYWORD)


@dataclass
class _Stage:
    fn: Callable[..., Any]
    name: str
    params: list[str]


# Sources a parameter can bind to, in precedence order.
_FROM_STAGE, _FROM_INPUT, _FROM_PREVIOUS = "stage", "input", "previous"


class Sequence:
    def __init__(self, name: str):
        self.name = name
        self._stages: list[_Stage] = []

    # ------------------------------------------------------------------ build
    def stage(self, fn):
        """Decorator: append ``fn`` as the next stage of the chain."""
        sig = inspect.signature(fn)
        for p in sig.parameters.values():
            if p.kind not in _PLAIN_KINDS:
                raise TypeError(
                    f"stage '{fn.__name__}': parameter '{p.name}' is "
                    f"{p.kind.description}; stages must use plain positional "
                    "parameters (no *args/**kwargs/keyword-only parameters -- "
                    "DecodeBench binds by name and position explicitly)")
        if fn.__name__ in {s.name for s in self._stages}:
            raise ValueError(f"duplicate stage name '{fn.__name__}'")
        self._stages.append(_Stage(fn, fn.__name__, list(sig.parameters)))
        return fn

    # ---------------------------------------------------------------- binding
    @staticmethod
    def _source(param: str, position: int, stage_index: int,
                earlier: Any, inputs) -> str | None:
        if param in earlier:
            return _FROM_STAGE
        if param in inputs:
            return _FROM_INPUT
        if stage_index > 0 and position == 0:
            return _FROM_PREVIOUS
        return None

    def _bind_args(self, stage, idx, prev_out, inputs, stage_outputs):
        """Arguments for ``stage`` (index ``idx``) in parameter order."""
        args = []
        for j, p in enumerate(stage.params):
            src = self._source(p, j, idx, stage_outputs, inputs)
            if src == _FROM_STAGE:
                args.append(stage_outputs[p])
            elif src == _FROM_INPUT:
                args.append(inputs[p])
            elif src == _FROM_PREVIOUS:
                args.append(prev_out)
            else:
                raise KeyError(
                    f"stage '{stage.name}' parameter '{p}' not found in earlier "
                    f"stage outputs {list(stage_outputs)} or inputs {list(inputs)}")
        return args

    def _dependency_consumer_counts(self, inputs) -> dict[str, int]:
        """Check every binding statically and count reads of each output.

        Runs before any stage executes, so a malformed chain fails without
        touching the device.  Every non-final stage output must be read by
        some later stage: the eliminable-byte model assumes it.
        """
        seen: list[str] = []
        counts: dict[str, int] = {}
        for idx, st in enumerate(self._stages):
            for j, p in enumerate(st.params):
                src = self._source(p, j, idx, seen, inputs)
                if src == _FROM_STAGE:
                    counts[p] = counts.get(p, 0) + 1
                elif src == _FROM_PREVIOUS:
                    counts[seen[-1]] = counts.get(seen[-1], 0) + 1
                elif src is None:
                    raise KeyError(
                        f"stage '{st.name}' parameter '{p}' not found in earlier "
                        f"stage outputs {seen} or inputs {list(inputs)}")
            seen.append(st.name)
        dead = [n for n in seen[:-1] if counts.get(n, 0) == 0]
        if dead:
            raise ValueError(
                f"non-final stage output(s) {dead} are never consumed by a "
                "later stage; the eliminable-byte model assumes every non-final "
                "write has a downstream read, so this chain is not a valid "
                "DecodeBench model")
        return counts

    # ------------------------------------------------------------ traced run
    @staticmethod
    def _storage_data_ptr(tensor) -> int:
        getter = getattr(tensor, "untyped_storage", None)
        if getter is not None:
            return getter().data_ptr()
        return tensor.storage().data_ptr()

    @staticmethod
    def _closure_tensors(fn, torch_module) -> list[str]:
        """Tensors a stage reaches through its closure or globals."""
        cv = inspect.getclosurevars(fn)
        hidden = [f"nonlocal:{k}" for k, v in cv.nonlocals.items()
                  if isinstance(v, torch_module.Tensor)]
        hidden += [f"global:{k}" for k, v in cv.globals.items()
                   if isinstance(v, torch_module.Tensor)]
        return hidden

    def _check_stage_io(self, st, args, out, torch) -> None:
        if not isinstance(out, torch.Tensor):
            raise TypeError(
                f"stage '{st.name}' must return a single torch.Tensor "
                f"(got {type(out).__name__}). DecodeBench v1 supports "
                "linear, single-output chains only.")
        if not out.is_contiguous():
            raise ValueError(
                f"stage '{st.name}' returned a non-contiguous tensor "
                f"(shape={tuple(out.shape)}, stride={out.stride()}); materialize "
                "it explicitly before using DecodeBench byte accounting")
        if out.nbytes > 0:
            base = self._storage_data_ptr(out)
            aliased = [j for j, a in enumerate(args)
                       if isinstance(a, torch.Tensor) and a.nbytes > 0
                       and self._storage_data_ptr(a) == base]
            if aliased:
                raise ValueError(
                    f"stage '{st.name}' output aliases tensor argument(s) "
                    f"{aliased}; in-place/view outputs do not represent a "
                    "materialized stage write")

    def _run_once(self, inputs, _check_temporaries=False):
        import torch

        if not self._stages:
            raise ValueError(
                "Sequence has no stages; register at least one with @seq.stage")
        counts = self._dependency_consumer_counts(inputs)
        watch_alloc = _check_temporaries and torch.cuda.is_available()
        prev = None
        outputs: dict[str, Any] = {}
        io = []
        for idx, st in enumerate(self._stages):
            args = self._bind_args(st, idx, prev, inputs, outputs)
            hidden = self._closure_tensors(st.fn, torch)
            if hidden:
                raise ValueError(
                    f"stage '{st.name}' captures tensor(s) {hidden} outside its "
                    "declared parameters; pass them through inputs so byte "
                    "accounting can see them")
            for j, a in enumerate(args):
                if isinstance(a, torch.Tensor) and not a.is_contiguous():
                    raise ValueError(
                        f"stage '{st.name}' tensor argument {j} is non-contiguous "
                        f"(shape={tuple(a.shape)}, stride={a.stride()}); "
                        "materialize it explicitly as a declared stage")
            before = (torch.cuda.memory_stats()["allocated_bytes.all.allocated"]
                      if watch_alloc else None)
            out = st.fn(*args)
            self._check_stage_io(st, args, out, torch)
            if before is not None:
                after = torch.cuda.memory_stats()["allocated_bytes.all.allocated"]
                extra_mb = (after - before - out.nbytes) / (1024 * 1024)
                if extra_mb > _HIDDEN_ALLOC_WARN_MB:
                    warnings.warn(
                        f"stage '{st.name}' allocated {extra_mb:.1f} MB internally; "
                        "byte model undercounts -- split it into single-op stages",
                        stacklevel=2)
            io.append((st.name,
                       [a for a in args if isinstance(a, torch.Tensor)], out))
            outputs[st.name] = out
            prev = out
        return prev, io, counts

    def trace(self, inputs) -> list[StageTrace]:
        """Run the chain once and return one :class:`StageTrace` per stage."""
        _, io, counts = self._run_once(inputs, _check_temporaries=True)
        last = len(io) - 1
        return [StageTrace(name, [t.nbytes for t in reads], out.nbytes,
                           i == last, 0 if i == last else counts[name])
                for i, (name, reads, out) in enumerate(io)]

    # --------------------------------------------------------------- profile
    def profile(self, inputs, trials: int = 30, target_ms: float = 20.0,
                warmup: int = 50,
                byte_threshold: float = DEFAULT_BYTE_THRESHOLD,
                seed: int = 42, input_replicas: list[dict] | None = None,
                fused: Callable[[dict], Any] | None = None):
        """Time the chain as stream launches and graph replay (and ``fused``).

        ``input_replicas``: dicts with identical structure; invocation ``i``
        uses replica ``i % N`` so a weight is not re-read from cache.
        ``fused``: a callable taking the inputs dict and returning the chain's
        final output; it is checked against the unfused chain (an element
        fails only if abs error >= 5e-2 and rel error >= 2e-2) before any
        timing, then timed on the same replicas.
        """
        import torch

        from decodebench_amd.report import Report
        from decodebench_amd.timing import time_callable

        torch.manual_seed(seed)
        replicas = list(input_replicas) if input_replicas else [inputs]
        self._validate_replicas(replicas)
        traces = self.trace(replicas[0])
        if fused is not None:
            self._check_fused_output(fused, replicas[0], torch)

        calls = {"stream": _cycled(replicas, self._replay_body)}
        graphs, reason = self._capture_replicas(replicas, torch)
        if graphs is None:
            # No graph: the report carries the stream times for both.
            stream_us = time_callable(calls["stream"], trials=trials,
                                      target_ms=target_ms, warmup=warmup)
            return Report(self.name, stream_us, stream_us, traces,
                          byte_threshold=byte_threshold, graph_ok=False,
                          graph_skip_reason=reason)
        calls["graph"] = _cycled(graphs, _replay)
        if fused is not None:
            calls["fused"] = _cycled(replicas, fused)

        times: dict[str, list[float]] = {name: [] for name in calls}
        for name, n, warm in _rotation_plan(list(calls), trials, warmup):
            times[name] += time_callable(calls[name], trials=n,
                                         target_ms=target_ms, warmup=warm)
        return Report(self.name, times["stream"], times["graph"], traces,
                      fused_us=times.get("fused"),
                      byte_threshold=byte_threshold)

    def _capture_replicas(self, replicas, torch):
        """One graph of the chain per replica, or ``(None, reason)``.

        All graphs record into one private memory pool: they are only ever
        replayed one after another, so their intermediates can share it.
        Capture stops at the first replica that fails.
        """
        from decodebench_amd.graph import try_capture

        make_pool = getattr(torch.cuda, "graph_pool_handle", None)
        pool = make_pool() if make_pool is not None else None
        graphs = []
        for rep in replicas:
            g = try_capture(functools.partial(self._replay_body, rep), pool=pool)
            if not g.ok:
                return None, g.reason
            graphs.append(g)
        return graphs, None

    def _check_fused_output(self, fused, inputs, torch) -> None:
        """Fused and unfused outputs must agree elementwise (abs OR rel)."""
        ref = self._replay_body(inputs)
        out = fused(inputs)
        if not isinstance(out, torch.Tensor):
            raise ValueError(
                "fused callable must return a single torch.Tensor "
                f"(got {type(out).__name__})")
        if out.shape != ref.shape:
            raise ValueError(
                f"fused output shape {tuple(out.shape)} != unfused chain "
                f"output shape {tuple(ref.shape)}")
        err = (out.float() - ref.float()).abs()
        rel = err / ref.float().abs().clamp_min(1e-12)
        if not bool(((err < _FUSED_ABS_TOL) | (rel < _FUSED_REL_TOL)).all()):
            raise ValueError(
                "fused output does not match the unfused chain: "
                f"max_abs={err.max().item():.3e}, max_rel={rel.max().item():.3e} "
                "(pass requires abs < 5e-2 or rel < 2e-2 elementwise)")

    def _replay_body(self, inp):
        """The chain on ``inp`` with no checks: the timed stream body."""
        outputs: dict[str, Any] = {}
        last = None
        for idx, st in enumerate(self._stages):
            last = outputs[st.name] = st.fn(
                *self._bind_args(st, idx, last, inp, outputs))
        return last

    @staticmethod
    def _validate_replicas(replicas: list[dict]) -> None:
        """Every replica has replica 0's keys and tensor metadata."""
        import torch

        def meta(v):
            if not isinstance(v, torch.Tensor):
                return (False,)
            return (True, tuple(v.shape), v.dtype, v.stride(), v.device)

        first = replicas[0]
        want = {key: meta(v) for key, v in first.items()}
        for i, rep in enumerate(replicas[1:], start=1):
            if rep.keys() != first.keys():
                raise ValueError(
                    f"input replica {i} keys {sorted(rep)} != replica 0 keys "
                    f"{sorted(first)}")
            for key, expected in want.items():
                v = rep[key]
                got = meta(v)
                if got == expected:
                    continue
                if got[0] != expected[0]:
                    raise ValueError(
                        f"replica {i}['{key}'] tensor-ness differs from replica 0")
                raise ValueError(
                    f"replica {i}['{key}'] (shape={tuple(v.shape)}, "
                    f"dtype={v.dtype}, stride={v.stride()}, device={v.device}) "
                    "does not match replica 0")


def _cycled(items, call):
    """A no-argument callable: the i-th invocation runs ``call(items[i % n])``."""
    it = itertools.cycle(items)
    return lambda: call(next(it))


def _replay(graph):
    graph.replay()


def _rotation_plan(names: list[str], trials: int,
                   warmup: int) -> list[tuple[str, int, int]]:
    """The timing passes of ``profile``: ``(variant, trials, warmup)`` in order.

    The trials of each variant are spread over up to three rounds (the first
    ``trials % rounds`` rounds take one more).  Round ``r`` starts at variant
    ``r mod len(names)`` and goes round the list, so slow drift in clocks or
    temperature reaches every variant instead of biasing the one timed last.
    The first round warms each variant up ``warmup`` calls, later rounds at
    most 5.  This is the reference's measurement procedure
    (src/decodebench/sequence.py:276-291).
    """
    rounds = min(3, trials)
    if rounds <= 0:
        return []
    base, extra = divmod(trials, rounds)
    plan = []
    for r in range(rounds):
        n = base + (1 if r < extra else 0)
        warm = warmup if r == 0 else min(warmup, 5)
        plan += [(names[(r + j) % len(names)], n, warm) for j in range(len(names))]
    return plan
