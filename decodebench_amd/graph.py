"""Record a body of GPU work once as a hipGraph, then replay it.

On ROCm ``torch.cuda.CUDAGraph`` is a hipGraph: a replay submits the whole
recorded chain at once, which is what ``Sequence.profile`` sets against
stream launches of the same stages (Δ_launch).

Interface kept from the reference (src/decodebench/graph.py:9-21):
``try_capture(body, warmup_iters=3, pool=None)`` returns a ``Captured`` and
never raises for a body that cannot be captured; ``Captured.ok`` says
whether it could, ``reason`` why not, and ``replay()`` of a failed capture
raises ``RuntimeError("cannot replay: capture failed (...)")``.

How it records:

* Every device has one recording stream, made on first use and kept.  The
  warm-up calls and the capture both run on it, so the blocks the caching
  allocator hands out while warming up already belong to the stream the
  graph records on, and the caller's stream is never put in capture mode.
  The recording stream waits for the caller's stream before the warm-up
  (pending writes of the inputs), and the caller's stream waits for it
  afterwards.
* The capture is opened and closed explicitly, so a body that raises while
  recording still has its capture closed, and the body's error and the
  closing error are reported together.
* A capture that fails after it began leaves torch's device random
  generators marked as capturing (their capture epilogue never ran), after
  which ``torch.randn`` on that device raises.  ``_reset_generators``
  records an empty graph on the recording stream: its opening and closing
  run the generators' prologue and epilogue and leave them idle.  If that
  fails as well, its error is appended to ``reason``.
"""

from __future__ import annotations

import threading
import warnings
from dataclasses import dataclass
from typing import Callable, Optional

_recording_streams: dict = {}
_recording_lock = threading.Lock()


@dataclass
class Captured:
    """Outcome of :func:`try_capture`: a replayable graph, or why there is none."""

    ok: bool
    reason: str = ""
    _graph: object = None

    def replay(self) -> None:
        if not self.ok:
            raise RuntimeError(f"cannot replay: capture failed ({self.reason})")
        self._graph.replay()


def try_capture(body: Callable[[], None], warmup_iters: int = 3, pool=None) -> Captured:
    """Run ``body`` ``warmup_iters`` times, then record one call of it.

    ``pool`` is an optional ``torch.cuda.graph_pool_handle()`` for graphs that
    always replay one after another in capture order and may share memory.
    Errors of the warm-up calls propagate: they are errors of the body, not
    of capturing it."""
    import torch

    caller = torch.cuda.current_stream()
    rec = _recording_stream(caller.device)
    rec.wait_stream(caller)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(rec):
        for _ in range(warmup_iters):
            body()
        rec.synchronize()
        failure = _record(graph, body, pool)
    caller.wait_stream(rec)
    if failure is None:
        return Captured(ok=True, _graph=graph)
    del graph
    leftover = _reset_generators(rec)
    if leftover:
        failure += (f"; resetting the device random generators afterwards failed too "
                    f"({leftover}), so random ops on this device may raise until the "
                    f"process restarts")
    return Captured(ok=False, reason=failure)


def _recording_stream(device):
    import torch

    key = device.index if device.index is not None else torch.cuda.current_device()
    with _recording_lock:
        stream = _recording_streams.get(key)
        if stream is None:
            stream = torch.cuda.Stream(device=key)
            _recording_streams[key] = stream
    return stream


def _describe(exc: BaseException) -> str:
    return f"{type(exc).__name__}: {exc}"


def _record(graph, body: Callable[[], None], pool) -> Optional[str]:
    """Capture one call of ``body`` into ``graph`` on the current stream.

    Returns None on success, else the error text.  Once the capture has been
    opened it is always closed, whatever the body does."""
    try:
        graph.capture_begin(pool=pool)
    except Exception as exc:  # the capture never started
        return _describe(exc)
    body_error = None
    try:
        body()
    except Exception as exc:  # anything the body raises ends the recording
        body_error = exc
    try:
        graph.capture_end()
    except Exception as exc:
        if body_error is None:
            return _describe(exc)
        return f"{_describe(body_error)} (closing the capture: {_describe(exc)})"
    return None if body_error is None else _describe(body_error)


def _reset_generators(stream) -> str:
    """Record an empty graph on ``stream`` so that torch runs the capture
    epilogue of its device generators; "" on success, else the error."""
    import torch

    empty = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.stream(stream), warnings.catch_warnings():
            # torch warns that a graph without nodes was captured; that is the point
            warnings.simplefilter("ignore")
            empty.capture_begin()
            empty.capture_end()
    except Exception as exc:
        return _describe(exc)
    finally:
        del empty
    return ""
