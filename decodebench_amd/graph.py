"""Graph capture and replay with an explicit success/failure result.

On ROCm ``torch.cuda.CUDAGraph`` records a hipGraph; replay launches the whole
recorded chain with one submission, which is what ``delta_launch`` measures
against plain stream launches.

Behaviour follows ``src/decodebench/graph.py:9-88`` of the reference: the body
is warmed up on a side stream, captured into a graph (optionally in a shared
memory pool), and a capture failure is returned as ``Captured(ok=False)``
rather than raised.  After a failed capture torch can leave its device RNG
generator registered with the aborted graph; a trivial capture that succeeds
clears that state, and any error in that clean-up is reported in ``reason``.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import Callable


@dataclass
class Captured:
    ok: bool
    reason: str = ""
    _graph: object = None

    def replay(self) -> None:
        if not self.ok:
            raise RuntimeError(f"cannot replay: capture failed ({self.reason})")
        self._graph.replay()


def try_capture(body: Callable[[], None], warmup_iters: int = 3,
                pool=None) -> Captured:
    """Warm ``body`` up on a side stream, then capture it into a graph.

    ``pool`` is an optional ``torch.cuda.graph_pool_handle()`` shared by graphs
    that always replay one after another in capture order.
    """
    import torch

    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        for _ in range(warmup_iters):
            body()
    torch.cuda.current_stream().wait_stream(warm)

    graph = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(graph, pool=pool):
            body()
    except Exception as exc:  # capture failures come in many types
        reason = f"{type(exc).__name__}: {exc}"
        problem = _clear_generator_registration()
        if problem:
            reason += (f" [additionally, RNG-registration cleanup failed: "
                       f"{problem}; torch.randn on this device may raise until "
                       "the process restarts]")
        return Captured(ok=False, reason=reason)
    return Captured(ok=True, _graph=graph)


def _clear_generator_registration() -> str:
    """Run one trivial, successful capture; return "" or the error text."""
    import torch

    try:
        if torch.cuda.is_current_stream_capturing():
            return "current stream is still in capture mode; skipped cleanup"
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        scratch = torch.zeros(1, device="cuda")   # allocated before capture
        g = torch.cuda.CUDAGraph()
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            with torch.cuda.stream(side):
                g.capture_begin()
                scratch.fill_(0.0)
                g.capture_end()
        torch.cuda.current_stream().wait_stream(side)
        del g, scratch
        return ""
    except Exception as exc:  # never mask the original capture failure
        return f"{type(exc).__name__}: {exc}"
