"""Event timing with warm-up, a probe batch and an adaptive repeat count.

``time_callable`` and ``n_weight_replicas`` keep the behaviour of
``src/decodebench/timing.py:8-65`` of the reference: arguments are validated
before torch is imported, a 5-invocation probe sets the repeat count
``K = max(200, ceil(target_ms / t_probe))`` (capped at one million), and each
trial reports microseconds per invocation between two events on the current
stream.  On ROCm ``torch.cuda.Event`` is a hipEvent.

MI355X note: the replica formula of the reference only sizes against the L2
that torch reports (one XCD's 4 MB).  The 256 MB Infinity Cache (MALL) sits
behind all eight XCD L2s, so rotating eight replicas of a 33 MB weight still
hits the MALL.  ``cache_defeat_replicas`` sizes a rotation that exceeds
twice the whole on-die cache hierarchy; the measurement driver uses it, while
``n_weight_replicas`` keeps the reference's formula for drop-in callers.
"""

from __future__ import annotations

import math
import os
from typing import Callable

# Whole-chip cache capacity in front of HBM on MI355X: 8 XCDs x 4 MB L2 plus
# the 256 MB Infinity Cache.  Overridable for other parts or experiments.
MI355X_CACHE_BYTES = 8 * 4 * 1024 * 1024 + 256 * 1024 * 1024


def n_weight_replicas(weight_bytes: int, l2_bytes: int | None = None) -> int:
    """Replica count ``min(8, max(4, ceil(2 * L2 / weight_bytes)))``."""
    if weight_bytes <= 0:
        raise ValueError("weight_bytes must be positive")
    if l2_bytes is None:
        import torch

        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        l2_bytes = (getattr(props, "L2_cache_size", None)
                    or getattr(props, "l2_cache_size", None))
    if l2_bytes is None or l2_bytes < 0:
        raise ValueError("l2_bytes must be non-negative")
    return min(8, max(4, -(-2 * l2_bytes // weight_bytes)))


def cache_bytes() -> int:
    """On-die cache bytes a rotation must defeat (env DECODEBENCH_CACHE_BYTES)."""
    env = os.environ.get("DECODEBENCH_CACHE_BYTES")
    return int(env) if env else MI355X_CACHE_BYTES


def cache_defeat_replicas(working_bytes: int, cache: int | None = None,
                          minimum: int = 2, maximum: int = 256) -> int:
    """Copies of a working set whose rotation spans at least 2x the caches."""
    if working_bytes <= 0:
        raise ValueError("working_bytes must be positive")
    cache = cache_bytes() if cache is None else cache
    if cache < 0:
        raise ValueError("cache bytes must be non-negative")
    need = -(-2 * cache // working_bytes)
    return int(min(maximum, max(minimum, need)))


def _check_timing_args(trials: int, target_ms: float, warmup: int) -> None:
    if trials <= 0:
        raise ValueError("trials must be positive")
    if not (math.isfinite(target_ms) and target_ms > 0):
        raise ValueError("target_ms must be finite and positive")
    if warmup < 0:
        raise ValueError("warmup must be non-negative")


def time_callable(fn: Callable[[], object], trials: int = 30,
                  target_ms: float = 20.0, warmup: int = 50) -> list[float]:
    """Microseconds per invocation of ``fn`` for each of ``trials`` trials."""
    _check_timing_args(trials, target_ms, warmup)
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()

    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    probe = 5
    t0.record()
    for _ in range(probe):
        fn()
    t1.record()
    torch.cuda.synchronize()
    per_call_ms = max(t0.elapsed_time(t1) / probe, 1e-4)
    reps = min(1_000_000, max(200, math.ceil(target_ms / per_call_ms)))

    samples: list[float] = []
    for _ in range(trials):
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        samples.append(t0.elapsed_time(t1) * 1000.0 / reps)
    return samples
