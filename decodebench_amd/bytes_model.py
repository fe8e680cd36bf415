"""Analytic byte accounting for an unfused decode chain.

A chain is described as a list of :class:`StageTrace` records, one per
unfused stage, holding the bytes that stage reads and the bytes it writes.
Fusing the chain into one kernel removes, for every non-final stage, its own
write plus one read of that write per downstream consumer.

Behaviour follows ``src/decodebench/bytes_model.py:20-70`` of the reference
(same field names, same validation rules, same two totals), so byte counts and
verdicts computed here agree with the reference's for identical traces.

Only declared stage boundaries are visible: casts or scratch buffers that a
stage allocates internally are not counted, which is why ``Sequence.trace``
warns when a stage allocates more than its declared output.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class StageTrace:
    """One unfused stage: bytes read, bytes written, and fan-out.

    ``reads``      byte count of every tensor argument the stage reads.
    ``write``      byte count of the stage's single output.
    ``is_final``   the chain's final output (never eliminable).
    ``consumers``  number of later stage arguments bound to this output; a
                   fused kernel saves the write plus one read per consumer.
    """

    name: str
    reads: list[int] = field(default_factory=list)
    write: int = 0
    is_final: bool = False
    consumers: int = 1

    def __post_init__(self) -> None:
        if self.write < 0 or min(self.reads, default=0) < 0:
            raise ValueError("StageTrace byte counts must be non-negative")
        if self.consumers < 0:
            raise ValueError("StageTrace consumers must be non-negative")
        if self.consumers == 0 and not self.is_final:
            raise ValueError(
                "non-final StageTrace must have at least one consumer")


def total_bytes(traces: list[StageTrace]) -> int:
    """All bytes the unfused chain moves: every read plus every write."""
    total = 0
    for t in traces:
        total += t.write
        total += sum(t.reads)
    return total


def eliminable_bytes(traces: list[StageTrace]) -> int:
    """Bytes a fully fused chain no longer moves.

    Each non-final stage contributes its write and one equally sized read for
    each consumer, i.e. ``(1 + consumers) * write``.
    """
    return sum(t.write * (t.consumers + 1) for t in traces if not t.is_final)
