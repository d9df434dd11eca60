"""The scheduler's plan contract consumed by packing.

Same fields and names as the reference's
src/micro_vllm/core/scheduler_output.py:8-53 (sampling parameters omitted:
packing only needs to know whether a request samples).
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True, slots=True)
class CacheGroupBlockTable:
    """One cache group's immutable logical-to-physical block snapshot."""

    block_ids: tuple[int, ...]

    def __post_init__(self) -> None:
        object.__setattr__(self, "block_ids", tuple(self.block_ids))


@dataclass(frozen=True, slots=True)
class ScheduledRequest:
    """Immutable request snapshot with tables in cache-topology order."""

    request_id: str
    input_token_ids: tuple[int, ...]
    num_computed_tokens: int
    num_scheduled_tokens: int
    requires_sampling: bool
    block_tables: tuple[CacheGroupBlockTable, ...]

    def __post_init__(self) -> None:
        object.__setattr__(self, "input_token_ids", tuple(self.input_token_ids))
        object.__setattr__(self, "block_tables", tuple(self.block_tables))


@dataclass(frozen=True, slots=True)
class SchedulerOutput:
    """Immutable execution plan produced for one scheduler step."""

    scheduled_requests: tuple[ScheduledRequest, ...]
    preempted_request_ids: tuple[str, ...] = ()

    def __post_init__(self) -> None:
        object.__setattr__(self, "scheduled_requests", tuple(self.scheduled_requests))
        object.__setattr__(self, "preempted_request_ids", tuple(self.preempted_request_ids))
