"""Immutable attention visibility semantics (the reference's spec.py:13-51).

Each spec also names the code the GPU kernels use for it (``kernel_code``:
kind and parameter), so per-query starts are computed on the device.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass

from micro_vllm_amd import _native


@dataclass(frozen=True, slots=True)
class AttentionSpec(ABC):
    """Define the first key visible to one absolute query position."""

    @abstractmethod
    def context_start(self, query_position: int) -> int:
        """Return the inclusive start of the query's visible key interval."""

    @abstractmethod
    def kernel_code(self) -> tuple[int, int]:
        """(kind, parameter) understood by ``mvllm_context_starts``."""


@dataclass(frozen=True, slots=True)
class FullAttentionSpec(AttentionSpec):
    """Retain the complete causal history."""

    def context_start(self, query_position: int) -> int:
        return 0

    def kernel_code(self) -> tuple[int, int]:
        return (_native.SPEC_FULL, 0)


@dataclass(frozen=True, slots=True)
class SlidingWindowSpec(AttentionSpec):
    """Retain at most ``window_size`` keys, including the query token."""

    window_size: int

    def __post_init__(self) -> None:
        if type(self.window_size) is not int or self.window_size <= 0:
            raise ValueError("window_size must be a positive integer")

    def context_start(self, query_position: int) -> int:
        return max(0, query_position - self.window_size + 1)

    def kernel_code(self) -> tuple[int, int]:
        return (_native.SPEC_SLIDING_WINDOW, self.window_size)


@dataclass(frozen=True, slots=True)
class ChunkedLocalSpec(AttentionSpec):
    """Retain the causal prefix within one aligned local chunk."""

    chunk_size: int

    def __post_init__(self) -> None:
        if type(self.chunk_size) is not int or self.chunk_size <= 0:
            raise ValueError("chunk_size must be a positive integer")

    def context_start(self, query_position: int) -> int:
        return (query_position // self.chunk_size) * self.chunk_size

    def kernel_code(self) -> tuple[int, int]:
        return (_native.SPEC_CHUNKED_LOCAL, self.chunk_size)
