"""Attention metadata, slot math and the semantic wrapper.

Mirrors the reference's src/micro_vllm/attention/attention.py:12-102 with the
same names and argument meaning. ``Attention.build_metadata`` computes the
per-query visibility starts on the GPU (``mvllm_context_starts``) instead
of the reference's ``.tolist()`` + Python loop (attention.py:68-75).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from micro_vllm_amd import _native
from micro_vllm_amd.attention.spec import AttentionSpec


@dataclass(frozen=True, slots=True, eq=False)
class AttentionMetadata:
    """Flattened queries, visibility bounds, and paged-cache inputs."""

    query_positions: torch.Tensor
    query_context_start_positions: torch.Tensor
    query_start_locations: torch.Tensor
    context_lengths: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    block_size: int
    # Optional host-side hint (not in the reference's metadata): the largest
    # number of queries of any request. Packing knows it without a device
    # read; 1 lets a decode-only batch skip the prefill launch (a request
    # with more queries then gets NaN rows).
    max_query_len: int | None = None

    @property
    def num_requests(self) -> int:
        """Number of requests represented by this batch."""

        return self.context_lengths.numel()


def map_cache_slots(
    positions: torch.Tensor,
    block_table: torch.Tensor,
    block_size: int,
) -> torch.Tensor:
    """Map logical token positions to flattened physical cache slots."""

    logical_blocks = positions // block_size
    block_offsets = positions % block_size
    physical_blocks = block_table.index_select(0, logical_blocks)
    return physical_blocks * block_size + block_offsets


def context_starts(positions: torch.Tensor, spec: AttentionSpec) -> torch.Tensor:
    """Per-query visibility start of ``spec``, computed by a HIP kernel."""

    if positions.device.type != "cuda":
        raise RuntimeError("context starts are computed on the GPU; got a CPU tensor")
    if positions.dtype != torch.int64:
        raise ValueError("query positions must be int64")
    positions = positions.contiguous()
    out = torch.empty_like(positions)
    kind, parameter = spec.kernel_code()
    lib = _native.load()
    _native.check(
        lib.mvllm_context_starts(
            positions.data_ptr() if positions.numel() else None,
            positions.numel(),
            kind,
            parameter,
            out.data_ptr() if out.numel() else None,
            _native.stream_handle(positions.device),
        ),
        "mvllm_context_starts",
    )
    return out


class Attention:
    """Own an operator and the metadata semantics it consumes."""

    def __init__(self, spec: AttentionSpec, operator_name: str) -> None:
        from micro_vllm_amd.attention.operators.registry import (
            get_attention_operator_class,
        )

        self.spec = spec
        operator_class = get_attention_operator_class(operator_name)
        self.operator = operator_class()

    def build_metadata(
        self,
        *,
        query_positions: torch.Tensor,
        query_start_locations: torch.Tensor,
        context_lengths: torch.Tensor,
        block_table: torch.Tensor,
        slot_mapping: torch.Tensor,
        block_size: int,
    ) -> AttentionMetadata:
        """Build per-query visibility metadata for this attention semantic."""

        return AttentionMetadata(
            query_positions=query_positions,
            query_context_start_positions=context_starts(query_positions, self.spec),
            query_start_locations=query_start_locations,
            context_lengths=context_lengths,
            block_table=block_table,
            slot_mapping=slot_mapping,
            block_size=block_size,
        )

    def __call__(
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        layer_kv_cache: torch.Tensor,
        metadata: AttentionMetadata,
        /,
    ) -> torch.Tensor:
        return self.operator(
            query,
            key,
            value,
            layer_kv_cache,
            metadata,
        )
