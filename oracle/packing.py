"""CPU oracle for the ragged-batch packing step (TEST INFRASTRUCTURE ONLY).

Restates how the reference ModelRunner turns one scheduler step into the
flattened tensors and per-cache-group ``AttentionMetadata`` that the
attention operator consumes, in plain Python/numpy:

* ``flatten_model_input``  src/micro_vllm/worker/model_runner.py:751-831
* ``build_slot_mapping``   src/micro_vllm/worker/model_runner.py:833-869
* ``build_block_table``    src/micro_vllm/worker/model_runner.py:871-900
* ``graph_pad``            src/micro_vllm/worker/model_runner.py:78-122
                           (``_CudaGraphExecution.copy_input``: fixed-capacity
                           padding with qsl tail = num_tokens, zero context
                           lengths/starts/positions/ids, null block ids and
                           slot -1)
* context starts           src/micro_vllm/attention/attention.py:68-75 with
                           src/micro_vllm/attention/spec.py:13-51

Only tests and the cpu baseline may use this module. It is pinned by the
literal vectors of the reference's worker tests (tests/golden/packing.json).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .paged_attention import context_starts, map_cache_slots


@dataclass(frozen=True)
class Request:
    """The fields of ``ScheduledRequest`` (scheduler_output.py:18-33) used here."""

    request_id: str
    input_token_ids: tuple[int, ...]
    num_computed_tokens: int
    num_scheduled_tokens: int
    requires_sampling: bool
    block_tables: tuple[tuple[int, ...], ...]


def flatten_model_input(requests: list[Request]) -> dict[str, np.ndarray]:
    """input_ids, positions, query_start_locations, context_lengths,
    sampling_row_indices of one step."""

    input_ids: list[int] = []
    positions: list[int] = []
    starts = [0]
    lengths: list[int] = []
    sampling_rows: list[int] = []
    for request in requests:
        input_ids.extend(request.input_token_ids)
        begin = request.num_computed_tokens
        positions.extend(range(begin, begin + request.num_scheduled_tokens))
        starts.append(len(input_ids))
        lengths.append(begin + request.num_scheduled_tokens)
        if request.requires_sampling:
            sampling_rows.append(len(input_ids) - 1)
    return {
        "input_ids": np.array(input_ids, dtype=np.int64),
        "positions": np.array(positions, dtype=np.int64),
        "query_start_locations": np.array(starts, dtype=np.int64),
        "context_lengths": np.array(lengths, dtype=np.int64),
        "sampling_row_indices": np.array(sampling_rows, dtype=np.int64),
    }


def build_slot_mapping(requests: list[Request], group: int, block_size: int) -> np.ndarray:
    """Each scheduled position mapped through its request's block ids."""

    pieces = []
    for request in requests:
        begin = request.num_computed_tokens
        positions = np.arange(begin, begin + request.num_scheduled_tokens, dtype=np.int64)
        table = np.array(request.block_tables[group], dtype=np.int64)
        pieces.append(map_cache_slots(positions, table, block_size))
    if not pieces:
        return np.zeros(0, dtype=np.int64)
    return np.concatenate(pieces)


def build_block_table(requests: list[Request], group: int, null_block_id: int) -> np.ndarray:
    """Rectangular table, rows padded on the right with the null block id."""

    width = max((len(r.block_tables[group]) for r in requests), default=0)
    table = np.full((len(requests), width), null_block_id, dtype=np.int64)
    for row, request in enumerate(requests):
        ids = request.block_tables[group]
        table[row, : len(ids)] = ids
    return table


def pack(
    requests: list[Request],
    *,
    group: int,
    block_size: int,
    null_block_id: int,
    spec: tuple[int, int],
) -> dict[str, np.ndarray]:
    """Everything one cache group's metadata needs, unpadded."""

    flat = flatten_model_input(requests)
    flat["context_starts"] = context_starts(spec[0], spec[1], flat["positions"])
    flat["slot_mapping"] = build_slot_mapping(requests, group, block_size)
    flat["block_table"] = build_block_table(requests, group, null_block_id)
    return flat


def graph_pad(
    packed: dict[str, np.ndarray],
    *,
    token_capacity: int,
    request_capacity: int,
    block_table_width: int,
    null_block_id: int,
) -> dict[str, np.ndarray]:
    """Copy a step into fixed-capacity buffers the way a captured graph sees it."""

    num_tokens = packed["positions"].size
    num_requests = packed["context_lengths"].size
    out = {}
    ids = np.zeros(token_capacity, dtype=np.int64)
    ids[:num_tokens] = packed["input_ids"]
    out["input_ids"] = ids
    positions = np.zeros(token_capacity, dtype=np.int64)
    positions[:num_tokens] = packed["positions"]
    out["positions"] = positions
    starts = np.full(request_capacity + 1, num_tokens, dtype=np.int64)
    starts[: num_requests + 1] = packed["query_start_locations"]
    out["query_start_locations"] = starts
    lengths = np.zeros(request_capacity, dtype=np.int64)
    lengths[:num_requests] = packed["context_lengths"]
    out["context_lengths"] = lengths
    cstarts = np.zeros(token_capacity, dtype=np.int64)
    cstarts[:num_tokens] = packed["context_starts"]
    out["context_starts"] = cstarts
    table = np.full((request_capacity, block_table_width), null_block_id, dtype=np.int64)
    src = packed["block_table"]
    table[: src.shape[0], : src.shape[1]] = src
    out["block_table"] = table
    slots = np.full(token_capacity, -1, dtype=np.int64)
    slots[:num_tokens] = packed["slot_mapping"]
    out["slot_mapping"] = slots
    out["sampling_row_indices"] = packed["sampling_row_indices"].copy()
    return out
