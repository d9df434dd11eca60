"""CPU oracle for micro-vLLM's ragged paged attention (TEST INFRASTRUCTURE ONLY).

This module restates, in numpy, what the reference's
``ReferenceAttentionOperator`` computes. The HIP library's results are
compared with it: only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and never as the thing
that is measured or shipped.

Followed reference code (paths relative to the reference checkout):

* ``map_cache_slots``      src/micro_vllm/attention/attention.py:31-41
* ``context_start``        src/micro_vllm/attention/spec.py:13-51
* ``write_kv_cache``       src/micro_vllm/attention/operators/reference.py:84-98
* ``gather_kv_cache``      src/micro_vllm/attention/operators/reference.py:101-138
* ``reference_forward``    src/micro_vllm/attention/operators/reference.py:14-81
* ``dense_attention``      tests/attention/operators/test_reference.py:325-360
                           (the dense causal closed form, here in float64)

Pinning (each function is checked in ``tests/test_oracle.py`` against the
reference tests' literal vectors and against closed forms; see the list in
that module's docstring). One deliberate difference: a request whose query
range is empty is skipped. The reference would index
``query_context_start_positions[query_start]`` with ``query_start ==
num_tokens`` and raise; such requests only occur in graph-padded batches,
which the reference operator never receives (config.py:45-57).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .numerics import from_f32, storage_kind, to_f32

FULL = 0
SLIDING_WINDOW = 1
CHUNKED_LOCAL = 2


@dataclass(frozen=True)
class Batch:
    """The fields of ``AttentionMetadata`` (attention.py:12-28), as numpy int64."""

    query_positions: np.ndarray
    query_context_start_positions: np.ndarray
    query_start_locations: np.ndarray
    context_lengths: np.ndarray
    block_table: np.ndarray
    slot_mapping: np.ndarray
    block_size: int

    @property
    def num_requests(self) -> int:
        return int(self.context_lengths.size)


def context_start(kind: int, parameter: int, position: int) -> int:
    """First visible key of a query (spec.py:13-51)."""

    if kind == FULL:
        return 0
    if kind == SLIDING_WINDOW:
        return max(0, position - parameter + 1)
    if kind == CHUNKED_LOCAL:
        return (position // parameter) * parameter
    raise ValueError(f"unknown spec kind {kind}")


def context_starts(kind: int, parameter: int, positions: np.ndarray) -> np.ndarray:
    """``Attention.build_metadata``'s per-query loop (attention.py:68-75)."""

    return np.array(
        [context_start(kind, parameter, int(p)) for p in positions],
        dtype=np.int64,
    )


def map_cache_slots(
    positions: np.ndarray, block_table_row: np.ndarray, block_size: int
) -> np.ndarray:
    """slot = table[pos // block_size] * block_size + pos % block_size."""

    positions = np.asarray(positions, dtype=np.int64)
    logical = positions // block_size
    offsets = positions % block_size
    physical = np.asarray(block_table_row, dtype=np.int64)[logical]
    return physical * block_size + offsets


def _flat_planes(cache: np.ndarray) -> np.ndarray:
    """View (2, blocks, block_size, heads, dim) as (2, slots, heads, dim)."""

    return cache.reshape(2, -1, *cache.shape[3:])


def write_kv_cache(
    key: np.ndarray, value: np.ndarray, cache: np.ndarray, slot_mapping: np.ndarray
) -> None:
    """Copy each token's K/V rows into its physical slot, in place.

    The reference uses ``index_copy_`` with every slot valid; the Triton
    kernel additionally skips negative (padding) slots
    (triton_paged.py:38-39, 62-68). Both behaviours hold here: a negative slot
    writes nothing.
    """

    flat = _flat_planes(cache)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    for token, slot in enumerate(slots):
        if slot < 0:
            continue
        flat[0, slot] = key[token]
        flat[1, slot] = value[token]


def request_key_range(batch: Batch, request: int) -> tuple[int, int, int]:
    """(query_start, first gathered position, context length) of a request."""

    query_start = int(batch.query_start_locations[request])
    first = int(batch.query_context_start_positions[query_start])
    return query_start, first, int(batch.context_lengths[request])


def gather_kv_cache(cache: np.ndarray, batch: Batch) -> list[tuple[np.ndarray, np.ndarray]]:
    """Each request's visible K/V rows ``[start(first query), context_len)``."""

    flat = _flat_planes(cache)
    histories = []
    for request in range(batch.num_requests):
        query_start = int(batch.query_start_locations[request])
        query_end = int(batch.query_start_locations[request + 1])
        if query_end <= query_start:
            histories.append(None)
            continue
        _, first, length = request_key_range(batch, request)
        positions = np.arange(first, length, dtype=np.int64)
        slots = map_cache_slots(positions, batch.block_table[request], batch.block_size)
        histories.append((flat[0, slots], flat[1, slots]))
    return histories


def reference_forward(
    query: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    cache: np.ndarray,
    batch: Batch,
    *,
    zero_uncovered: bool = True,
) -> np.ndarray:
    """Write K/V, then causal GQA attention per request in float32.

    Mirrors the reference's per-request loop: gather, repeat K/V heads for
    the query-head group, fp32 scores, mask ``key < start(q)`` or ``key >
    pos(q)``, fp32 softmax of ``scores * head_dim**-0.5``, fp32 P·V, narrow to
    the query's type. Tokens outside every request come back zero (the
    Triton operator's ``zeros_like`` output, triton_paged.py:343) when
    ``zero_uncovered``.
    """

    kind = storage_kind(query)
    num_q_heads = query.shape[1]
    num_kv_heads = key.shape[1]
    group = num_q_heads // num_kv_heads
    scale = np.float32(1.0 / math.sqrt(query.shape[-1]))
    write_kv_cache(key, value, cache, batch.slot_mapping)
    histories = gather_kv_cache(cache, batch)
    output = np.zeros(query.shape, dtype=np.float32)
    query32 = to_f32(query)
    for request, history in enumerate(histories):
        if history is None:
            continue
        query_start = int(batch.query_start_locations[request])
        query_end = int(batch.query_start_locations[request + 1])
        cached_key, cached_value = history
        k32 = np.repeat(to_f32(cached_key), group, axis=1)
        v32 = np.repeat(to_f32(cached_value), group, axis=1)
        q32 = query32[query_start:query_end]
        scores = np.einsum("qhd,khd->hqk", q32, k32, dtype=np.float32)
        first = int(batch.query_context_start_positions[query_start])
        key_positions = np.arange(first, first + k32.shape[0], dtype=np.int64)
        query_positions = batch.query_positions[query_start:query_end]
        query_starts = batch.query_context_start_positions[query_start:query_end]
        masked = (key_positions[None, :] < query_starts[:, None]) | (
            key_positions[None, :] > query_positions[:, None]
        )
        scores = np.where(masked[None], np.float32(-np.inf), scores * scale)
        with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
            peak = scores.max(axis=-1, keepdims=True)
            weights = np.exp(scores - peak)
            weights = weights / weights.sum(axis=-1, keepdims=True)
        attention = np.einsum("hqk,khd->qhd", weights.astype(np.float32), v32, dtype=np.float32)
        output[query_start:query_end] = attention
    if not zero_uncovered:
        raise NotImplementedError("the oracle always zero-fills uncovered tokens")
    return from_f32(output, kind)


def dense_attention(
    query: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    *,
    query_positions: np.ndarray | None = None,
    query_context_starts: np.ndarray | None = None,
    key_positions: np.ndarray | None = None,
) -> np.ndarray:
    """float64 causal attention over contiguous K/V (the dense closed form).

    ``key[i]``/``value[i]`` sit at ``key_positions[i]`` (default ``i``).
    Returns float64 ``[queries, q_heads, dim]``.
    """

    q = to_f32(query).astype(np.float64) if query.dtype != np.float64 else query
    k = to_f32(key).astype(np.float64) if key.dtype != np.float64 else key
    v = to_f32(value).astype(np.float64) if value.dtype != np.float64 else value
    group = q.shape[1] // k.shape[1]
    k = np.repeat(k, group, axis=1)
    v = np.repeat(v, group, axis=1)
    if query_positions is None:
        query_positions = np.arange(q.shape[0], dtype=np.int64)
    if query_context_starts is None:
        query_context_starts = np.zeros_like(query_positions)
    if key_positions is None:
        key_positions = np.arange(k.shape[0], dtype=np.int64)
    scores = np.einsum("qhd,khd->hqk", q, k) / math.sqrt(q.shape[-1])
    masked = (key_positions[None, :] < query_context_starts[:, None]) | (
        key_positions[None, :] > query_positions[:, None]
    )
    scores = np.where(masked[None], -np.inf, scores)
    with np.errstate(invalid="ignore"):
        peak = scores.max(axis=-1, keepdims=True)
        weights = np.exp(scores - peak)
        weights = weights / weights.sum(axis=-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", weights, v)


def make_batch(
    query_positions: list[list[int]],
    block_tables: list[list[int]],
    *,
    block_size: int,
    null_block_id: int,
    spec: tuple[int, int] = (FULL, 0),
    context_lengths: list[int] | None = None,
) -> Batch:
    """Build a Batch the way the reference tests' ``make_attention_metadata``
    does (test_reference.py:363-424): flattened positions, prefix-sum query
    starts, context length = last position + 1, null-padded block table,
    slots by ``map_cache_slots``."""

    flat_positions = [p for positions in query_positions for p in positions]
    starts = [0]
    for positions in query_positions:
        starts.append(starts[-1] + len(positions))
    width = max((len(t) for t in block_tables), default=0)
    table = np.full((len(block_tables), width), null_block_id, dtype=np.int64)
    for row, ids in enumerate(block_tables):
        table[row, : len(ids)] = ids
    slots = [
        int(map_cache_slots(np.array([p]), table[row], block_size)[0])
        for row, positions in enumerate(query_positions)
        for p in positions
    ]
    if context_lengths is None:
        context_lengths = [positions[-1] + 1 for positions in query_positions]
    positions_array = np.array(flat_positions, dtype=np.int64)
    return Batch(
        query_positions=positions_array,
        query_context_start_positions=context_starts(spec[0], spec[1], positions_array),
        query_start_locations=np.array(starts, dtype=np.int64),
        context_lengths=np.array(context_lengths, dtype=np.int64),
        block_table=table,
        slot_mapping=np.array(slots, dtype=np.int64),
        block_size=block_size,
    )
