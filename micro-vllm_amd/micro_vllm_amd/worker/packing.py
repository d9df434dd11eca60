"""Build one step's flattened model input and attention metadata on the GPU.

Replaces the reference ModelRunner's packing (model_runner.py:724-900:
``_build_model_input``, ``_flatten_model_input``, ``_build_slot_mapping``,
``_build_block_table``; attention.py:56-85 ``build_metadata``) and, when
capacities are given, the graph-padding copy (model_runner.py:78-122,
``_CudaGraphExecution.copy_input``).

The host side only concatenates what the plan already holds into one int32
payload (per-request counts, block ids, token ids) and sends it with one
host-to-device copy; positions, query starts, context lengths, context
starts, slot mapping, the null-padded block table and the sampling rows are
then produced by two HIP launches per cache group (``mvllm_pack_batch``).
No device value is read back.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from itertools import chain

import numpy as np
import torch

from micro_vllm_amd import _native
from micro_vllm_amd.attention.attention import AttentionMetadata
from micro_vllm_amd.attention.spec import AttentionSpec
from micro_vllm_amd.worker.scheduler_output import SchedulerOutput


@dataclass(frozen=True, slots=True, eq=False)
class PackedBatch:
    """Flattened tensors of one step (the reference's ``ModelInput``,
    model_runner.py:51-60) with one metadata object per cache group."""

    input_ids: torch.Tensor
    positions: torch.Tensor
    group_metadata: tuple[AttentionMetadata, ...]
    request_ids: tuple[str, ...]
    sampling_row_indices: torch.Tensor


class DeviceBlockRows:
    """A device-resident copy of every live request's block ids, updated by
    deltas (``mvllm_pack_batch_rows``).

    The reference's ModelRunner rebuilds each step's block table from the
    scheduler's full per-request lists, with one host-to-device copy per row
    (model_runner.py:871-900); the list-based ``pack_scheduler_output``
    still re-sends every id. Here each running request owns a row of
    ``rows`` ([num_slots, width] int32 on the device) for as long as it holds
    blocks, and a step sends only the ids that changed since the row was last
    written: blocks appended since, or entries replaced (the prefix cache's
    switch to a canonical block). The caller keeps that bookkeeping (it knows
    which ids changed) and passes ``(request_id, first, ids)`` updates."""

    def __init__(self, num_slots: int, width: int, device: torch.device | str) -> None:
        if num_slots <= 0 or width <= 0:
            raise ValueError("block rows need a positive slot count and width")
        self.num_slots = num_slots
        self.width = width
        self.rows = torch.full((num_slots, width), -1, dtype=torch.int32, device=torch.device(device))
        self._free = list(range(num_slots - 1, -1, -1))
        self._slot_of: dict[str, int] = {}

    def slot(self, request_id: str) -> int:
        """The request's row, assigned on first use."""

        slot = self._slot_of.get(request_id)
        if slot is None:
            if not self._free:
                raise RuntimeError(f"no free block row for request {request_id!r} ({self.num_slots} rows)")
            slot = self._free.pop()
            self._slot_of[request_id] = slot
        return slot

    def release(self, request_id: str) -> None:
        slot = self._slot_of.pop(request_id, None)
        if slot is not None:
            self._free.append(slot)


def pack_scheduler_output(
    plan: SchedulerOutput,
    *,
    specs: Sequence[AttentionSpec],
    block_size: int,
    null_block_id: int,
    device: torch.device | str,
    token_capacity: int | None = None,
    request_capacity: int | None = None,
    block_table_width: int | None = None,
    into: PackedBatch | None = None,
    block_rows: DeviceBlockRows | None = None,
    row_updates: Sequence[tuple[str, int, Sequence[int]]] = (),
) -> PackedBatch:
    """Pack ``plan`` for every cache group (``specs[g]`` is group g's spec).

    Without capacities the outputs have the reference's unpadded shapes
    (block table width = the longest block list of the group). With
    capacities they are padded the way a captured graph expects.

    ``into`` (from ``allocate_packed_batch``) makes the call write into
    existing tensors, whose shapes set the capacities: a captured graph keeps
    reading the same buffers while every step re-packs them. The returned
    batch then shares those tensors (its sampling rows are a prefix view of
    ``into.sampling_row_indices``).

    With ``block_rows`` (one cache group) the block ids come from the
    device-resident rows after ``row_updates`` are applied; only the length
    of each request's block list is read from the plan.
    """

    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError("GPU packing requires a GPU device")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    requests = plan.scheduled_requests
    num_groups = len(specs)
    num_requests = len(requests)
    for request in requests:
        if len(request.block_tables) < num_groups:
            raise ValueError(
                f"request {request.request_id!r} has {len(request.block_tables)} block tables "
                f"for {num_groups} cache groups"
            )
        if len(request.input_token_ids) != request.num_scheduled_tokens:
            raise ValueError(
                f"request {request.request_id!r} schedules {request.num_scheduled_tokens} "
                f"tokens but carries {len(request.input_token_ids)} input ids"
            )
    scheduled = np.fromiter((r.num_scheduled_tokens for r in requests), dtype=np.int64, count=num_requests)
    computed = np.fromiter((r.num_computed_tokens for r in requests), dtype=np.int64, count=num_requests)
    sampling = np.fromiter((r.requires_sampling for r in requests), dtype=np.int64, count=num_requests)
    num_tokens = int(scheduled.sum())
    num_sampling = int(sampling.sum())
    if into is not None:
        if len(into.group_metadata) != num_groups:
            raise ValueError(f"`into` holds {len(into.group_metadata)} cache groups, the plan needs {num_groups}")
        token_capacity = into.input_ids.numel()
        request_capacity = into.group_metadata[0].context_lengths.numel()
        block_table_width = into.group_metadata[0].block_table.shape[1]
        if into.sampling_row_indices.numel() < num_sampling:
            raise ValueError("`into` has too few sampling rows for the plan")
    token_capacity = num_tokens if token_capacity is None else token_capacity
    request_capacity = num_requests if request_capacity is None else request_capacity
    if token_capacity < num_tokens or request_capacity < num_requests:
        raise ValueError(
            f"capacities ({token_capacity} tokens, {request_capacity} requests) are below the "
            f"plan ({num_tokens}, {num_requests})"
        )
    if num_tokens + 1 > np.iinfo(np.int32).max:
        raise ValueError("too many tokens for the int32 payload")

    if block_rows is not None and num_groups != 1:
        raise ValueError("device-resident block rows serve one cache group")

    # Host payload: [token ids | per group: request info, block ids] and,
    # with block rows, [update records] at the end.
    segments = [
        np.fromiter(chain.from_iterable(r.input_token_ids for r in requests), dtype=np.int32, count=num_tokens)
    ]
    group_layout = []
    widths = []
    offset = num_tokens
    update_records = None
    for g in range(num_groups):
        lengths = np.fromiter((len(r.block_tables[g].block_ids) for r in requests), dtype=np.int64, count=num_requests)
        info = np.zeros((num_requests, _native.PACK_FIELDS), dtype=np.int32)
        info[:, 0] = computed
        info[:, 1] = scheduled
        info[:, 2] = lengths
        info[:, 3] = sampling
        if block_rows is None:
            total_blocks = int(lengths.sum())
            ids = np.fromiter(
                chain.from_iterable(r.block_tables[g].block_ids for r in requests), dtype=np.int32, count=total_blocks
            )
        else:
            if num_requests and int(lengths.max()) > block_rows.width:
                raise ValueError(f"a block list is longer than the block rows' width {block_rows.width}")
            info[:, 6] = np.fromiter((block_rows.slot(r.request_id) for r in requests), dtype=np.int32,
                                     count=num_requests)
            counts = [len(u[2]) for u in row_updates]
            total_blocks = sum(counts)
            ids = np.fromiter(chain.from_iterable(u[2] for u in row_updates), dtype=np.int32, count=total_blocks)
            update_records = np.zeros((len(row_updates), 4), dtype=np.int32)
            ids_offset = 0
            for i, ((request_id, first, _), n) in enumerate(zip(row_updates, counts)):
                if first < 0 or first + n > block_rows.width:
                    raise ValueError(f"row update of {request_id!r} exceeds the block rows' width")
                update_records[i] = (block_rows.slot(request_id), first, n, ids_offset)
                ids_offset += n
        max_len = int(lengths.max()) if num_requests else 0
        width = max_len if block_table_width is None else block_table_width
        if width < max_len:
            raise ValueError(f"block_table_width {width} is below the longest block list ({max_len})")
        widths.append(width)
        group_layout.append((offset, offset + info.size, total_blocks))
        segments.extend((info.reshape(-1), ids))
        offset += info.size + total_blocks
    updates_offset = offset
    if update_records is not None:
        segments.append(update_records.reshape(-1))
    host = torch.from_numpy(np.concatenate(segments) if segments else np.zeros(0, np.int32))
    if host.numel() == 0:
        host = torch.zeros(1, dtype=torch.int32)
    payload = host.pin_memory().to(device, non_blocking=True)

    if into is None:
        into = allocate_packed_batch(
            num_groups=num_groups,
            block_size=block_size,
            token_capacity=token_capacity,
            request_capacity=request_capacity,
            block_table_widths=widths,
            sampling_capacity=num_sampling,
            device=device,
            max_query_len=int(scheduled.max()) if num_requests else 0,
        )
    else:
        if any(m.block_table.shape[1] != w for m, w in zip(into.group_metadata, widths)):
            raise ValueError("`into` block tables do not have the plan's width")
        hint = into.group_metadata[0].max_query_len
        if hint is not None and num_requests and int(scheduled.max()) > hint:
            raise ValueError(f"`into` is for steps of at most {hint} query tokens per request")
    lib = _native.load()
    stream = _native.stream_handle(device)
    base = payload.data_ptr()
    for g, spec in enumerate(specs):
        info_offset, ids_offset, total_blocks = group_layout[g]
        args = _pack_args(
            into, g, spec, base, info_offset=info_offset, ids_offset=ids_offset, total_blocks=total_blocks,
            num_requests=num_requests, num_tokens=num_tokens, num_sampling=num_sampling, block_size=block_size,
            null_block_id=null_block_id, token_capacity=token_capacity, request_capacity=request_capacity,
            width=widths[g],
        )
        if block_rows is None:
            _native.check(lib.mvllm_pack_batch(args, stream), "mvllm_pack_batch")
        else:
            rows = _rows_args(block_rows, base, updates_offset, len(row_updates))
            _native.check(lib.mvllm_pack_batch_rows(args, rows, stream), "mvllm_pack_batch_rows")
    # `payload` was allocated on the current stream, so the caching allocator
    # reuses its memory only for work ordered after these launches.
    return PackedBatch(
        input_ids=into.input_ids,
        positions=into.positions,
        group_metadata=into.group_metadata,
        request_ids=tuple(r.request_id for r in requests),
        sampling_row_indices=into.sampling_row_indices[:num_sampling],
    )


def allocate_packed_batch(
    *,
    num_groups: int,
    block_size: int,
    token_capacity: int,
    request_capacity: int,
    block_table_widths: Sequence[int],
    sampling_capacity: int,
    device: torch.device | str,
    max_query_len: int | None = None,
) -> PackedBatch:
    """Uninitialised device tensors of a packed step at fixed capacities."""

    i64 = dict(dtype=torch.int64, device=torch.device(device))
    positions = torch.empty(token_capacity, **i64)
    query_start_locations = torch.empty(request_capacity + 1, **i64)
    context_lengths = torch.empty(request_capacity, **i64)
    metadata = tuple(
        AttentionMetadata(
            query_positions=positions,
            query_context_start_positions=torch.empty(token_capacity, **i64),
            query_start_locations=query_start_locations,
            context_lengths=context_lengths,
            block_table=torch.empty((request_capacity, block_table_widths[g]), **i64),
            slot_mapping=torch.empty(token_capacity, **i64),
            block_size=block_size,
            max_query_len=max_query_len,
        )
        for g in range(num_groups)
    )
    return PackedBatch(
        input_ids=torch.empty(token_capacity, **i64),
        positions=positions,
        group_metadata=metadata,
        request_ids=(),
        sampling_row_indices=torch.empty(sampling_capacity, **i64),
    )


def _pack_args(into: PackedBatch, g: int, spec: AttentionSpec, base: int, *, info_offset: int, ids_offset: int,
               total_blocks: int, num_requests: int, num_tokens: int, num_sampling: int, block_size: int,
               null_block_id: int, token_capacity: int, request_capacity: int, width: int) -> "_native.PackArgs":
    """The C arguments of one cache group's pack launch: payload sections
    at the given int32 offsets from ``base``, outputs into ``into``."""

    group = into.group_metadata[g]
    kind, parameter = spec.kernel_code()
    first = g == 0
    args = _native.PackArgs()
    args.request_info = base + 4 * info_offset if num_requests else None
    args.block_ids = base + 4 * ids_offset if total_blocks else None
    args.token_ids = base if num_tokens else None
    args.num_requests = num_requests
    args.num_tokens = num_tokens
    args.num_block_ids = total_blocks
    args.block_size = block_size
    args.null_block_id = null_block_id
    args.spec_kind = kind
    args.spec_parameter = parameter
    args.token_capacity = token_capacity
    args.request_capacity = request_capacity
    args.block_table_width = width
    args.input_ids = into.input_ids.data_ptr() if first and token_capacity else None
    args.positions = into.positions.data_ptr() if first and token_capacity else None
    args.context_starts = group.query_context_start_positions.data_ptr() if token_capacity else None
    args.query_start_locations = group.query_start_locations.data_ptr() if first else None
    args.context_lengths = group.context_lengths.data_ptr() if first and request_capacity else None
    args.block_table = group.block_table.data_ptr() if group.block_table.numel() else None
    args.slot_mapping = group.slot_mapping.data_ptr() if token_capacity else None
    args.sampling_rows = into.sampling_row_indices.data_ptr() if first and num_sampling else None
    return args


def _rows_args(block_rows: DeviceBlockRows, base: int, updates_offset: int, num_updates: int) -> "_native.BlockRows":
    rows = _native.BlockRows()
    rows.rows = block_rows.rows.data_ptr()
    rows.num_slots = block_rows.num_slots
    rows.width = block_rows.width
    rows.updates = base + 4 * updates_offset if num_updates else None
    rows.num_updates = num_updates
    return rows


def pack_decode_rows(
    token_ids: np.ndarray,
    computed: np.ndarray,
    block_lengths: np.ndarray,
    slots: np.ndarray,
    row_updates: Sequence[tuple[int, int, Sequence[int]]],
    *,
    spec: AttentionSpec,
    block_size: int,
    null_block_id: int,
    block_rows: DeviceBlockRows,
    into: PackedBatch,
    staging: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> PackedBatch:
    """Pack a decode-only step (every request: one token, sampled) from
    per-request arrays, without a ``SchedulerOutput``: the same launch and
    outputs as ``pack_scheduler_output(plan, into=into, block_rows=...,
    row_updates=...)`` for the plan whose request r has input token
    ``token_ids[r]``, ``computed[r]`` computed tokens and
    ``block_lengths[r]`` block ids in block row ``slots[r]``.
    ``row_updates`` lists ``(slot, first, ids)``: the ids that changed in a
    row since it was last written. ``staging`` (pinned host int32, device
    int32) carries the payload without allocating when it fits; the caller
    guarantees that the previous copy out of it and the previous pack
    launch reading it have completed."""

    device = into.input_ids.device
    n = int(len(token_ids))
    token_capacity = into.input_ids.numel()
    request_capacity = into.group_metadata[0].context_lengths.numel()
    width = into.group_metadata[0].block_table.shape[1]
    if n > token_capacity or n > request_capacity or into.sampling_row_indices.numel() < n:
        raise ValueError(f"a decode step of {n} requests exceeds the buffers' capacities")
    if n and int(block_lengths.max()) > min(width, block_rows.width):
        raise ValueError("a block list is longer than the block table")
    counts = [len(u[2]) for u in row_updates]
    total_blocks = sum(counts)
    info = np.zeros((n, _native.PACK_FIELDS), dtype=np.int32)
    info[:, 0] = computed
    info[:, 1] = 1
    info[:, 2] = block_lengths
    info[:, 3] = 1
    info[:, 6] = slots
    records = np.zeros((len(row_updates), 4), dtype=np.int32)
    ids_offset = 0
    for i, ((slot, first, _), k) in enumerate(zip(row_updates, counts)):
        if first < 0 or first + k > block_rows.width:
            raise ValueError(f"row update of slot {slot} exceeds the block rows' width")
        records[i] = (slot, first, k, ids_offset)
        ids_offset += k
    ids = np.fromiter(chain.from_iterable(u[2] for u in row_updates), dtype=np.int32, count=total_blocks)
    info_offset = n
    ids_at = n + info.size
    updates_offset = ids_at + total_blocks
    words = updates_offset + records.size
    if staging is not None and 0 < words <= staging[0].numel() <= staging[1].numel():
        hbuf, dbuf = staging
        hv = hbuf.numpy()
        hv[:n] = token_ids
        hv[info_offset:ids_at] = info.reshape(-1)
        hv[ids_at:updates_offset] = ids
        hv[updates_offset:words] = records.reshape(-1)
        dbuf[:words].copy_(hbuf[:words], non_blocking=True)
        payload = dbuf
    else:
        host = torch.from_numpy(np.concatenate((np.asarray(token_ids, np.int32), info.reshape(-1), ids, records.reshape(-1))))
        if host.numel() == 0:
            host = torch.zeros(1, dtype=torch.int32)
        payload = host.pin_memory().to(device, non_blocking=True)
    base = payload.data_ptr()
    args = _pack_args(
        into, 0, spec, base, info_offset=info_offset, ids_offset=ids_at, total_blocks=total_blocks, num_requests=n,
        num_tokens=n, num_sampling=n, block_size=block_size, null_block_id=null_block_id,
        token_capacity=token_capacity, request_capacity=request_capacity, width=width,
    )
    rows = _rows_args(block_rows, base, updates_offset, len(row_updates))
    lib = _native.load()
    _native.check(lib.mvllm_pack_batch_rows(args, rows, _native.stream_handle(device)), "mvllm_pack_batch_rows")
    return PackedBatch(
        input_ids=into.input_ids,
        positions=into.positions,
        group_metadata=into.group_metadata,
        request_ids=(),
        sampling_row_indices=into.sampling_row_indices[:n],
    )
