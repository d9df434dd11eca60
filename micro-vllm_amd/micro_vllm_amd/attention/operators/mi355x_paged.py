"""The gfx950 paged-attention operator (registered as ``"mi355x_paged"``).

Drop-in for the reference's attention operators
(src/micro_vllm/attention/operators/reference.py:11-81,
triton_paged.py:392-418): same positional signature, same in-place cache
write, a new output tensor like ``query``. All work runs in the HIP library
through its C ABI on the current torch stream; nothing here synchronises
with the host, so a forward can be captured in a HIP graph.

Error conventions follow the reference: tensors off the GPU raise
``RuntimeError``; an unsupported dtype raises ``ValueError``.
"""

from __future__ import annotations

import math

import torch

from micro_vllm_amd import _native
from micro_vllm_amd.attention.attention import AttentionMetadata
from micro_vllm_amd.attention.operators.base import AttentionOperator

SUPPORTED_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _index(t: torch.Tensor, name: str, device: torch.device) -> torch.Tensor:
    if t.dtype != torch.int64:
        raise ValueError(f"metadata.{name} must be int64, got {t.dtype}")
    if t.device != device:
        raise RuntimeError(f"metadata.{name} is on {t.device}, expected {device}")
    return t if t.dim() != 1 or t.is_contiguous() else t.contiguous()


def batch_descriptor(metadata: AttentionMetadata, device: torch.device) -> tuple[_native.Batch, list]:
    """C-ABI view of ``metadata``; the list keeps any made-contiguous copies alive."""

    keep = []
    positions = _index(metadata.query_positions, "query_positions", device)
    starts = _index(metadata.query_context_start_positions, "query_context_start_positions", device)
    qsl = _index(metadata.query_start_locations, "query_start_locations", device)
    lengths = _index(metadata.context_lengths, "context_lengths", device)
    slots = _index(metadata.slot_mapping, "slot_mapping", device)
    table = _index(metadata.block_table, "block_table", device)
    if table.dim() != 2:
        raise ValueError(f"metadata.block_table must be 2-D, got shape {tuple(table.shape)}")
    num_requests = lengths.numel()
    if qsl.numel() != num_requests + 1:
        raise ValueError(
            f"query_start_locations has {qsl.numel()} entries for {num_requests} requests"
        )
    if table.shape[0] < num_requests:
        raise ValueError(f"block_table has {table.shape[0]} rows for {num_requests} requests")
    num_tokens = positions.numel()
    if starts.numel() != num_tokens or slots.numel() != num_tokens:
        raise ValueError("query positions, context starts and slot_mapping differ in length")
    keep.extend((positions, starts, qsl, lengths, slots, table))
    b = _native.Batch()
    b.query_positions = positions.data_ptr() if num_tokens else None
    b.query_context_start_positions = starts.data_ptr() if num_tokens else None
    b.query_start_locations = qsl.data_ptr()
    b.context_lengths = lengths.data_ptr() if num_requests else None
    b.block_table = table.data_ptr() if table.numel() else None
    b.slot_mapping = slots.data_ptr() if num_tokens else None
    b.num_tokens = num_tokens
    b.num_requests = num_requests
    b.block_table_width = table.shape[1]
    b.block_table_stride[0] = table.stride(0)
    b.block_table_stride[1] = table.stride(1)
    b.block_size = metadata.block_size
    hint = getattr(metadata, "max_query_len", None)
    b.max_query_len = hint if hint is not None else -1
    return b, keep


def _check_inputs(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    layer_kv_cache: torch.Tensor,
    metadata: AttentionMetadata,
) -> None:
    if query.device.type != "cuda":
        raise RuntimeError("mi355x_paged attention requires GPU tensors")
    if query.dtype not in SUPPORTED_DTYPES:
        raise ValueError(
            "mi355x_paged attention supports torch.bfloat16, torch.float16 and torch.float32, "
            f"got {query.dtype}"
        )
    for name, t in (("key", key), ("value", value), ("layer_kv_cache", layer_kv_cache)):
        if t.device != query.device:
            raise RuntimeError(f"{name} is on {t.device}, query on {query.device}")
        if t.dtype != query.dtype:
            raise ValueError(f"{name} dtype {t.dtype} differs from query dtype {query.dtype}")
    if layer_kv_cache.dim() != 5 or layer_kv_cache.shape[2] != metadata.block_size:
        raise ValueError(
            f"layer_kv_cache shape {tuple(layer_kv_cache.shape)} does not match block_size "
            f"{metadata.block_size}"
        )
    if key.shape[0] != query.shape[0] or value.shape != key.shape:
        raise ValueError("query, key and value must have the same number of tokens")
    if query.shape[1] % key.shape[1] != 0:
        raise ValueError("query heads must be a multiple of key/value heads")


def hip_write_kv_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    layer_kv_cache: torch.Tensor,
    metadata: AttentionMetadata,
) -> None:
    """Scatter K/V into their cache slots (bit-exact; slot -1 writes nothing)."""

    device = layer_kv_cache.device
    if device.type != "cuda":
        raise RuntimeError("mi355x_paged cache writes require GPU tensors")
    slots = _index(metadata.slot_mapping, "slot_mapping", device)
    if slots.numel() != key.shape[0]:
        raise ValueError("slot_mapping length differs from the number of key rows")
    lib = _native.load()
    _native.check(
        lib.mvllm_kv_write(
            _native.tensor3(key),
            _native.tensor3(value),
            _native.kv_cache(layer_kv_cache),
            slots.data_ptr() if slots.numel() else None,
            key.shape[0],
            _native.stream_handle(device),
        ),
        "mvllm_kv_write",
    )


def hip_paged_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    layer_kv_cache: torch.Tensor,
    metadata: AttentionMetadata,
    *,
    timing: _native.Timing | None = None,
) -> torch.Tensor:
    """Write current K/V, then ragged causal attention through the block table.

    ``timing`` (measurement only) carries hipEvent_t handles recorded around
    the decode and prefill kernel launches.
    """

    _check_inputs(query, key, value, layer_kv_cache, metadata)
    device = query.device
    batch, keep = batch_descriptor(metadata, device)
    output = torch.empty_like(query)
    lib = _native.load()
    workspace_bytes = lib.mvllm_attention_workspace_bytes(batch, query.shape[1], query.shape[2])
    workspace = torch.empty(max(workspace_bytes, 1), dtype=torch.uint8, device=device)
    args = (
        _native.tensor3(query),
        _native.tensor3(key),
        _native.tensor3(value),
        _native.kv_cache(layer_kv_cache),
        batch,
        _native.tensor3(output),
        1.0 / math.sqrt(query.shape[-1]),
        workspace.data_ptr(),
        workspace.numel(),
    )
    stream = _native.stream_handle(device)
    if timing is None:
        status = lib.mvllm_attention_forward(*args, stream)
    else:
        status = lib.mvllm_attention_forward_timed(*args, timing, stream)
    _native.check(status, "mvllm_attention_forward")
    del keep
    return output


class AttentionPlan:
    """Work lists of one batch, built once and shared by every layer of a step.

    The reference's operator runs per layer (qwen.py:89-99); the lists depend
    only on the batch, so a model whose layers share one metadata bundle and
    one cache geometry plans once per step (``mvllm_attention_plan``) and
    each layer's ``hip_attention_over_cache(..., plan=plan)`` skips the
    list kernels. The plan owns the workspace, which every planned call on
    the same stream reuses for its split-KV partials.
    """

    def __init__(self, metadata: AttentionMetadata, num_q_heads: int, layer_kv_cache: torch.Tensor):
        device = layer_kv_cache.device
        if device.type != "cuda":
            raise RuntimeError("mi355x_paged attention plans require a GPU cache")
        self.metadata = metadata
        self.num_q_heads = num_q_heads
        self.batch, self._keep = batch_descriptor(metadata, device)
        lib = _native.load()
        head_dim = layer_kv_cache.shape[-1]
        nbytes = lib.mvllm_attention_workspace_bytes(self.batch, num_q_heads, head_dim)
        self.workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _native.check(
            lib.mvllm_attention_plan(
                self.batch,
                num_q_heads,
                _native.kv_cache(layer_kv_cache),
                self.workspace.data_ptr(),
                self.workspace.numel(),
                _native.stream_handle(device),
            ),
            "mvllm_attention_plan",
        )


def hip_attention_over_cache(
    query: torch.Tensor,
    layer_kv_cache: torch.Tensor,
    metadata: AttentionMetadata,
    plan: AttentionPlan | None = None,
) -> torch.Tensor:
    """Ragged causal attention over a cache that already holds the step's
    K/V (written by ``layers.qk_norm_rope_kv_write``): the attention part of
    ``hip_paged_attention``, without the cache write. With ``plan`` (made for
    this metadata and head count) the work lists are not rebuilt."""

    if query.device.type != "cuda" or layer_kv_cache.device != query.device:
        raise RuntimeError("mi355x_paged attention requires GPU tensors on one device")
    if query.dtype not in SUPPORTED_DTYPES or layer_kv_cache.dtype != query.dtype:
        raise ValueError(f"unsupported or mismatched dtypes {query.dtype} / {layer_kv_cache.dtype}")
    device = query.device
    output = torch.empty_like(query)
    lib = _native.load()
    if plan is not None:
        if plan.metadata is not metadata or plan.num_q_heads != query.shape[1]:
            raise ValueError("attention plan was made for other metadata or another head count")
        batch, keep, workspace, entry = plan.batch, None, plan.workspace, "mvllm_paged_attention_planned"
    else:
        batch, keep = batch_descriptor(metadata, device)
        workspace_bytes = lib.mvllm_attention_workspace_bytes(batch, query.shape[1], query.shape[2])
        workspace = torch.empty(max(workspace_bytes, 1), dtype=torch.uint8, device=device)
        entry = "mvllm_paged_attention"
    _native.check(
        getattr(lib, entry)(
            _native.tensor3(query),
            _native.kv_cache(layer_kv_cache),
            batch,
            _native.tensor3(output),
            1.0 / math.sqrt(query.shape[-1]),
            workspace.data_ptr(),
            workspace.numel(),
            _native.stream_handle(device),
        ),
        entry,
    )
    del keep
    return output


def hip_gather_kv_cache(
    layer_kv_cache: torch.Tensor,
    metadata: AttentionMetadata,
    capacity: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Padded ``[requests, capacity, heads, dim]`` K and V histories (bit-exact).

    Row ``i`` of request ``r`` holds position ``start(first query) + i``;
    rows past the request's context are left as allocated (zeros here).
    ``capacity`` defaults to ``block_table.shape[1] * block_size``.
    """

    device = layer_kv_cache.device
    if device.type != "cuda":
        raise RuntimeError("mi355x_paged gathers require GPU tensors")
    batch, keep = batch_descriptor(metadata, device)
    if capacity is None:
        capacity = metadata.block_table.shape[1] * metadata.block_size
    shape = (metadata.num_requests, capacity, *layer_kv_cache.shape[3:])
    keys = torch.zeros(shape, dtype=layer_kv_cache.dtype, device=device)
    values = torch.zeros(shape, dtype=layer_kv_cache.dtype, device=device)
    lib = _native.load()
    _native.check(
        lib.mvllm_gather_kv(
            _native.kv_cache(layer_kv_cache),
            batch,
            capacity,
            keys.data_ptr() if keys.numel() else None,
            values.data_ptr() if values.numel() else None,
            _native.stream_handle(device),
        ),
        "mvllm_gather_kv",
    )
    del keep
    return keys, values


class MI355XPagedAttentionOperator(AttentionOperator):
    """gfx950 HIP paged attention: split-KV MFMA decode + MFMA prefill."""

    def forward(
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        layer_kv_cache: torch.Tensor,
        metadata: AttentionMetadata,
        /,
    ) -> torch.Tensor:
        return hip_paged_attention(
            query,
            key,
            value,
            layer_kv_cache,
            metadata,
        )
