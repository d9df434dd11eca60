"""Moving data between device tensors and the oracle's numpy arrays."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from micro_vllm_amd.attention import AttentionMetadata


def to_oracle(t: torch.Tensor) -> np.ndarray:
    """Device/host tensor -> oracle storage array (bf16 as uint16 bits)."""

    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype in (torch.float16, torch.float32):
        return t.contiguous().numpy().copy()
    if t.dtype == torch.int64:
        return t.contiguous().numpy().copy()
    raise TypeError(t.dtype)


def batch_to_oracle(md: AttentionMetadata) -> oracle.Batch:
    return oracle.Batch(
        query_positions=to_oracle(md.query_positions),
        query_context_start_positions=to_oracle(md.query_context_start_positions),
        query_start_locations=to_oracle(md.query_start_locations),
        context_lengths=to_oracle(md.context_lengths),
        block_table=to_oracle(md.block_table),
        slot_mapping=to_oracle(md.slot_mapping),
        block_size=md.block_size,
    )


def oracle_step(query, key, value, cache_before: torch.Tensor, md: AttentionMetadata):
    """Run the oracle on host copies: returns (cache after write as storage
    bits, fp32 attention output)."""

    cache = to_oracle(cache_before)
    batch = batch_to_oracle(md)
    oracle.write_kv_cache(to_oracle(key), to_oracle(value), cache, batch.slot_mapping)
    cache32 = oracle.to_f32(cache)
    out = oracle.reference_forward(
        oracle.to_f32(to_oracle(query)), oracle.to_f32(to_oracle(key)), oracle.to_f32(to_oracle(value)), cache32, batch
    )
    return cache, out


def assert_cache_bit_exact(gpu_cache: torch.Tensor, oracle_cache: np.ndarray) -> None:
    got = to_oracle(gpu_cache)
    if got.dtype == np.uint16:
        assert np.array_equal(got, oracle_cache)
    else:
        # Same bits, NaN sentinels included.
        assert np.array_equal(got.view(np.uint32 if got.dtype == np.float32 else np.uint16),
                              oracle_cache.view(np.uint32 if got.dtype == np.float32 else np.uint16))


def assert_attention_close(out: torch.Tensor, expected: np.ndarray, *, atol: float, rtol: float) -> None:
    got = out.detach().float().cpu()
    torch.testing.assert_close(got, torch.from_numpy(np.asarray(expected, np.float32)), atol=atol, rtol=rtol, equal_nan=True)


def subset_step(w, requests: list[int], out: torch.Tensor):
    """Oracle reference for a subset of a large workload, after the GPU step.

    Copies only the listed requests' blocks (the GPU cache already holds
    their new K/V) into a compact host cache, re-labels block ids, and runs
    the oracle attention. Returns (expected fp32 [tokens, Hq, D], GPU rows)."""

    md = w.metadata
    qsl = to_oracle(md.query_start_locations)
    blocks = [w.block_lists[r] for r in requests]
    ids = np.concatenate(blocks)
    compact = w.cache[:, torch.as_tensor(ids, device=w.cache.device)]
    cache = oracle.to_f32(to_oracle(compact))
    cache = np.concatenate([cache, np.zeros_like(cache[:, :1])], axis=1)  # null block
    null = len(ids)
    tables, positions, starts_q = [], [], []
    cursor = 0
    rows = []
    for r, b in zip(requests, blocks):
        tables.append(list(range(cursor, cursor + len(b))))
        cursor += len(b)
        L, q = int(w.context_lengths[r]), int(w.query_lengths[r])
        positions.append(list(range(L - q, L)))
        rows.extend(range(int(qsl[r]), int(qsl[r + 1])))
    batch = oracle.make_batch(positions, tables, block_size=w.block_size, null_block_id=null)
    # No write: the GPU cache already holds this step's K/V; pass slots -1.
    batch = oracle.Batch(
        query_positions=batch.query_positions,
        query_context_start_positions=batch.query_context_start_positions,
        query_start_locations=batch.query_start_locations,
        context_lengths=batch.context_lengths,
        block_table=batch.block_table,
        slot_mapping=np.full_like(batch.slot_mapping, -1),
        block_size=batch.block_size,
    )
    rows_t = torch.as_tensor(rows, device=out.device)
    q32 = oracle.to_f32(to_oracle(w.query[rows_t]))
    k32 = oracle.to_f32(to_oracle(w.key[rows_t]))
    expected = oracle.reference_forward(q32, k32, k32, cache, batch)
    return expected, out[rows_t]
