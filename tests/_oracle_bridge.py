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


def forward_checking_write(op, query, key, value, cache, md: AttentionMetadata) -> torch.Tensor:
    """Run ``op``'s forward on the batch and check its KV-cache write bit for
    bit over the WHOLE cache: the rows at the step's slots hold the step's
    K/V rows, and every other byte is unchanged (reference.py:84-98; slot -1
    writes nothing, test_triton_paged.py:178-247). The expected cache is
    built with torch's index assignment on the device, so full-size caches
    (gigabytes) need no host copy. Returns the forward's output."""

    hkv, d = key.shape[1], key.shape[2]
    slots = md.slot_mapping
    keep = slots >= 0
    valid = slots[keep]
    # Distinct slots: the expected write does not depend on the order.
    assert torch.unique(valid).numel() == valid.numel()
    expected = cache.clone()
    out = op(query, key, value, cache, md)
    flat = expected.view(2, -1, hkv, d)
    flat[0, valid] = key[keep]
    flat[1, valid] = value[keep]
    torch.cuda.synchronize()
    bits = torch.int16 if cache.element_size() == 2 else torch.int32
    assert torch.equal(cache.view(bits), expected.view(bits)), "KV-cache write is not bit-exact"
    del expected
    return out


def sampled_rows_step(query: torch.Tensor, cache: torch.Tensor, md: AttentionMetadata, rows) -> tuple[np.ndarray, np.ndarray]:
    """Oracle reference for chosen query rows of a step, after the GPU step
    (the cache already holds the step's K/V; check the write separately).

    The chosen rows of each request become one oracle request (their own
    positions and context starts, context length = the last chosen
    position + 1) over a compact host copy of that request's blocks, with
    every slot -1 so nothing is written. The oracle's per-query mask then
    gives each row exactly the keys it sees in the full step, so long
    contexts cost only the chosen rows. Returns (sorted rows, expected fp32
    [len(rows), Hq, D])."""

    rows = np.unique(np.asarray(rows, dtype=np.int64))
    qsl = to_oracle(md.query_start_locations)
    pos = to_oracle(md.query_positions)
    starts = to_oracle(md.query_context_start_positions)
    table = to_oracle(md.block_table)
    bs = md.block_size
    hkv, d = cache.shape[3], cache.shape[4]
    req = np.searchsorted(qsl, rows, side="right") - 1
    q32 = oracle.to_f32(to_oracle(query[torch.as_tensor(rows, device=query.device)]))
    expected = np.empty(q32.shape, np.float32)
    for r in np.unique(req):
        sel = np.nonzero(req == r)[0]
        chosen = rows[sel]
        last = int(pos[chosen].max())
        nblk = last // bs + 1
        ids = torch.as_tensor(table[r, :nblk], device=cache.device)
        compact = oracle.to_f32(to_oracle(cache[:, ids]))
        compact = np.concatenate([compact, np.zeros_like(compact[:, :1])], axis=1)  # null block
        batch = oracle.Batch(
            query_positions=pos[chosen],
            query_context_start_positions=starts[chosen],
            query_start_locations=np.array([0, len(chosen)], np.int64),
            context_lengths=np.array([last + 1], np.int64),
            block_table=np.arange(nblk, dtype=np.int64)[None],
            slot_mapping=np.full(len(chosen), -1, np.int64),
            block_size=bs,
        )
        no_kv = np.zeros((len(chosen), hkv, d), np.float32)
        expected[sel] = oracle.reference_forward(q32[sel], no_kv, no_kv, compact, batch)
    return rows, expected


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
