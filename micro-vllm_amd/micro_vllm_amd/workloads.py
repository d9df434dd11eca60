"""Seeded synthetic ragged batches for parity tests and benchmarks.

Each builder returns a ``Workload``: device Q/K/V for the step's new tokens,
a paged cache whose history positions are filled, and the step's
``AttentionMetadata`` built the way the reference ModelRunner builds it
(positions ``computed .. computed + scheduled - 1``, prefix-sum query starts,
context length = computed + scheduled, null-padded block table, slots by
``block_table[pos // block_size] * block_size + pos % block_size``).

Integer metadata comes from ``numpy.random.default_rng(seed)``; tensor values
from a ``torch.Generator`` seeded with the same seed on the target device.
Named builders:

* ``small_mixed``   4 requests, contexts [17, 64, 130, 255], one 17-token
                    prefill + 3 decodes, 16 q / 8 KV heads, head_dim 128,
                    block 16, fp32, blocks from a permutation of 64 + null 64.
* ``qwen3_decode``  256 decodes, contexts U[128, 4096], 16 q / 8 KV heads,
                    head_dim 128, block 16, bf16, values N(0,1)*0.5, blocks
                    drawn without replacement from a shuffled 70,000 pool.
* ``llama3_mixed``  8 prefill chunks of 512 tokens at prior offsets
                    U[0, 2048] + 248 decodes with contexts U[256, 8192]
                    (4,344 tokens), 32 q / 8 KV heads, head_dim 128, block 16,
                    bf16, values N(0,1), shuffled pool.
* ``llama3_long_decode``  64 decodes with contexts U[8192, 33280] (the
                    Llama-3-8B e2e config's prefix + suffix + decode range),
                    32 q / 8 KV heads, head_dim 128, block 16, bf16, values
                    N(0,1), shuffled pool.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from micro_vllm_amd.attention.attention import AttentionMetadata


@dataclass
class Workload:
    name: str
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor
    cache: torch.Tensor
    metadata: AttentionMetadata
    context_lengths: np.ndarray  # per request (host copy)
    query_lengths: np.ndarray    # per request (host copy)
    block_lists: list[np.ndarray]
    null_block_id: int

    @property
    def num_q_heads(self) -> int:
        return self.query.shape[1]

    @property
    def num_kv_heads(self) -> int:
        return self.key.shape[1]

    @property
    def head_dim(self) -> int:
        return self.query.shape[2]

    @property
    def block_size(self) -> int:
        return self.metadata.block_size


def build(
    name: str,
    *,
    context_lengths: np.ndarray,
    query_lengths: np.ndarray,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    pool_blocks: int,
    dtype: torch.dtype,
    value_scale: float,
    seed: int,
    device: torch.device | str,
    rng: np.random.Generator | None = None,
    fill_cache: bool = True,
) -> Workload:
    """Assemble a batch: request r has ``query_lengths[r]`` new tokens ending
    at position ``context_lengths[r] - 1``; its blocks are taken in order from
    a shuffled pool of ``pool_blocks`` ids (the null block is ``pool_blocks``)."""

    device = torch.device(device)
    rng = rng or np.random.default_rng(seed)
    context_lengths = np.asarray(context_lengths, dtype=np.int64)
    query_lengths = np.asarray(query_lengths, dtype=np.int64)
    blocks_needed = (context_lengths + block_size - 1) // block_size
    if int(blocks_needed.sum()) > pool_blocks:
        raise ValueError(f"{name}: pool of {pool_blocks} blocks is too small")
    pool = rng.permutation(pool_blocks)
    null_block = pool_blocks
    block_lists = []
    cursor = 0
    for n in blocks_needed:
        block_lists.append(pool[cursor : cursor + n].astype(np.int64))
        cursor += int(n)
    width = int(blocks_needed.max()) if len(blocks_needed) else 0
    table = np.full((len(block_lists), width), null_block, dtype=np.int64)
    for r, ids in enumerate(block_lists):
        table[r, : len(ids)] = ids
    positions = np.concatenate(
        [np.arange(L - q, L, dtype=np.int64) for L, q in zip(context_lengths, query_lengths)]
    ) if len(context_lengths) else np.zeros(0, np.int64)
    qsl = np.concatenate([[0], np.cumsum(query_lengths)]).astype(np.int64)
    req_of_token = np.repeat(np.arange(len(query_lengths)), query_lengths)
    slots = table[req_of_token, positions // block_size] * block_size + positions % block_size

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    num_tokens = int(query_lengths.sum())
    query = torch.randn((num_tokens, num_q_heads, head_dim), generator=gen, device=device, dtype=torch.float32)
    key = torch.randn((num_tokens, num_kv_heads, head_dim), generator=gen, device=device, dtype=torch.float32)
    value = torch.randn((num_tokens, num_kv_heads, head_dim), generator=gen, device=device, dtype=torch.float32)
    cache_shape = (2, pool_blocks + 1, block_size, num_kv_heads, head_dim)
    if fill_cache:
        cache = torch.empty(cache_shape, device=device, dtype=dtype)
        # Fill plane by plane in fp32 chunks to bound temporary memory.
        flat = cache.view(-1)
        chunk = 1 << 26
        for start in range(0, flat.numel(), chunk):
            n = min(chunk, flat.numel() - start)
            flat[start : start + n] = (
                torch.randn(n, generator=gen, device=device, dtype=torch.float32) * value_scale
            ).to(dtype)
    else:
        cache = torch.zeros(cache_shape, device=device, dtype=dtype)
    as_dev = lambda a: torch.as_tensor(a, dtype=torch.int64).to(device)  # noqa: E731
    metadata = AttentionMetadata(
        query_positions=as_dev(positions),
        query_context_start_positions=torch.zeros(num_tokens, dtype=torch.int64, device=device),
        query_start_locations=as_dev(qsl),
        context_lengths=as_dev(context_lengths),
        block_table=as_dev(table),
        slot_mapping=as_dev(slots),
        block_size=block_size,
        max_query_len=int(query_lengths.max()) if len(query_lengths) else 0,
    )
    return Workload(
        name=name,
        query=(query * value_scale).to(dtype),
        key=(key * value_scale).to(dtype),
        value=(value * value_scale).to(dtype),
        cache=cache,
        metadata=metadata,
        context_lengths=context_lengths,
        query_lengths=query_lengths,
        block_lists=block_lists,
        null_block_id=null_block,
    )


def small_mixed(device: torch.device | str, *, dtype: torch.dtype = torch.float32, seed: int = 0) -> Workload:
    """One 17-token prefill and three decodes at contexts 64, 130, 255."""

    return build(
        "small_mixed",
        context_lengths=np.array([17, 64, 130, 255]),
        query_lengths=np.array([17, 1, 1, 1]),
        num_q_heads=16,
        num_kv_heads=8,
        head_dim=128,
        block_size=16,
        pool_blocks=64,
        dtype=dtype,
        value_scale=1.0,
        seed=seed,
        device=device,
    )


def qwen3_decode(
    device: torch.device | str,
    *,
    num_seqs: int = 256,
    context_range: tuple[int, int] = (128, 4096),
    pool_blocks: int = 70_000,
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
) -> Workload:
    """Decode-only ragged batch with Qwen3-0.6B attention heads."""

    rng = np.random.default_rng(seed)
    lengths = rng.integers(context_range[0], context_range[1] + 1, size=num_seqs)
    return build(
        "qwen3_decode",
        context_lengths=lengths,
        query_lengths=np.ones(num_seqs, dtype=np.int64),
        num_q_heads=16,
        num_kv_heads=8,
        head_dim=128,
        block_size=16,
        pool_blocks=pool_blocks,
        dtype=dtype,
        value_scale=0.5,
        seed=seed,
        device=device,
        rng=rng,
    )


def llama3_mixed(
    device: torch.device | str,
    *,
    num_chunks: int = 8,
    chunk_tokens: int = 512,
    offset_range: tuple[int, int] = (0, 2048),
    num_decodes: int = 248,
    decode_range: tuple[int, int] = (256, 8192),
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
) -> Workload:
    """Chunked-prefill + decode continuous batch with Llama-3-8B heads."""

    rng = np.random.default_rng(seed)
    offsets = rng.integers(offset_range[0], offset_range[1] + 1, size=num_chunks)
    decode_lengths = rng.integers(decode_range[0], decode_range[1] + 1, size=num_decodes)
    lengths = np.concatenate([offsets + chunk_tokens, decode_lengths])
    queries = np.concatenate([np.full(num_chunks, chunk_tokens), np.ones(num_decodes, dtype=np.int64)])
    needed = int(((lengths + 15) // 16).sum())
    return build(
        "llama3_mixed",
        context_lengths=lengths,
        query_lengths=queries,
        num_q_heads=32,
        num_kv_heads=8,
        head_dim=128,
        block_size=16,
        pool_blocks=needed + needed // 20 + 16,
        dtype=dtype,
        value_scale=1.0,
        seed=seed,
        device=device,
        rng=rng,
    )


def llama3_long_decode(
    device: torch.device | str,
    *,
    num_seqs: int = 64,
    context_range: tuple[int, int] = (8192, 33280),
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
) -> Workload:
    """Long-context decode batch with Llama-3-8B attention heads."""

    rng = np.random.default_rng(seed)
    lengths = rng.integers(context_range[0], context_range[1] + 1, size=num_seqs)
    needed = int(((lengths + 15) // 16).sum())
    return build(
        "llama3_long_decode",
        context_lengths=lengths,
        query_lengths=np.ones(num_seqs, dtype=np.int64),
        num_q_heads=32,
        num_kv_heads=8,
        head_dim=128,
        block_size=16,
        pool_blocks=needed + needed // 20 + 16,
        dtype=dtype,
        value_scale=1.0,
        seed=seed,
        device=device,
        rng=rng,
    )


def decode_bytes(w: Workload) -> int:
    """Algorithmic HBM bytes of the attention step of a decode batch: every
    visible K and V row once, Q read, O written, the new K/V read and written
    to the cache, the block-table entries walked, query starts and lengths."""

    es = w.query.element_size()
    rows = int(w.context_lengths.sum())
    kv = rows * w.num_kv_heads * w.head_dim * 2 * es
    n = int(w.query_lengths.sum())
    qo = n * w.num_q_heads * w.head_dim * es * 2
    new_kv = n * w.num_kv_heads * w.head_dim * 2 * es * 2
    table = int(((w.context_lengths + w.block_size - 1) // w.block_size).sum()) * 8
    meta = (len(w.context_lengths) + 1) * 8 + len(w.context_lengths) * 8 + n * 8 * 3
    return kv + qo + new_kv + table + meta


def prefill_flops(w: Workload) -> int:
    """Causal-visible multiply-adds (x2) of the multi-query requests:
    4 * Hq * D * (visible (query, key) pairs)."""

    pairs = 0
    for L, q in zip(w.context_lengths, w.query_lengths):
        if q > 1:
            offset = int(L - q)
            pairs += int(q) * offset + int(q) * (int(q) + 1) // 2
    return 4 * w.num_q_heads * w.head_dim * pairs
