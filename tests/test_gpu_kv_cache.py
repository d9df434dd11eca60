"""GPU parity of the paged KV-cache write and block gather (bit-exact).

Cases follow the reference's tests: exact slot placement and untouched
slots (test_reference.py:157-199), padding slot -1 with a NaN-sentinel cache
(test_triton_paged.py:178-247), a strided key and a masked head dimension
(test_spike_triton_paged.py:84-128), ragged gathers with a -1 table entry
(test_spike_triton_paged.py:131-212) and the literal gather vectors
(test_reference.py:202-322). At the Qwen3 decode size the write is checked
by properties (written rows equal the inputs, every other byte unchanged).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _golden import GOLDEN, batch_from_case, cache_from_case, key_value
from _oracle_bridge import assert_cache_bit_exact, to_oracle
from micro_vllm_amd import workloads
from micro_vllm_amd.attention import AttentionMetadata
from micro_vllm_amd.attention.operators.mi355x_paged import hip_gather_kv_cache, hip_write_kv_cache

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _md_from_oracle(b: oracle.Batch, device) -> AttentionMetadata:
    t = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int64, device=device)  # noqa: E731
    return AttentionMetadata(
        query_positions=t(b.query_positions),
        query_context_start_positions=t(b.query_context_start_positions),
        query_start_locations=t(b.query_start_locations),
        context_lengths=t(b.context_lengths),
        block_table=t(b.block_table),
        slot_mapping=t(b.slot_mapping),
        block_size=b.block_size,
    )


def _write_md(slots: list[int], device, block_size: int) -> AttentionMetadata:
    n = len(slots)
    return AttentionMetadata(
        query_positions=torch.arange(n, device=device),
        query_context_start_positions=torch.zeros(n, dtype=torch.int64, device=device),
        query_start_locations=torch.tensor([0, n], device=device),
        context_lengths=torch.tensor([n], device=device),
        block_table=torch.zeros((1, 1), dtype=torch.int64, device=device),
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        block_size=block_size,
    )


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("c", [c for c in GOLDEN["cache_cases"] if c["op"] == "write"], ids=lambda c: c["name"])
def test_write_golden_vectors(device, c, dtype):
    key, value = key_value(c)
    cache = torch.as_tensor(cache_from_case(c), dtype=dtype, device=device)
    expected = to_oracle(cache)
    oracle.write_kv_cache(to_oracle(torch.as_tensor(key, dtype=dtype)), to_oracle(torch.as_tensor(value, dtype=dtype)),
                          expected, np.array(c["slot_mapping"]))
    md = _write_md(c["slot_mapping"], device, c["cache_shape"][2])
    hip_write_kv_cache(torch.as_tensor(key, dtype=dtype, device=device), torch.as_tensor(value, dtype=dtype, device=device), cache, md)
    torch.cuda.synchronize()
    assert_cache_bit_exact(cache, expected)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("num_kv_heads", "head_dim", "strided"), [(2, 7, True), (8, 128, True), (8, 128, False), (1, 64, False)])
def test_write_strided_and_padding_slots_with_nan_sentinels(device, dtype, num_kv_heads, head_dim, strided):
    block_size = 4
    gen = torch.Generator(device=device).manual_seed(0)
    slots = [7, 2, -1, 8, 13]
    n = len(slots)
    if strided:
        storage = torch.randn((n, num_kv_heads, head_dim * 2), generator=gen, device=device).to(dtype)
        key = storage[..., ::2]
    else:
        key = torch.randn((n, num_kv_heads, head_dim), generator=gen, device=device).to(dtype)
    value = torch.randn((n, num_kv_heads, head_dim), generator=gen, device=device).to(dtype)
    cache = torch.full((2, 4, block_size, num_kv_heads, head_dim), float("nan"), dtype=dtype, device=device)
    expected = to_oracle(cache)
    oracle.write_kv_cache(to_oracle(key), to_oracle(value), expected, np.array(slots))
    md = _write_md(slots, device, block_size)
    hip_write_kv_cache(key, value, cache, md)
    torch.cuda.synchronize()
    assert_cache_bit_exact(cache, expected)


def test_write_at_qwen3_decode_size_touches_only_its_slots(device):
    w = workloads.qwen3_decode(device, num_seqs=256)
    before = w.cache.clone()
    hip_write_kv_cache(w.key, w.value, w.cache, w.metadata)
    torch.cuda.synchronize()
    slots = w.metadata.slot_mapping
    flat = w.cache.view(2, -1, w.num_kv_heads, w.head_dim)
    assert torch.equal(flat[0, slots], w.key)
    assert torch.equal(flat[1, slots], w.value)
    flat[:, slots] = before.view(2, -1, w.num_kv_heads, w.head_dim)[:, slots]
    assert torch.equal(w.cache, before)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("c", [c for c in GOLDEN["cache_cases"] if c["op"] in ("gather", "write_then_gather")], ids=lambda c: c["name"])
def test_gather_golden_vectors(device, c, dtype):
    cache = torch.as_tensor(cache_from_case(c), dtype=dtype, device=device)
    batch = batch_from_case(c)
    md = _md_from_oracle(batch, device)
    if c["op"] == "write_then_gather":
        key, value = key_value(c)
        hip_write_kv_cache(torch.as_tensor(key, dtype=dtype, device=device), torch.as_tensor(value, dtype=dtype, device=device), cache, md)
    keys, values = hip_gather_kv_cache(cache, md)
    torch.cuda.synchronize()
    for r, (ek, ev) in enumerate(zip(c["expect_keys"], c["expect_values"])):
        assert keys[r, : len(ek)].flatten().float().tolist() == ek
        assert values[r, : len(ev)].flatten().float().tolist() == ev


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("num_kv_heads", "head_dim"), [(2, 7), (8, 128)])
def test_ragged_gather_with_negative_table_entry_is_bit_exact(device, dtype, num_kv_heads, head_dim):
    block_size = 2
    cache = torch.arange(2 * 6 * block_size * num_kv_heads * head_dim, dtype=torch.float32, device=device)
    cache = cache.reshape(2, 6, block_size, num_kv_heads, head_dim).to(dtype)
    c = next(c for c in GOLDEN["cache_cases"] if c["name"] == "ragged_gather_with_negative_table_entry")
    batch = batch_from_case(c)
    md = _md_from_oracle(batch, device)
    keys, values = hip_gather_kv_cache(cache, md, capacity=6)
    torch.cuda.synchronize()
    host = to_oracle(cache)
    expected = oracle.gather_kv_cache(host, batch)
    for r, (ek, ev) in enumerate(expected):
        assert np.array_equal(to_oracle(keys[r, : ek.shape[0]]), ek)
        assert np.array_equal(to_oracle(values[r, : ev.shape[0]]), ev)
