"""Pins the CPU oracle before it is trusted.

Each oracle function is checked against something independent of its own
formula:

* the reference tests' literal vectors (tests/golden/reference_vectors.json):
  KV write placement, gathers, the 25.0 visibility-start case, the fp16
  single-key identity, slot mappings, block-table padding, flattening,
  sampling rows, per-group metadata, graph padding, context starts;
* closed forms: a two-key softmax with a known answer (pins the
  1/sqrt(head_dim) scale and the causal direction), GQA head mapping with
  constant per-head values, torch's own bfloat16 rounding;
* brute force: the paged per-request oracle against the float64 dense
  attention over contiguous K/V, over the reference tests' equivalence
  classes (MHA/GQA/MQA, bounded specs, chunked == full, prefill+decode ==
  full, mixed == independent, non-contiguous blocks, stale blocks, shared
  prefix) and a config-1-shaped ragged batch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from _golden import (
    GOLDEN,
    SPEC_KINDS,
    batch_from_case,
    cache_from_case,
    key_value,
    linspace_tensors,
    requests_from_case,
)

# ---------------------------------------------------------------- numerics


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    values = np.concatenate(
        [
            rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-8, 8, 4096),
            np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 3.3895e38], np.float32),
        ]
    ).astype(np.float32)
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_bits(values), expected)
    # Ties go to even.
    assert oracle.f32_to_bf16_bits(np.array([1.0 + 2**-8], np.float32))[0] == 0x3F80
    assert oracle.f32_to_bf16_bits(np.array([1.0 + 3 * 2**-8], np.float32))[0] == 0x3F82
    assert np.isnan(oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]
    # Widening is exact.
    bits = np.arange(0, 0x7F80, 7, dtype=np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(bits)), bits)


# ----------------------------------------------------------- golden vectors


@pytest.mark.parametrize("c", GOLDEN["spec_cases"], ids=lambda c: f"{c['spec'][0]}-{c['spec'][1]}-{c['positions']}")
def test_context_starts_match_reference_vectors(c):
    kind = SPEC_KINDS[c["spec"][0]]
    got = oracle.context_starts(kind, c["spec"][1], np.array(c["positions"]))
    assert got.tolist() == c["expect"]


@pytest.mark.parametrize("c", GOLDEN["cache_cases"], ids=lambda c: c["name"])
def test_cache_cases_match_reference_vectors(c):
    if c["op"] == "gather_slots":
        batch = batch_from_case(c)
        for r, expected in enumerate(c["expect_gathered_slots"]):
            _, first, length = oracle.paged_attention.request_key_range(batch, r)
            slots = oracle.map_cache_slots(np.arange(first, length), batch.block_table[r], batch.block_size)
            assert slots.tolist() == expected
        return
    cache = cache_from_case(c)
    if c["op"] == "write":
        key, value = key_value(c)
        oracle.write_kv_cache(key, value, cache, np.array(c["slot_mapping"]))
        flat = cache.reshape(2, -1, *cache.shape[3:])
        for plane, slots in c["expect_slots"].items():
            for slot, rows in slots.items():
                assert np.array_equal(flat[int(plane), int(slot)], np.array(rows))
        for slot in c.get("expect_zero_slots", []):
            assert not np.any(flat[:, slot])
        for block, fill in c.get("expect_block_fill", {}).items():
            assert np.all(cache[:, int(block)] == fill)
        return
    batch = batch_from_case(c)
    if c["op"] == "write_then_gather":
        key, value = key_value(c)
        oracle.write_kv_cache(key, value, cache, batch.slot_mapping)
    histories = oracle.gather_kv_cache(cache, batch)
    assert [k.flatten().tolist() for k, _ in histories] == c["expect_keys"]
    assert [v.flatten().tolist() for _, v in histories] == c["expect_values"]


@pytest.mark.parametrize("c", GOLDEN["attention_cases"], ids=lambda c: c["name"])
def test_attention_cases_match_reference_vectors(c):
    dtype = np.float16 if c["dtype"] == "float16" else np.float32
    cache = cache_from_case(c, dtype)
    batch = batch_from_case(c)
    out = oracle.reference_forward(
        np.array(c["query"], dtype), np.array(c["key"], dtype), np.array(c["value"], dtype), cache, batch
    )
    assert out.dtype == dtype
    np.testing.assert_allclose(out.astype(np.float64), np.array(c["expect_output"]), atol=c["tolerance"], rtol=0)


@pytest.mark.parametrize("c", GOLDEN["packing_cases"], ids=lambda c: c["name"])
def test_packing_cases_match_reference_vectors(c):
    requests = requests_from_case(c)
    specs = [(SPEC_KINDS[g["spec"][0]], g["spec"][1]) for g in c.get("groups", [{"spec": ["full", 0]}])]
    packs = [
        oracle.pack(requests, group=g, block_size=c["block_size"], null_block_id=c["null_block_id"], spec=spec)
        for g, spec in enumerate(specs)
    ]
    expect = c.get("expect", {})
    p = packs[0]
    if "graph" in c:
        p = oracle.graph_pad(
            p,
            token_capacity=c["graph"]["token_capacity"],
            request_capacity=c["graph"]["request_capacity"],
            block_table_width=p["block_table"].shape[1],
            null_block_id=c["null_block_id"],
        )
        assert p["slot_mapping"][-1] == expect["last_slot"]
    for field in ("input_ids", "positions", "query_start_locations", "context_lengths",
                  "slot_mapping", "sampling_row_indices", "block_table"):
        if field in expect:
            assert p[field].tolist() == expect[field], field
    if "block_table_shape" in expect:
        assert list(p["block_table"].shape) == expect["block_table_shape"]
    if "sampling_input_ids" in expect:
        rows = p["sampling_row_indices"]
        assert p["input_ids"][rows].tolist() == expect["sampling_input_ids"]
        assert p["positions"][rows].tolist() == expect["sampling_positions"]
    for g, eg in enumerate(c.get("expect_groups", [])):
        for field, value in eg.items():
            got = packs[g]["context_starts" if field == "context_starts" else field]
            assert got.tolist() == value, (g, field)


# ------------------------------------------------------------ closed forms


def test_two_key_softmax_known_answer_pins_scale_and_causality():
    head_dim = 4
    q = np.ones((2, 1, head_dim), np.float32)
    k = np.stack([np.ones((1, head_dim)), np.zeros((1, head_dim))]).astype(np.float32)
    v = np.stack([np.full((1, head_dim), 1.0), np.zeros((1, head_dim))]).astype(np.float32)
    cache = np.zeros((2, 2, 2, 1, head_dim), np.float32)
    batch = oracle.make_batch([[0, 1]], [[1, 0]], block_size=2, null_block_id=0)
    out = oracle.reference_forward(q, k, v, cache, batch)
    # Query 0 sees only key 0; query 1 sees scores 4/sqrt(4)=2 and 0.
    assert np.all(out[0] == 1.0)
    expected = math.exp(2.0) / (math.exp(2.0) + 1.0)
    np.testing.assert_allclose(out[1], expected, rtol=1e-6)
    np.testing.assert_allclose(
        oracle.dense_attention(q, k, v)[1, 0, 0], expected, rtol=1e-12
    )


def test_gqa_maps_consecutive_query_heads_to_one_kv_head():
    rng = np.random.default_rng(1)
    num_tokens, head_dim = 5, 8
    q = rng.standard_normal((num_tokens, 4, head_dim)).astype(np.float32)
    k = rng.standard_normal((num_tokens, 2, head_dim)).astype(np.float32)
    v = np.empty((num_tokens, 2, head_dim), np.float32)
    v[:, 0] = 10.0
    v[:, 1] = 20.0
    cache = np.zeros((2, 4, 2, 2, head_dim), np.float32)
    batch = oracle.make_batch([list(range(num_tokens))], [[3, 0, 2]], block_size=2, null_block_id=1)
    out = oracle.reference_forward(q, k, v, cache, batch)
    np.testing.assert_allclose(out[:, :2], 10.0, rtol=1e-6)
    np.testing.assert_allclose(out[:, 2:], 20.0, rtol=1e-6)


def test_uncovered_tokens_are_zero():
    q, k, v = linspace_tensors(3)
    cache = np.zeros((2, 4, 2, 2, 3), np.float32)
    batch = oracle.make_batch([[0, 1]], [[2]], block_size=2, null_block_id=3)
    padded = oracle.Batch(
        query_positions=np.array([0, 1, 0]),
        query_context_start_positions=np.zeros(3, np.int64),
        query_start_locations=np.array([0, 2, 2]),
        context_lengths=np.array([2, 0]),
        block_table=np.array([[2], [3]]),
        slot_mapping=np.array([4, 5, -1]),
        block_size=2,
    )
    out = oracle.reference_forward(q, k, v, cache, padded)
    assert not np.any(out[2])
    ref = oracle.reference_forward(q[:2], k[:2], v[:2], np.zeros_like(cache), batch)
    np.testing.assert_array_equal(out[:2], ref)
    # Slot -1 wrote nothing.
    assert not np.any(cache[:, 3])


# ---------------------------------------------- brute force vs dense float64


def _paged_vs_dense(query, key, value, positions_per_request, tables, *, block_size, num_blocks, spec=(oracle.FULL, 0)):
    cache = np.zeros((2, num_blocks, block_size, key.shape[1], key.shape[2]), np.float32)
    batch = oracle.make_batch(positions_per_request, tables, block_size=block_size, null_block_id=num_blocks - 1, spec=spec)
    return oracle.reference_forward(query, key, value, cache, batch), batch


@pytest.mark.parametrize("num_kv_heads", [4, 2, 1])
def test_dense_equivalence_mha_gqa_mqa(num_kv_heads):
    q = (np.arange(24, dtype=np.float32).reshape(3, 4, 2) / 10)
    k = (np.arange(3 * num_kv_heads * 2, dtype=np.float32).reshape(3, num_kv_heads, 2) / 20)
    v = k + 1
    out, _ = _paged_vs_dense(q, k, v, [[0, 1, 2]], [[2, 0]], block_size=2, num_blocks=4)
    np.testing.assert_allclose(out, oracle.dense_attention(q, k, v), atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("num_kv_heads", [4, 2])
@pytest.mark.parametrize(
    "spec", [(oracle.SLIDING_WINDOW, 2), (oracle.SLIDING_WINDOW, 4), (oracle.SLIDING_WINDOW, 6),
             (oracle.CHUNKED_LOCAL, 2), (oracle.CHUNKED_LOCAL, 4), (oracle.CHUNKED_LOCAL, 6)]
)
def test_dense_equivalence_bounded_specs(spec, num_kv_heads):
    q, k, v = linspace_tensors(9, 4, num_kv_heads, 3)
    out, batch = _paged_vs_dense(q, k, v, [list(range(9))], [[4, 1, 3]], block_size=4, num_blocks=6, spec=spec)
    expected = oracle.dense_attention(
        q, k, v, query_positions=batch.query_positions, query_context_starts=batch.query_context_start_positions
    )
    np.testing.assert_allclose(out, expected, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("spec", [(oracle.FULL, 0), (oracle.SLIDING_WINDOW, 3), (oracle.CHUNKED_LOCAL, 4)])
def test_chunked_prefill_and_decode_equal_full_sequence(spec):
    q, k, v = linspace_tensors(8)
    table = [[6, 1, 4]]
    cache = np.zeros((2, 7, 3, 2, 3), np.float32)
    outs = []
    for start, end in ((0, 3), (3, 6), (6, 7), (7, 8)):
        batch = oracle.make_batch([list(range(start, end))], table, block_size=3, null_block_id=0, spec=spec)
        outs.append(oracle.reference_forward(q[start:end], k[start:end], v[start:end], cache, batch))
    positions = np.arange(8)
    expected = oracle.dense_attention(
        q, k, v, query_positions=positions, query_context_starts=oracle.context_starts(spec[0], spec[1], positions)
    )
    np.testing.assert_allclose(np.concatenate(outs), expected, atol=1e-6, rtol=1e-6)


def test_mixed_batch_equals_independent_requests():
    qa, ka, va = linspace_tensors(2)
    qb, kb, vb = linspace_tensors(3)
    qb, kb, vb = qb + 0.3, kb - 0.2, vb + 0.5
    cache = np.zeros((2, 4, 2, 2, 3), np.float32)
    oracle.reference_forward(qb[:2], kb[:2], vb[:2], cache, oracle.make_batch([[0, 1]], [[2, 3]], block_size=2, null_block_id=1))
    mixed = oracle.reference_forward(
        np.concatenate((qa, qb[2:])), np.concatenate((ka, kb[2:])), np.concatenate((va, vb[2:])), cache,
        oracle.make_batch([[0, 1], [2]], [[0], [2, 3]], block_size=2, null_block_id=1),
    )
    np.testing.assert_allclose(mixed[:2], oracle.dense_attention(qa, ka, va), atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(mixed[2:], oracle.dense_attention(qb, kb, vb)[2:], atol=1e-6, rtol=1e-6)


def test_non_contiguous_blocks_and_stale_data_do_not_change_attention():
    q, k, v = linspace_tensors(6)
    a, _ = _paged_vs_dense(q, k, v, [list(range(6))], [[0, 1, 2]], block_size=2, num_blocks=5)
    cache = np.full((2, 5, 2, 2, 3), 1e3, np.float32)  # stale garbage everywhere
    batch = oracle.make_batch([list(range(6))], [[4, 1, 3]], block_size=2, null_block_id=0)
    b = oracle.reference_forward(q, k, v, cache, batch)
    np.testing.assert_allclose(a, b, atol=1e-6, rtol=1e-6)


def test_shared_prefix_gives_identical_history_attention():
    pq, pk, pv = linspace_tensors(2, 2, 1, 3)
    cache = np.zeros((2, 3, 2, 1, 3), np.float32)
    oracle.reference_forward(pq, pk, pv, cache, oracle.make_batch([[0, 1]], [[0]], block_size=2, null_block_id=2))
    q, k, v = linspace_tensors(1, 2, 1, 3)
    q, k, v = q + 0.25, k - 0.15, v + 0.35
    out = oracle.reference_forward(
        np.concatenate((q, q)), np.concatenate((k, k)), np.concatenate((v, v)), cache,
        oracle.make_batch([[2], [2]], [[0, 1], [0, 2]], block_size=2, null_block_id=2),
    )
    expected = oracle.dense_attention(np.concatenate((pq, q)), np.concatenate((pk, k)), np.concatenate((pv, v)))[-1]
    np.testing.assert_allclose(out[0], expected, atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(out[1], expected, atol=1e-6, rtol=1e-6)


def test_ragged_config1_batch_matches_dense():
    """Config-1 shape: contexts [17, 64, 130, 255]; a 17-token prefill and
    three decodes; 16/8 heads, head_dim 128, block 16, blocks from a
    permutation of a 64-block pool (null block 64)."""

    rng = np.random.default_rng(0)
    lengths = [17, 64, 130, 255]
    queries = [17, 1, 1, 1]
    hq, hkv, d, bs = 16, 8, 128, 16
    perm = rng.permutation(64)
    tables, cursor = [], 0
    for L in lengths:
        n = -(-L // bs)
        tables.append(perm[cursor : cursor + n].tolist())
        cursor += n
    full_k = [rng.standard_normal((L, hkv, d)).astype(np.float32) for L in lengths]
    full_v = [rng.standard_normal((L, hkv, d)).astype(np.float32) for L in lengths]
    full_q = [rng.standard_normal((L, hq, d)).astype(np.float32) for L in lengths]
    cache = np.full((2, 65, bs, hkv, d), np.nan, np.float32)
    flat = cache.reshape(2, -1, hkv, d)
    for r, L in enumerate(lengths):
        hist = np.arange(L - queries[r])
        slots = oracle.map_cache_slots(hist, np.array(tables[r]), bs)
        flat[0, slots] = full_k[r][: L - queries[r]]
        flat[1, slots] = full_v[r][: L - queries[r]]
    batch = oracle.make_batch([list(range(L - q, L)) for L, q in zip(lengths, queries)], tables, block_size=bs, null_block_id=64)
    q = np.concatenate([full_q[r][L - queries[r]:] for r, L in enumerate(lengths)])
    k = np.concatenate([full_k[r][L - queries[r]:] for r, L in enumerate(lengths)])
    v = np.concatenate([full_v[r][L - queries[r]:] for r, L in enumerate(lengths)])
    out = oracle.reference_forward(q, k, v, cache, batch)
    cursor = 0
    for r, L in enumerate(lengths):
        expected = oracle.dense_attention(full_q[r], full_k[r], full_v[r])[L - queries[r]:]
        np.testing.assert_allclose(out[cursor : cursor + queries[r]], expected, atol=2e-5, rtol=1e-5)
        cursor += queries[r]
    assert not np.isnan(out).any()


# ------------------------------- the torch CPU path (bench's CPU baseline)


def _torch_call(torch, q, k, v, cache, batch):
    from oracle import reference_cpu

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    return reference_cpu.reference_forward(
        t(q), t(k), t(v), cache,
        t(batch.query_positions), t(batch.query_context_start_positions), t(batch.query_start_locations),
        t(batch.context_lengths), t(batch.block_table), t(batch.slot_mapping), batch.block_size,
    )


@pytest.mark.parametrize("c", GOLDEN["attention_cases"], ids=lambda c: c["name"])
def test_torch_cpu_path_matches_reference_vectors(c):
    torch = pytest.importorskip("torch")
    dtype = np.float16 if c["dtype"] == "float16" else np.float32
    cache = torch.from_numpy(cache_from_case(c, dtype))
    batch = batch_from_case(c)
    out = _torch_call(torch, np.array(c["query"], dtype), np.array(c["key"], dtype), np.array(c["value"], dtype), cache, batch)
    np.testing.assert_allclose(out.double().numpy(), np.array(c["expect_output"]), atol=c["tolerance"], rtol=0)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_torch_cpu_path_matches_the_oracle_on_a_ragged_gqa_batch(dtype):
    """A 40-token chunk at offset 20, two decodes and a 3-token chunk, 8 q /
    2 KV heads, head_dim 16, block 4, shuffled blocks: the cache after the
    write is bit-identical and the outputs agree to fp32 rounding."""

    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    lengths, qlens = [60, 9, 33, 5], [40, 1, 1, 3]
    need = [-(-L // 4) for L in lengths]
    pool = rng.permutation(sum(need) + 2)
    tables, cursor = [], 0
    for n in need:
        tables.append(pool[cursor : cursor + n].tolist())
        cursor += n
    num_blocks = len(pool) + 1
    positions = [list(range(L - q, L)) for L, q in zip(lengths, qlens)]
    batch = oracle.make_batch(positions, tables, block_size=4, null_block_id=num_blocks - 1)
    n = sum(qlens)
    tdt = torch.float32 if dtype == "float32" else torch.bfloat16
    q = torch.randn(n, 8, 16).to(tdt)
    k = torch.randn(n, 2, 16).to(tdt)
    v = torch.randn(n, 2, 16).to(tdt)
    cache = torch.randn(2, num_blocks, 4, 2, 16).to(tdt)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()  # noqa: E731
    np_cache = bits(cache).copy()
    oracle.write_kv_cache(bits(k), bits(v), np_cache, batch.slot_mapping)
    expected = oracle.reference_forward(
        oracle.to_f32(bits(q)), oracle.to_f32(bits(k)), oracle.to_f32(bits(v)), oracle.to_f32(np_cache), batch
    )
    out = _torch_call(torch, bits(q), bits(k), bits(v), cache, batch) if dtype == "float32" else None
    if dtype == "bfloat16":
        from oracle import reference_cpu

        t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
        out = reference_cpu.reference_forward(
            q, k, v, cache, t(batch.query_positions), t(batch.query_context_start_positions),
            t(batch.query_start_locations), t(batch.context_lengths), t(batch.block_table), t(batch.slot_mapping), 4,
        )
    assert np.array_equal(bits(cache), np_cache)
    tol = 1e-5 if dtype == "float32" else 8e-3  # bf16 output rounding
    np.testing.assert_allclose(out.float().numpy(), expected, atol=tol, rtol=tol)
