"""Loaders for the golden vectors in tests/golden/reference_vectors.json."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

import oracle

GOLDEN_PATH = Path(__file__).resolve().parent / "golden" / "reference_vectors.json"
GOLDEN = json.loads(GOLDEN_PATH.read_text())

SPEC_KINDS = {"full": oracle.FULL, "sliding_window": oracle.SLIDING_WINDOW, "chunked_local": oracle.CHUNKED_LOCAL}


def case(section: str, name: str) -> dict:
    for c in GOLDEN[section]:
        if c.get("name") == name:
            return c
    raise KeyError(name)


def cache_from_case(c: dict, dtype=np.float32) -> np.ndarray:
    """Build the case's initial cache (float values) as a float64 array."""

    cache = np.full(c["cache_shape"], c.get("cache_fill", 0.0), dtype=np.float64)
    for block, value in c.get("cache_block_fill", {}).items():
        cache[:, int(block)] = value
    flat = cache.reshape(2, -1, *cache.shape[3:])
    for plane, slots in c.get("cache_slots", {}).items():
        for slot, value in slots.items():
            flat[int(plane), int(slot)] = value
    return cache.astype(dtype)


def batch_from_case(c: dict) -> oracle.Batch:
    m = c["metadata"]
    return oracle.Batch(
        query_positions=np.array(m["query_positions"], dtype=np.int64),
        query_context_start_positions=np.array(m["query_context_start_positions"], dtype=np.int64),
        query_start_locations=np.array(m["query_start_locations"], dtype=np.int64),
        context_lengths=np.array(m["context_lengths"], dtype=np.int64),
        block_table=np.array(m["block_table"], dtype=np.int64),
        slot_mapping=np.array(m["slot_mapping"], dtype=np.int64),
        block_size=int(m["block_size"]),
    )


def requests_from_case(c: dict) -> list[oracle.Request]:
    return [
        oracle.Request(
            request_id=r["id"],
            input_token_ids=tuple(r["tokens"]),
            num_computed_tokens=r["computed"],
            num_scheduled_tokens=len(r["tokens"]),
            requires_sampling=r["sampling"],
            block_tables=tuple(tuple(g) for g in r["blocks"]),
        )
        for r in c["requests"]
    ]


def group_specs(c: dict) -> list[tuple[int, int]]:
    return [(SPEC_KINDS[g["spec"][0]], g["spec"][1]) for g in c.get("groups", [{"spec": ["full", 0]}])]


def key_value(c: dict) -> tuple[np.ndarray, np.ndarray]:
    key = np.array(c["key"], dtype=np.float64)
    value = np.array(c["value"], dtype=np.float64) if "value" in c else key + c["value_offset"]
    return key, value


def linspace_tensors(num_tokens: int, num_q_heads: int = 4, num_kv_heads: int = 2, head_dim: int = 3):
    """The reference tests' ``make_attention_tensors`` inputs
    (test_reference.py:427-460): linspace-filled Q/K/V in float32."""

    q = np.linspace(-0.8, 0.9, num_tokens * num_q_heads * head_dim, dtype=np.float32)
    k = np.linspace(0.7, -0.6, num_tokens * num_kv_heads * head_dim, dtype=np.float32)
    v = np.linspace(-1.0, 1.0, num_tokens * num_kv_heads * head_dim, dtype=np.float32)
    return (
        q.reshape(num_tokens, num_q_heads, head_dim),
        k.reshape(num_tokens, num_kv_heads, head_dim),
        v.reshape(num_tokens, num_kv_heads, head_dim),
    )
