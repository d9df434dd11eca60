"""Prefix-cache block identities (the reference's core/prefix_cache.py:12-40
and cache_group_manager.py:193-212) and the incremental chain.

Pinned by the reference's known answer (tests/core/test_prefix_cache.py:28-35:
the digest of tokens (1, 2, 3, 4), block size 4, namespace "model-a") and by
its sensitivity properties (:50-92). The incremental chain must reproduce
the from-scratch digests exactly.
"""

from __future__ import annotations

import numpy as np
import pytest

from micro_vllm_amd.harness.prefix_hash import BlockHashChain, block_hashes, hash_block, measure_step_cost


def make(tokens, parent=None, namespace="model-a", group=0):
    return hash_block(parent, tokens, block_size=len(tokens), cache_namespace=namespace, cache_group_id=group)


def test_known_answer_from_the_reference_tests():
    assert make((1, 2, 3, 4)).hex() == "fe7ca7b417786c985f1887b3d0ac9dace5ab4cbb74e201f115d7ee22cd15a52e"
    assert make((1, 2, 3, 4)) == make([1, 2, 3, 4])  # sequence type does not matter
    assert len(make((1, 2, 3, 4))) == 32


def test_parent_tokens_namespace_and_group_are_part_of_the_digest():
    p1, p2 = make((1, 2)), make((3, 4))
    assert make((5, 6), parent=p1) != make((5, 6), parent=p2)
    assert make((3, 4), parent=p1) != make((3, 5), parent=p1)
    assert make((1, 2), namespace="model-a") != make((1, 2), namespace="model-b")
    assert make((1, 2), group=0) == make((1, 2))
    assert make((1, 2), group=1) != make((1, 2))
    # No parent differs from any parent (the 0x00 / 0x01 marker).
    assert make((5, 6)) != make((5, 6), parent=make((5, 6)))


def test_negative_token_ids_are_rejected():
    with pytest.raises(OverflowError):
        make((1, -2))


def test_chain_links_each_block_to_its_parent():
    tokens = list(range(100, 164))
    chain = block_hashes(tokens, 4, block_size=16, cache_namespace="m")
    parent = None
    for b in range(4):
        parent = hash_block(parent, tokens[16 * b : 16 * b + 16], block_size=16, cache_namespace="m")
        assert chain[b] == parent
    assert block_hashes(tokens, 0, block_size=16, cache_namespace="m") == ()


def test_incremental_chain_equals_from_scratch_chains():
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, 2**40, size=700).tolist()
    chain = BlockHashChain(block_size=16, cache_namespace="m", cache_group_id=2)
    for n in (0, 5, 16, 17, 160, 161, 400, 700, 700):
        want = block_hashes(tokens[:n], n // 16, block_size=16, cache_namespace="m", cache_group_id=2)
        assert chain.extend(tokens[:n], n // 16) == want
    # Asking for fewer blocks returns a prefix of the same digests.
    assert chain.extend(tokens, 3) == want[:3]


def test_vectorized_chain_gives_the_same_digests():
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, 2**40, size=500).tolist()
    plain = BlockHashChain(block_size=16, cache_namespace="model-a", cache_group_id=1)
    fast = BlockHashChain(block_size=16, cache_namespace="model-a", cache_group_id=1, vectorized=True)
    for n in (0, 15, 16, 48, 49, 300, 500):
        assert fast.extend(tokens[:n], n // 16) == plain.extend(tokens[:n], n // 16)
    known = BlockHashChain(block_size=4, cache_namespace="model-a", vectorized=True)
    assert known.extend((1, 2, 3, 4), 1)[0].hex() == "fe7ca7b417786c985f1887b3d0ac9dace5ab4cbb74e201f115d7ee22cd15a52e"
    with pytest.raises(ValueError):
        BlockHashChain(block_size=4, cache_namespace="m", vectorized=True).extend((1, 2, -3, 4), 1)


def test_measure_step_cost_reports_both_paths():
    r = measure_step_cost([100, 300], steps=2)
    assert r["requests"] == 2 and r["full_blocks"] == 100 // 16 + 300 // 16
    assert r["from_scratch_ms_per_step"] >= 0 and r["incremental_ms_per_step"] >= 0
