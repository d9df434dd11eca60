"""Scheduling semantics of the end-to-end harness (host only).

Mirrors the reference scheduler's behaviour (core/scheduler.py:72-223) on
small cases: token budget and chunked prefill, running-first order, FIFO
admission, the sequence cap, sampling only at the end of the known tokens,
and newest-victim preemption when the block pool runs dry.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from micro_vllm_amd.harness import GenerationEngine, Request
from micro_vllm_amd.harness.model import DecoderConfig


def engine(num_blocks=64, budget=8, seqs=4):
    cfg = DecoderConfig.qwen3_0_6b(num_hidden_layers=1, num_key_value_heads=1, head_dim=8, vocab_size=32)
    model = SimpleNamespace(config=cfg, dtype=torch.float32, device=torch.device("cpu"))
    return GenerationEngine(model, num_blocks=num_blocks, block_size=4, max_num_batched_tokens=budget, max_num_seqs=seqs)


def summary(plan):
    return [(s.request_id, s.num_computed_tokens, s.num_scheduled_tokens, s.requires_sampling) for s in plan.scheduled_requests]


def test_budget_chunks_prefill_and_admits_fifo():
    e = engine(budget=8)
    e.add_request(Request("a", list(range(10)), max_tokens=2))
    e.add_request(Request("b", list(range(3)), max_tokens=2))
    plan = e.schedule()
    assert summary(plan) == [("a", 0, 8, False)]
    e._update(plan, [])
    plan = e.schedule()
    # running first: a finishes its prompt (2 tokens) and samples; b is admitted with the rest.
    assert summary(plan) == [("a", 8, 2, True), ("b", 0, 3, True)]
    e._update(plan, [7, 9])
    plan = e.schedule()
    assert summary(plan) == [("a", 10, 1, True), ("b", 3, 1, True)]
    assert plan.scheduled_requests[0].input_token_ids == (7,)
    e._update(plan, [1, 2])
    assert not e.has_unfinished_requests()
    assert e._requests["a"].output_token_ids == [7, 1]


def test_sequence_cap_limits_admission():
    e = engine(budget=100, seqs=2)
    for name in "abc":
        e.add_request(Request(name, [1, 2], max_tokens=1))
    plan = e.schedule()
    assert [s.request_id for s in plan.scheduled_requests] == ["a", "b"]


def test_block_tables_cover_the_scheduled_tokens():
    e = engine(budget=100)
    e.add_request(Request("a", list(range(9)), max_tokens=1))
    plan = e.schedule()
    (item,) = plan.scheduled_requests
    assert len(item.block_tables[0].block_ids) == 3  # 9 tokens in blocks of 4
    assert e.null_block_id == 63
    assert e.null_block_id not in item.block_tables[0].block_ids


def test_newest_request_is_preempted_when_blocks_run_out():
    # 5 allocatable blocks of 4 tokens (+ the null block).
    e = engine(num_blocks=6, budget=100)
    e.add_request(Request("a", list(range(8)), max_tokens=8))  # 2 blocks
    e.add_request(Request("b", list(range(12)), max_tokens=8))  # 3 blocks
    plan = e.schedule()
    assert [s.request_id for s in plan.scheduled_requests] == ["a", "b"]
    e._update(plan, [1, 1])
    # a needs a third block for token 9: b (newest) is preempted and recomputes later.
    plan = e.schedule()
    assert plan.preempted_request_ids == ("b",)
    assert summary(plan) == [("a", 8, 1, True)]
    assert e._requests["b"].num_computed_tokens == 0
    assert e.pool.num_free_blocks == 2


def test_a_request_that_can_never_fit_raises():
    e = engine(num_blocks=3, budget=100)
    e.add_request(Request("a", list(range(20)), max_tokens=1))
    with pytest.raises(RuntimeError, match="cannot fit"):
        e.schedule()


def test_duplicate_and_empty_requests_are_rejected():
    e = engine()
    e.add_request(Request("a", [1], max_tokens=1))
    with pytest.raises(ValueError):
        e.add_request(Request("a", [1], max_tokens=1))
    with pytest.raises(ValueError):
        e.add_request(Request("b", [], max_tokens=1))


# ------------------------------------------------------------- prefix cache
# Semantics of the reference's full-attention prefix cache
# (kv_cache_manager.py:113-222, cache_group_manager.py:98-132, 235-253,
# block.py:20-158, scheduler.py:124-157), block size 4.


def cached_engine(num_blocks=64, budget=100, seqs=4):
    e = engine(num_blocks=num_blocks, budget=budget, seqs=seqs)
    e.enable_prefix_cache = True
    return e


def test_second_request_starts_after_the_shared_prefix():
    e = cached_engine()
    prefix = list(range(100, 112))  # 3 full blocks
    e.add_request(Request("a", prefix + [1, 2, 3], max_tokens=2))
    plan = e.schedule()
    e._update(plan, [7])
    a_blocks = list(e._requests["a"].block_ids)
    e.add_request(Request("b", prefix + [4, 5], max_tokens=2))
    plan = e.schedule()
    b = plan.scheduled_requests[1]
    assert (b.request_id, b.num_computed_tokens, b.num_scheduled_tokens) == ("b", 12, 2)
    assert b.input_token_ids == (4, 5)
    assert b.block_tables[0].block_ids[:3] == tuple(a_blocks[:3])
    assert b.block_tables[0].block_ids[3] not in a_blocks
    assert [e.pool.ref_count(x) for x in a_blocks[:3]] == [2, 2, 2]
    assert e.prefix_hit_tokens == 12


def test_hit_never_covers_the_last_prompt_token():
    e = cached_engine()
    e.add_request(Request("a", list(range(8)), max_tokens=1))
    e._update(e.schedule(), [9])  # a finishes; its 2 full blocks stay indexed
    e.add_request(Request("b", list(range(8)), max_tokens=1))
    (b,) = e.schedule().scheduled_requests
    # (8 - 1) // 4 = 1 block may hit; the second block is recomputed.
    assert (b.num_computed_tokens, b.num_scheduled_tokens) == (4, 4)


def test_identical_blocks_computed_twice_collapse_to_one_canonical_block():
    e = cached_engine()
    e.add_request(Request("a", list(range(9)), max_tokens=3))
    e.add_request(Request("b", list(range(9)), max_tokens=3))
    plan = e.schedule()  # nothing is indexed yet: both compute their blocks
    a_ids = plan.scheduled_requests[0].block_tables[0].block_ids
    b_ids = plan.scheduled_requests[1].block_tables[0].block_ids
    assert not set(a_ids) & set(b_ids)
    free_before = e.pool.num_free_blocks
    e._update(plan, [1, 1])
    # b's two complete blocks are replaced by a's and released.
    assert e._requests["b"].block_ids[:2] == list(a_ids[:2])
    assert e._requests["b"].block_ids[2] == b_ids[2]
    assert e.pool.num_free_blocks == free_before + 2
    plan = e.schedule()
    assert plan.scheduled_requests[1].block_tables[0].block_ids[:2] == a_ids[:2]


def test_freed_blocks_stay_hittable_until_reallocated():
    e = cached_engine(num_blocks=6)  # 5 allocatable blocks
    e.add_request(Request("a", list(range(8)), max_tokens=1))
    plan = e.schedule()
    a_first = plan.scheduled_requests[0].block_tables[0].block_ids[0]
    e._update(plan, [3])  # a finishes: its blocks go to the free list, still indexed
    assert e.pool.num_free_blocks == 5
    e.add_request(Request("b", list(range(5)), max_tokens=1))
    plan = e.schedule()
    (b,) = plan.scheduled_requests
    # (5 - 1) // 4 = 1 block may hit: a's first block, taken off the free list.
    assert (b.num_computed_tokens, b.num_scheduled_tokens) == (4, 1)
    assert b.block_tables[0].block_ids[0] == a_first and e.pool.ref_count(a_first) == 1
    e._update(plan, [9])
    # A request that needs every free block reallocates them and drops their digests.
    e.add_request(Request("c", list(range(50, 70)), max_tokens=1))
    plan = e.schedule()
    assert summary(plan) == [("c", 0, 20, True)]
    e._update(plan, [4])
    e.add_request(Request("d", list(range(8)), max_tokens=1))
    (d,) = e.schedule().scheduled_requests
    assert d.num_computed_tokens == 0


def test_preempted_request_readmits_onto_the_shared_prefix():
    """A victim's blocks that another request still holds are not freed, so
    on readmission it hits the shared prefix again (the Llama-3 e2e
    configuration's pattern under preemption)."""

    e = cached_engine(num_blocks=8, budget=100)  # 7 allocatable blocks of 4
    prefix = list(range(100, 108))
    e.add_request(Request("a", prefix + [1, 2, 3, 4], max_tokens=12))
    e._update(e.schedule(), [1])
    e.add_request(Request("b", prefix + [5, 6, 7, 8], max_tokens=12))
    plan = e.schedule()
    assert summary(plan)[1] == ("b", 8, 4, True)
    shared = plan.scheduled_requests[0].block_tables[0].block_ids[:2]
    e._update(plan, [1, 1])
    preempted = readmitted = None
    for _ in range(40):
        plan = e.schedule()
        if "b" in plan.preempted_request_ids:
            preempted = True
            assert [e.pool.ref_count(x) for x in shared] == [1, 1]  # a still holds them
        for s_ in plan.scheduled_requests:
            if preempted and s_.request_id == "b" and readmitted is None:
                readmitted = s_
        e._update(plan, [1] * sum(s_.requires_sampling for s_ in plan.scheduled_requests))
        if readmitted is not None or not e.has_unfinished_requests():
            break
    assert preempted and readmitted is not None
    assert readmitted.num_computed_tokens >= 8
    assert readmitted.block_tables[0].block_ids[:2] == shared
