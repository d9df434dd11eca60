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
    assert len(e._free_blocks) == 2


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
