"""GPU parity of ragged paged attention against the oracle.

The bar: the cache after the step is bit-exact with the oracle's write; the
attention output is within max-abs 2e-2 / rtol 1e-2 (bf16) or 2e-3 / 2e-3
(fp16) or 1e-5 (fp32) of the oracle's fp32 reference. Scenarios follow the
reference's tests (test_triton_paged.py:119-292 with NaN-sentinel caches,
graph padding and bounded specs; test_spike_triton_paged.py:215-319 ragged
MHA/GQA/7:1/MQA/Qwen3 shapes) plus decode-kernel stress cases (contexts
around split and block boundaries, every supported group size, sliding
windows), the small mixed batch (contexts [17, 64, 130, 255]), a sampled
check of the 256-sequence Qwen3 decode batch, and graph replay.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import pytest
import torch

import oracle
from _golden import GOLDEN, batch_from_case, cache_from_case
from _oracle_bridge import (
    assert_attention_close,
    assert_cache_bit_exact,
    forward_checking_write,
    oracle_step,
    sampled_rows_step,
    subset_step,
    to_oracle,
)
from micro_vllm_amd import workloads
from micro_vllm_amd.attention import (
    Attention,
    AttentionMetadata,
    ChunkedLocalSpec,
    FullAttentionSpec,
    SlidingWindowSpec,
    map_cache_slots,
)
from micro_vllm_amd.attention.operators.registry import get_attention_operator_class

pytestmark = pytest.mark.gpu

TOL = {
    torch.bfloat16: dict(atol=2e-2, rtol=1e-2),
    torch.float16: dict(atol=2e-3, rtol=2e-3),
    torch.float32: dict(atol=1e-5, rtol=1e-5),
}


def operator():
    return get_attention_operator_class("mi355x_paged")()


def run_and_check(query, key, value, cache, md, dtype):
    before = cache.clone()
    out = operator()(query, key, value, cache, md)
    torch.cuda.synchronize()
    expected_cache, expected = oracle_step(query, key, value, before, md)
    assert out.shape == query.shape and out.dtype == query.dtype and out.device == query.device
    assert_cache_bit_exact(cache, expected_cache)
    assert_attention_close(out, expected, **TOL[dtype])
    return out


# ------------------------------------------------------------ golden cases


@pytest.mark.parametrize("c", GOLDEN["attention_cases"], ids=lambda c: c["name"])
def test_golden_attention_cases(device, c):
    dtype = torch.float16 if c["dtype"] == "float16" else torch.float32
    cache = torch.as_tensor(cache_from_case(c), dtype=dtype, device=device)
    b = batch_from_case(c)
    md = AttentionMetadata(
        query_positions=torch.as_tensor(b.query_positions, device=device),
        query_context_start_positions=torch.as_tensor(b.query_context_start_positions, device=device),
        query_start_locations=torch.as_tensor(b.query_start_locations, device=device),
        context_lengths=torch.as_tensor(b.context_lengths, device=device),
        block_table=torch.as_tensor(b.block_table, device=device),
        slot_mapping=torch.as_tensor(b.slot_mapping, device=device),
        block_size=b.block_size,
    )
    t = lambda x: torch.tensor(x, dtype=dtype, device=device)  # noqa: E731
    out = operator()(t(c["query"]), t(c["key"]), t(c["value"]), cache, md)
    torch.cuda.synchronize()
    expected = torch.tensor(c["expect_output"], dtype=torch.float64)
    torch.testing.assert_close(out.double().cpu(), expected, atol=c["tolerance"], rtol=0)


# ------------------------------- reference operator scenarios (NaN caches)

BLOCK_SIZE = 3
BLOCK_TABLE = (6, 1, 4)


def _inputs(num_tokens, device, dtype, hq=4, hkv=2, d=16):
    gen = torch.Generator(device=device).manual_seed(0)
    q = torch.randn((num_tokens, hq, d), generator=gen, device=device).to(dtype)
    k = torch.randn((num_tokens, hkv, d), generator=gen, device=device).to(dtype)
    v = torch.randn((num_tokens, hkv, d), generator=gen, device=device).to(dtype)
    cache = torch.full((2, 7, BLOCK_SIZE, hkv, d), float("nan"), dtype=dtype, device=device)
    return q, k, v, cache


def _run_chunks(attention, q, k, v, cache, chunks, dtype):
    table = torch.tensor((BLOCK_TABLE,), dtype=torch.int64, device=q.device)
    outs = []
    for start, end in chunks:
        positions = torch.arange(start, end, dtype=torch.int64, device=q.device)
        md = attention.build_metadata(
            query_positions=positions,
            query_start_locations=torch.tensor((0, end - start), device=q.device),
            context_lengths=torch.tensor((end,), device=q.device),
            block_table=table,
            slot_mapping=map_cache_slots(positions, table[0], BLOCK_SIZE),
            block_size=BLOCK_SIZE,
        )
        outs.append(run_and_check(q[start:end], k[start:end], v[start:end], cache, md, dtype))
    return torch.cat(outs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("spec", [FullAttentionSpec(), SlidingWindowSpec(3), ChunkedLocalSpec(4)], ids=repr)
@pytest.mark.parametrize("head_dim", [16, 128])
def test_full_and_chunked_prefill_and_decode(device, dtype, spec, head_dim):
    q, k, v, cache = _inputs(8, device, dtype, d=head_dim)
    attention = Attention(spec, "mi355x_paged")
    full_cache = cache.clone()
    full = _run_chunks(attention, q, k, v, full_cache, ((0, 8),), dtype)
    inc_cache = cache.clone()
    incremental = _run_chunks(attention, q, k, v, inc_cache, ((0, 3), (3, 6), (6, 7), (7, 8)), dtype)
    torch.testing.assert_close(incremental.float(), full.float(), **TOL[dtype])
    torch.testing.assert_close(full_cache, inc_cache, atol=0, rtol=0, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [16, 128])
def test_graph_padding_neither_writes_cache_nor_returns_garbage(device, dtype, head_dim):
    q, k, v, cache = _inputs(4, device, dtype, d=head_dim)
    md = AttentionMetadata(
        query_positions=torch.tensor((0, 1, 2, 0), device=device),
        query_context_start_positions=torch.zeros(4, dtype=torch.int64, device=device),
        query_start_locations=torch.tensor((0, 3, 3), device=device),
        context_lengths=torch.tensor((3, 0), device=device),
        block_table=torch.tensor((BLOCK_TABLE, (0, 0, 0)), device=device),
        slot_mapping=torch.tensor((18, 19, 20, -1), device=device),
        block_size=BLOCK_SIZE,
    )
    out = run_and_check(q, k, v, cache, md, dtype)
    assert torch.count_nonzero(out[3]) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    ("hq", "hkv", "d"),
    [(4, 4, 8), (4, 2, 8), (7, 1, 8), (4, 1, 7), (16, 8, 128), (32, 8, 128), (16, 16, 128)],
    ids=["mha", "gqa", "group7", "mqa-dim7", "qwen3", "llama3", "mha128"],
)
def test_ragged_multi_request_with_arbitrary_starts(device, dtype, hq, hkv, d):
    gen = torch.Generator(device=device).manual_seed(0)
    q = torch.randn((6, hq, d), generator=gen, device=device).to(dtype)
    k = torch.randn((6, hkv, d), generator=gen, device=device).to(dtype)
    v = torch.randn((6, hkv, d), generator=gen, device=device).to(dtype)
    cache = torch.randn((2, 6, 2, hkv, d), generator=gen, device=device).to(dtype)
    md = AttentionMetadata(
        query_positions=torch.tensor((0, 1, 2, 3, 4, 2), device=device),
        query_context_start_positions=torch.tensor((0, 0, 1, 1, 2, 0), device=device),
        query_start_locations=torch.tensor((0, 5, 6), device=device),
        context_lengths=torch.tensor((5, 3), device=device),
        block_table=torch.tensor(((3, 1, 5), (4, 0, -1)), device=device),
        slot_mapping=torch.tensor((6, 7, 2, 3, 10, 0), device=device),
        block_size=2,
    )
    run_and_check(q, k, v, cache, md, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize(
    ("hq", "hkv", "d", "bs"),
    [(8, 2, 64, 16), (6, 2, 96, 8), (12, 4, 256, 32), (4, 2, 320, 16), (4, 4, 512, 16)],
    ids=["d64", "d96-bs8", "d256-bs32", "d320", "d512"],
)
@pytest.mark.parametrize("longest", [4100, 1000], ids=["reach-4100", "reach-1000"])
def test_generic_kernel_ranges_merged_over_waves(device, dtype, hq, hkv, d, bs, longest):
    """Shapes only the generic kernel takes (fp32; head_dim 64, 96, 256, 320,
    512; block 8): visible ranges of 5 keys up to ``longest``, so the waves
    of a (token, head) workgroup (4 when the table reaches at most 1,024
    keys, 8 or 16 beyond) each walk none, one or many 64-key blocks and
    their states are merged; NaN-sentinel cache slots stay out."""

    lengths, qlens = [5, 300, min(1500, longest), longest, 64], [5, 1, 20, 1, 3]
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, hq, hkv, d, bs, seed=97)
    run_and_check(q, k, v, cache, md, dtype)


# ------------------------------------------------------ decode kernel stress


def build_case(device, dtype, lengths, qlens, hq, hkv, d, bs, spec=None, seed=0, nan_cache=True):
    """Random sequences; history rows written at their slots, everything
    else in the cache NaN (stale/unmapped slots must never be read)."""

    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    blocks_needed = [-(-L // bs) for L in lengths]
    pool = rng.permutation(sum(blocks_needed) + 3)
    num_blocks = len(pool) + 1
    tables, cursor = [], 0
    for n in blocks_needed:
        tables.append(pool[cursor : cursor + n].tolist())
        cursor += n
    fill = float("nan") if nan_cache else 0.0
    cache = torch.full((2, num_blocks, bs, hkv, d), fill, dtype=dtype, device=device)
    flat = cache.view(2, -1, hkv, d)
    positions = []
    for r, (L, ql) in enumerate(zip(lengths, qlens)):
        hist = torch.arange(0, L - ql, device=device)
        if hist.numel():
            slots = map_cache_slots(hist, torch.tensor(tables[r], device=device), bs)
            flat[0, slots] = torch.randn((hist.numel(), hkv, d), generator=gen, device=device).to(dtype)
            flat[1, slots] = torch.randn((hist.numel(), hkv, d), generator=gen, device=device).to(dtype)
        positions.append(list(range(L - ql, L)))
    kind, param = (spec.kernel_code() if spec is not None else (oracle.FULL, 0))
    b = oracle.make_batch(positions, tables, block_size=bs, null_block_id=num_blocks - 1, spec=(kind, param))
    md = AttentionMetadata(
        query_positions=torch.as_tensor(b.query_positions, device=device),
        query_context_start_positions=torch.as_tensor(b.query_context_start_positions, device=device),
        query_start_locations=torch.as_tensor(b.query_start_locations, device=device),
        context_lengths=torch.as_tensor(b.context_lengths, device=device),
        block_table=torch.as_tensor(b.block_table, device=device),
        slot_mapping=torch.as_tensor(b.slot_mapping, device=device),
        block_size=bs,
    )
    n = sum(qlens)
    q = torch.randn((n, hq, d), generator=gen, device=device).to(dtype)
    k = torch.randn((n, hkv, d), generator=gen, device=device).to(dtype)
    v = torch.randn((n, hkv, d), generator=gen, device=device).to(dtype)
    return q, k, v, cache, md


DECODE_LENGTHS = [1, 2, 15, 16, 17, 63, 64, 65, 255, 256, 257, 1000, 3000, 5003]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("hq", "hkv"), [(8, 8), (16, 8), (32, 8), (16, 2), (16, 1), (64, 4)], ids=lambda x: str(x))
def test_decode_kernel_group_sizes_and_context_boundaries(device, dtype, hq, hkv):
    lengths = DECODE_LENGTHS
    q, k, v, cache, md = build_case(device, dtype, lengths, [1] * len(lengths), hq, hkv, 128, 16, seed=hq + hkv)
    run_and_check(q, k, v, cache, md, dtype)


@pytest.mark.parametrize(
    ("requests", "longest"),
    [(128, 1024), (16, 1024), (4, 3000)],
    ids=["9-splits", "17-splits", "48-splits"],
)
def test_decode_combine_of_many_splits(device, requests, longest):
    """Split lengths follow the batch (about two items per CU, at least 64
    tokens), so smaller batches split each request more finely: on 256 CUs
    these batches reach 9, 17 and 48 splits per request, which the combine
    merges from one round of loads (up to 16 and 32) or in passes."""

    rng = np.random.default_rng(requests)
    lengths = rng.integers(1, longest + 1, size=requests)
    lengths[0] = longest
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths.tolist(), [1] * requests, 16, 8, 128, 16,
                                    seed=requests)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


@pytest.mark.parametrize("bs", [1, 5, 8, 32, 64])
def test_decode_kernel_other_block_sizes(device, bs):
    lengths = [1, 7, 33, 200, 777]
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, [1] * len(lengths), 16, 8, 128, bs, seed=bs)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


@pytest.mark.parametrize("spec", [SlidingWindowSpec(1), SlidingWindowSpec(100), SlidingWindowSpec(300), ChunkedLocalSpec(256), ChunkedLocalSpec(48)], ids=repr)
def test_decode_kernel_bounded_specs(device, spec):
    lengths = [5, 99, 100, 101, 300, 301, 1024, 2500]
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, [1] * len(lengths), 16, 8, 128, 16, spec=spec, seed=3)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_mixed_prefill_and_decode_batch(device, dtype):
    lengths = [40, 700, 1, 64, 3000, 17, 129]
    qlens = [40, 33, 1, 1, 1, 5, 1]
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, 32, 8, 128, 16, seed=11)
    run_and_check(q, k, v, cache, md, dtype)


# ----------------------------------------------------- prefill kernel stress

# Chunks of every alignment against the 16-token pages and 64-key tiles:
# whole prompts, chunks after a history, single-page and multi-tile chunks,
# chunks shorter than a workgroup's token block and ones spanning several.
PREFILL_LENGTHS = [2, 17, 64, 700, 3000, 129, 600, 1100, 5000, 90]
PREFILL_QLENS = [2, 17, 64, 33, 512, 100, 600, 77, 130, 3]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    ("hq", "hkv"),
    [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1), (32, 2)],
    ids=["g1", "g2-qwen3", "g4-llama3", "g8", "g16", "g16b"],
)
def test_prefill_kernel_group_sizes_and_chunk_offsets(device, dtype, hq, hkv):
    q, k, v, cache, md = build_case(device, dtype, PREFILL_LENGTHS, PREFILL_QLENS, hq, hkv, 128, 16, seed=hq * 7 + hkv)
    run_and_check(q, k, v, cache, md, dtype)


@pytest.mark.parametrize("bs", [32, 64])
def test_prefill_kernel_larger_blocks(device, bs):
    lengths = [40, 700, 1, 300, 2049]
    qlens = [40, 200, 1, 300, 65]
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, qlens, 32, 8, 128, bs, seed=bs)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


@pytest.mark.parametrize(
    "spec",
    [SlidingWindowSpec(1), SlidingWindowSpec(37), SlidingWindowSpec(300), ChunkedLocalSpec(64), ChunkedLocalSpec(48), ChunkedLocalSpec(256)],
    ids=repr,
)
@pytest.mark.parametrize(("hq", "hkv"), [(16, 8), (32, 8)], ids=["qwen3", "llama3"])
def test_prefill_kernel_bounded_specs(device, spec, hq, hkv):
    """Per-row windows: tiles cross every row's start, and keys before a
    window (NaN in the cache here) must never reach the output."""

    lengths = [300, 1000, 700, 129]
    qlens = [300, 250, 512, 70]
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, qlens, hq, hkv, 128, 16, spec=spec, seed=29)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_scores_that_jump_inside_unmasked_tiles(device, dtype):
    """Scores that grow sharply at key positions inside tiles no row masks.
    The bf16 kernel takes such tiles' probabilities against the running
    offset without a row maximum and must notice the growth and redo them
    (by 10, 14 and 150 powers of two over the first keys here), and both
    dtypes must rescale their accumulators."""

    lengths, qlens = [3000, 700], [64, 33]
    hq, hkv, d, bs = 32, 8, 128, 16
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, hq, hkv, d, bs, seed=41)
    gen = torch.Generator(device="cpu").manual_seed(41)
    u = torch.randn(d, generator=gen)
    u = (u / u.norm()).to(device)
    scale_log2 = math.log2(math.e) / math.sqrt(d)
    # Request 0's queries all point along u; its history keys gain a component
    # along u that lifts their scores by 10, 14 and then 150 powers of two: a
    # lane's 16 probabilities then sum to about 2^12, far above it, and past
    # the fp32 range (2^128), where skipping the redo would give infinities.
    q[:64] = (q[:64].float() * 0.1 + 8.0 * u).to(dtype)
    table = md.block_table[0]
    for lo, hi, lift in ((1024, 1536, 10.0), (1536, 2048, 14.0), (2048, 3000 - 64, 150.0)):
        c = lift / scale_log2 / 8.0
        pos = torch.arange(lo, hi, device=device)
        blocks, rows = table[pos // bs], pos % bs
        cache[0, blocks, rows] = (cache[0, blocks, rows].float() + c * u).to(dtype)
    run_and_check(q, k, v, cache, md, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("hq", "hkv"), [(16, 8), (32, 8), (16, 16)], ids=["qwen3", "llama3", "mha"])
def test_prefill_matches_platform_flash_attention(device, hq, hkv, dtype):
    """An independent cross-check beside the oracle: the chunks' outputs
    against PyTorch-ROCm's flash attention (``aten._flash_attention_forward``,
    variable-length, causal with the mask aligned to the end of each
    context, GQA by head grouping) over the same K/V, gathered from the
    cache after the forward wrote the chunks' rows. Both compute in the
    input type with fp32 accumulation."""

    flash = getattr(torch.ops.aten, "_flash_attention_forward", None)
    if flash is None:
        pytest.skip("this torch build has no flash attention operator")
    lengths = [700, 3000, 129, 600, 1100, 5000, 64]
    qlens = [33, 512, 100, 600, 77, 130, 64]
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, hq, hkv, 128, 16, seed=hq + 5 * hkv)
    out = operator()(q, k, v, cache, md)
    torch.cuda.synchronize()
    table, bs = md.block_table, md.block_size
    keys, values = [], []
    for r, length in enumerate(lengths):
        pos = torch.arange(length, device=device)
        blocks = table[r, pos // bs]
        keys.append(cache[0, blocks, pos % bs])
        values.append(cache[1, blocks, pos % bs])
    cum_q = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=device)
    cum_k = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=device)
    try:
        ref = flash(
            q.contiguous(), torch.cat(keys).contiguous(), torch.cat(values).contiguous(), cum_q, cum_k,
            max(qlens), max(lengths), 0.0, True, False, scale=1.0 / math.sqrt(128),
        )[0]
    except RuntimeError as exc:
        pytest.skip(f"flash attention is not available here: {exc}")
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), **TOL[dtype])


def test_decode_work_list_beyond_65535_slots(device, monkeypatch):
    """One 16,384-token context beside 4,095 short ones: 1,024-token splits,
    17 per request, make 69,632 decode work-list slots (more than a 2-D grid
    dimension holds); every split must be computed once and merged."""

    monkeypatch.setenv("MVLLM_DECODE_SPLIT", "1024")
    lengths = [16_384] + [5 + (i % 60) for i in range(4095)]
    qlens = [1] * len(lengths)
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, qlens, 16, 8, 128, 16, seed=47)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


def test_prefill_work_list_of_more_than_8192_slots(device):
    """8,202 requests (8,200 of two tokens) make 8,332 work-list slots, more
    than the sorted list holds (8,192): the list keeps slot order, and every
    query block must still be computed exactly once."""

    lengths = [300, 40] + [2] * 8200
    qlens = [300, 17] + [2] * 8200
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, qlens, 8, 8, 128, 16, seed=43)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


@pytest.mark.parametrize(("hq", "hkv"), [(16, 8), (32, 8)], ids=["qwen3", "llama3"])
def test_prefill_kernel_rows_outside_the_work_list_hull(device, hq, hkv):
    """Context starts that do not grow with the token: every fifth query sees
    from key 0, the others only their last 64 keys. Rows of a query block
    then reach keys before the block's first row's start (the work-list
    record's hull), and the kernel must fall back to the rows' own bounds."""

    q, k, v, cache, md = build_case(device, torch.bfloat16, [600, 300], [400, 300], hq, hkv, 128, 16, seed=53)
    pos = md.query_positions
    starts = torch.where(pos % 5 == 0, torch.zeros_like(pos), (pos - 64).clamp(min=0))
    md = AttentionMetadata(
        query_positions=md.query_positions,
        query_context_start_positions=starts,
        query_start_locations=md.query_start_locations,
        context_lengths=md.context_lengths,
        block_table=md.block_table,
        slot_mapping=md.slot_mapping,
        block_size=md.block_size,
    )
    run_and_check(q, k, v, cache, md, torch.bfloat16)


PLAN_CASES = {
    "mixed": ([300, 1000, 17, 2049, 600, 5], [300, 1, 17, 1, 64, 1]),
    "decode": ([129, 4100, 700, 16, 33, 2500], [1] * 6),
    "prefill": ([600, 90, 2100], [600, 90, 48]),
}


@pytest.mark.parametrize("case", sorted(PLAN_CASES))
def test_planned_attention_matches_per_call_lists(device, case):
    """One plan (work lists built once) serves three layers whose caches share
    the geometry but not the contents: every planned call equals the call
    that builds its own lists, bit for bit."""

    from micro_vllm_amd.attention.operators.mi355x_paged import AttentionPlan, hip_attention_over_cache

    lengths, qlens = PLAN_CASES[case]
    dtype = torch.bfloat16
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, 32, 8, 128, 16, seed=67, nan_cache=False)
    operator()(q, k, v, cache, md)  # writes the step's K/V
    caches = [cache, cache * 0.5, cache.flip(1).contiguous()]
    plan = AttentionPlan(md, 32, caches[0])
    for layer_cache in caches:
        planned = hip_attention_over_cache(q, layer_cache, md, plan=plan)
        direct = hip_attention_over_cache(q, layer_cache, md)
        torch.cuda.synchronize()
        assert torch.equal(planned.view(torch.int16), direct.view(torch.int16))


def test_prefill_beside_decode_matches_serial_step(device, monkeypatch):
    """A mixed batch runs as one step kernel (decode and prefill workgroups in
    one grid) by default, or with the step kernel off, its prefill kernel on
    a second stream beside the decode kernel. Every form must equal the
    serial step's outputs bit for bit, and the oracle's within tolerance."""

    lengths = [300, 1000, 17, 2049, 600, 5, 4000]
    qlens = [300, 1, 17, 1, 64, 1, 1]
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, qlens, 32, 8, 128, 16, seed=73)
    md = dataclasses.replace(md, max_query_len=max(qlens))  # the hint that enables the second stream
    step = run_and_check(q, k, v, cache.clone(), md, torch.bfloat16)
    monkeypatch.setenv("MVLLM_STEP_KERNEL", "0")
    overlapped = run_and_check(q, k, v, cache.clone(), md, torch.bfloat16)
    monkeypatch.setenv("MVLLM_PREFILL_CONCURRENT", "0")
    serial = run_and_check(q, k, v, cache.clone(), md, torch.bfloat16)
    assert torch.equal(overlapped.view(torch.int16), serial.view(torch.int16))
    assert torch.equal(step.view(torch.int16), serial.view(torch.int16))


@pytest.mark.parametrize(
    "dtype,hq,hkv,hint,order",
    [
        (torch.bfloat16, 32, 8, None, None),
        (torch.bfloat16, 32, 8, "max", "prefill"),
        (torch.bfloat16, 16, 8, None, "prefill"),
        (torch.float16, 16, 8, "max", None),
        (torch.bfloat16, 16, 2, None, None),
        (torch.bfloat16, 16, 1, "max", None),
        (torch.bfloat16, 24, 6, None, None),
    ],
)
def test_step_kernel_matches_separate_launches(device, monkeypatch, dtype, hq, hkv, hint, order):
    """The step kernel runs the decode and prefill kernels' own work items in
    one grid, in either order, so its outputs equal the separate launches'
    bit for bit: with and without the hint, fewer KV heads than the step's
    decode waves, and fp16."""

    lengths = [700, 2300, 33, 1, 4100, 90, 129]
    qlens = [128, 1, 33, 1, 1, 90, 1]
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, hq, hkv, 128, 16, seed=91)
    if hint == "max":
        md = dataclasses.replace(md, max_query_len=max(qlens))
    if order:
        monkeypatch.setenv("MVLLM_STEP_ORDER", order)
    step = run_and_check(q, k, v, cache.clone(), md, dtype)
    monkeypatch.setenv("MVLLM_STEP_KERNEL", "0")
    monkeypatch.setenv("MVLLM_PREFILL_CONCURRENT", "0")
    separate = run_and_check(q, k, v, cache.clone(), md, dtype)
    assert torch.equal(step.view(torch.int16), separate.view(torch.int16))


def test_step_kernel_on_a_decode_only_batch_without_the_hint(device, monkeypatch):
    """Without the hint a decode-only batch takes the step kernel, whose
    prefill workgroups all find empty records; the outputs equal the hinted
    decode-only launch's."""

    lengths = [5000, 17, 300, 2048, 2049, 1]
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, [1] * len(lengths), 16, 8, 128, 16, seed=93)
    unhinted = run_and_check(q, k, v, cache.clone(), md, torch.bfloat16)
    hinted = run_and_check(q, k, v, cache.clone(), dataclasses.replace(md, max_query_len=1), torch.bfloat16)
    assert torch.equal(unhinted.view(torch.int16), hinted.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wrong_decode_only_hint_leaves_nan_rows_not_stale_memory(device, dtype):
    """A hint of max_query_len = 1 skips the prefill launch. If a request
    has more queries anyway, its rows come back NaN (not whatever the output
    memory held); the decode rows and the cache write stay correct."""

    lengths, qlens = [40, 300, 17, 2500], [5, 1, 1, 1]
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, 16, 8, 128, 16, seed=95)
    before = cache.clone()
    out = operator()(q, k, v, cache, dataclasses.replace(md, max_query_len=1))
    torch.cuda.synchronize()
    expected_cache, expected = oracle_step(q, k, v, before, md)
    assert_cache_bit_exact(cache, expected_cache)
    assert torch.isnan(out[:5].float()).all()
    assert_attention_close(out[5:], expected[5:], **TOL[dtype])


def test_plan_for_other_metadata_is_rejected(device):
    from micro_vllm_amd.attention.operators.mi355x_paged import AttentionPlan, hip_attention_over_cache

    q, k, v, cache, md = build_case(device, torch.bfloat16, [40, 7], [40, 1], 16, 8, 128, 16, seed=71)
    _, _, _, _, md2 = build_case(device, torch.bfloat16, [40, 7], [40, 1], 16, 8, 128, 16, seed=71)
    plan = AttentionPlan(md, 16, cache)
    with pytest.raises(ValueError):
        hip_attention_over_cache(q, cache, md2, plan=plan)
    with pytest.raises(ValueError):
        hip_attention_over_cache(q[:, :8].contiguous(), cache, md, plan=plan)


def test_prefill_kernel_reloads_page_table_on_long_context(device):
    """A 40,000-key visible range spans more than one LDS page-table load
    (2,048 pages)."""

    q, k, v, cache, md = build_case(device, torch.bfloat16, [40_000, 33], [48, 33], 16, 8, 128, 16, seed=41)
    run_and_check(q, k, v, cache, md, torch.bfloat16)


def test_prefill_kernel_unmapped_pages_are_masked(device):
    """Block-table entries that are not valid block ids inside a visible
    range are treated as masked keys (the decode kernel does the same)."""

    dtype = torch.bfloat16
    q, k, v, cache, md = build_case(device, dtype, [200, 150], [200, 40], 16, 8, 128, 16, seed=43, nan_cache=False)
    table = md.block_table.clone()
    table[0, 3] = -1                      # keys 48..63 of request 0
    table[1, 1] = cache.shape[1] + 5      # keys 16..31 of request 1: out of range
    slots = md.slot_mapping.clone()
    req = torch.repeat_interleave(torch.arange(2, device=device), torch.tensor([200, 40], device=device))
    logical = md.query_positions // 16
    bad = ((req == 0) & (logical == 3)) | ((req == 1) & (logical == 1))
    slots[bad] = -1
    md2 = AttentionMetadata(
        query_positions=md.query_positions,
        query_context_start_positions=md.query_context_start_positions,
        query_start_locations=md.query_start_locations,
        context_lengths=md.context_lengths,
        block_table=table,
        slot_mapping=slots,
        block_size=16,
    )
    before = cache.clone()
    out = operator()(q, k, v, cache, md2)
    torch.cuda.synchronize()
    # Oracle: the same batch with the unmapped keys removed by a per-query
    # visibility mask, computed densely in float64.
    qf, kf, vf = q.double().cpu(), k.double().cpu(), v.double().cpu()
    flat = before.double().cpu().view(2, -1, 8, 128)
    tbl = md.block_table.cpu()
    pos = md.query_positions.cpu()
    lens = (200, 150)
    qsl = (0, 200, 240)
    expected = torch.zeros_like(qf)
    for r in range(2):
        L = lens[r]
        keys_pos = torch.arange(L)
        slot_ids = tbl[r, keys_pos // 16] * 16 + keys_pos % 16
        kc = flat[0, slot_ids].clone()
        vc = flat[1, slot_ids].clone()
        # New tokens come from this step's K/V.
        for t in range(qsl[r], qsl[r + 1]):
            kc[pos[t]] = kf[t]
            vc[pos[t]] = vf[t]
        mapped = torch.ones(L, dtype=torch.bool)
        mapped[(keys_pos // 16) == (3 if r == 0 else 1)] = False
        kc[~mapped] = 0
        vc[~mapped] = 0
        for t in range(qsl[r], qsl[r + 1]):
            for hq_ in range(16):
                sc = (kc[:, hq_ // 2] @ qf[t, hq_]) / math.sqrt(128)
                ok = mapped & (keys_pos <= pos[t])
                sc[~ok] = -math.inf
                expected[t, hq_] = torch.softmax(sc, 0) @ vc[:, hq_ // 2]
    torch.testing.assert_close(out.double().cpu(), expected, **TOL[dtype])


def check_whole_batch(w, out, group=32):
    """Every request of a large workload against the oracle, ``group``
    requests at a time (bounded host memory); also that no token outside
    the requests' rows is NaN."""

    assert not torch.isnan(out).any()
    requests = list(range(len(w.context_lengths)))
    for i in range(0, len(requests), group):
        expected, got = subset_step(w, requests[i : i + group], out)
        assert_attention_close(got, expected, **TOL[torch.bfloat16])


def test_llama3_mixed_batch_whole(device):
    """The Llama-3-head mixed batch (8 chunks of 512 at offsets U[0, 2048] +
    248 decodes U[256, 8192], 4,344 tokens) through the shipped forward (one
    step kernel, K/V written in its prologue): the whole cache bit-exact
    after the write, every request against the oracle."""

    w = workloads.llama3_mixed(device)
    out = forward_checking_write(operator(), w.query, w.key, w.value, w.cache, w.metadata)
    check_whole_batch(w, out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_mixed_batch(device, dtype):
    """Contexts [17, 64, 130, 255]: one 17-token prefill and three decodes."""

    w = workloads.small_mixed(device, dtype=dtype)
    run_and_check(w.query, w.key, w.value, w.cache, w.metadata, dtype)


def test_qwen3_decode_batch_whole(device):
    """The 256-sequence Qwen3 decode batch (contexts U[128, 4096], 70k-block
    pool) through the shipped forward: the whole 4.6 GB cache bit-exact after
    the write, every request against the oracle."""

    w = workloads.qwen3_decode(device)
    out = forward_checking_write(operator(), w.query, w.key, w.value, w.cache, w.metadata)
    check_whole_batch(w, out, group=64)


# ------------------------------------------------------ seeded random batches

RANDOM_LAYOUTS = [(16, 8, 128), (32, 8, 128), (8, 8, 128), (16, 2, 128), (64, 4, 128), (12, 4, 128), (16, 8, 64),
                  (8, 2, 96)]


def random_batch(seed: int):
    """Draw one ragged batch: head layout, block size, dtype, spec, 1-10
    requests, each a decode or a prefill chunk at a random prior context,
    and whether the max_query_len hint is given."""

    rng = np.random.default_rng(1000 + seed)
    hq, hkv, d = RANDOM_LAYOUTS[rng.integers(len(RANDOM_LAYOUTS))]
    bs = int(rng.choice([16, 16, 32, 8, 64]))
    dtype = [torch.bfloat16, torch.float16][rng.integers(2)]
    spec = [None, None, None, SlidingWindowSpec(int(rng.integers(1, 400))), ChunkedLocalSpec(int(rng.choice([16, 64, 250])))][
        rng.integers(5)
    ]
    nreq = int(rng.integers(1, 11))
    lengths, qlens = [], []
    for _ in range(nreq):
        ql = 1 if rng.random() < 0.5 else int(rng.integers(2, 301))
        prior = int(rng.integers(0, 3001))
        lengths.append(prior + ql)
        qlens.append(ql)
    hint = bool(rng.integers(2))
    return dtype, hq, hkv, d, bs, spec, lengths, qlens, hint


@pytest.mark.parametrize("seed", range(24))
def test_random_ragged_batches(device, monkeypatch, seed):
    """Seeded random batches across head layouts (the specialised kernels'
    group sizes, a group of 3 and head_dim 64 / 96 on the generic kernel),
    block sizes 8-64, bf16 / fp16, full, sliding-window and chunked-local
    specs, decodes and prefill chunks at prior contexts up to 3,000, with
    and without the max_query_len hint: the cache bit-exact, every output
    row against the oracle, and the same outputs bit for bit when the
    decode and prefill kernels run as separate launches instead of one
    step kernel."""

    dtype, hq, hkv, d, bs, spec, lengths, qlens, hint = random_batch(seed)
    q, k, v, cache, md = build_case(device, dtype, lengths, qlens, hq, hkv, d, bs, spec=spec, seed=seed)
    if hint:
        md = dataclasses.replace(md, max_query_len=max(qlens))
    print(f"seed {seed}: {dtype} heads {hq}/{hkv} d {d} block {bs} spec {spec} qlens {qlens} lengths {lengths} "
          f"hint {hint}", flush=True)
    before = cache.clone()
    out = run_and_check(q, k, v, cache, md, dtype)
    monkeypatch.setenv("MVLLM_STEP_KERNEL", "0")
    separate = operator()(q, k, v, before, md)
    torch.cuda.synchronize()
    assert torch.equal(separate.view(torch.int16), out.view(torch.int16))


# ------------------------------------------------- shared prefix (prefix cache)


def shared_prefix_case(device, prefix_len, plan, hq, hkv, seed, twins=()):
    """Requests whose block tables start with the same physical blocks (the
    prefix cache hands a hit's blocks to every request that shares the
    prefix, kv_cache_manager.py:113-134). ``plan`` lists per request
    (suffix history length, query length); each request owns the blocks
    past the prefix. Requests in a pair of ``twins`` get identical suffix
    history, queries, keys and values. Everything the batch must not read
    is NaN."""

    bs, d = 16, 128
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    prefix_blocks = prefix_len // bs
    lengths = [prefix_len + h + q for h, q in plan]
    own = [-(-L // bs) - prefix_blocks for L in lengths]
    pool = rng.permutation(prefix_blocks + sum(own) + 5)
    num_blocks = len(pool) + 1
    shared = pool[:prefix_blocks].tolist()
    tables, cursor = [], prefix_blocks
    for n in own:
        tables.append(shared + pool[cursor : cursor + n].tolist())
        cursor += n
    cache = torch.full((2, num_blocks, bs, hkv, d), float("nan"), dtype=torch.bfloat16, device=device)
    flat = cache.view(2, -1, hkv, d)
    pos = torch.arange(prefix_len, device=device)
    slots = map_cache_slots(pos, torch.tensor(shared, device=device), bs)
    flat[:, slots] = torch.randn((2, prefix_len, hkv, d), generator=gen, device=device).to(torch.bfloat16)
    suffix = {}
    for r, (h, q) in enumerate(plan):
        if h:
            hist = torch.arange(prefix_len, prefix_len + h, device=device)
            rows = torch.randn((2, h, hkv, d), generator=gen, device=device).to(torch.bfloat16)
            suffix[r] = rows
            flat[:, map_cache_slots(hist, torch.tensor(tables[r], device=device), bs)] = rows
    for first, second in twins:
        if plan[second][0]:
            hist = torch.arange(prefix_len, prefix_len + plan[second][0], device=device)
            flat[:, map_cache_slots(hist, torch.tensor(tables[second], device=device), bs)] = suffix[first]
    positions = [list(range(L - q, L)) for L, (_, q) in zip(lengths, plan)]
    b = oracle.make_batch(positions, tables, block_size=bs, null_block_id=num_blocks - 1)
    md = AttentionMetadata(
        query_positions=torch.as_tensor(b.query_positions, device=device),
        query_context_start_positions=torch.as_tensor(b.query_context_start_positions, device=device),
        query_start_locations=torch.as_tensor(b.query_start_locations, device=device),
        context_lengths=torch.as_tensor(b.context_lengths, device=device),
        block_table=torch.as_tensor(b.block_table, device=device),
        slot_mapping=torch.as_tensor(b.slot_mapping, device=device),
        block_size=bs,
        max_query_len=max(q for _, q in plan),
    )
    n = sum(q for _, q in plan)
    q_, k_, v_ = (torch.randn((n, h_, d), generator=gen, device=device).to(torch.bfloat16) for h_ in (hq, hkv, hkv))
    qsl = b.query_start_locations
    for first, second in twins:
        for t in (q_, k_, v_):
            t[qsl[second] : qsl[second + 1]] = t[qsl[first] : qsl[first + 1]]
    return q_, k_, v_, cache, md, shared


def test_shared_prefix_requests_see_identical_history(device):
    """The reference's shared-prefix case (test_reference.py:923-968) at
    GPU scale: two requests share block 0 of a 16-token prefix and decode the
    same token from different last blocks; both equal the dense oracle."""

    q, k, v, cache, md, _ = shared_prefix_case(device, 16, [(0, 1), (0, 1)], 16, 8, seed=61, twins=[(0, 1)])
    out = run_and_check(q, k, v, cache, md, torch.bfloat16)
    assert torch.equal(out[0], out[1])


@pytest.mark.parametrize(("hq", "hkv"), [(32, 8), (16, 8)], ids=["llama3", "qwen3"])
def test_shared_4096_token_prefix_suffix_prefill_and_decode(device, hq, hkv):
    """The Llama-3 e2e prefix-cache pattern: a 4,096-token prefix held once
    (256 shared blocks) and read by every request; suffix prefill chunks
    starting at the computed offset 4,096 and further in, beside decodes
    whose suffixes run past it. The prefix blocks are never written; twin
    requests (same suffix through different blocks) give identical rows."""

    plan = [(0, 512), (0, 512), (1000, 300), (2500, 1), (37, 1), (0, 1), (4000, 64)]
    q, k, v, cache, md, shared = shared_prefix_case(device, 4096, plan, hq, hkv, seed=62, twins=[(0, 1)])
    prefix_before = cache[:, shared].clone()
    out = run_and_check(q, k, v, cache, md, torch.bfloat16)
    assert torch.equal(cache[:, shared].view(torch.int16), prefix_before.view(torch.int16))
    assert torch.equal(out[:512], out[512:1024])


@pytest.mark.parametrize("hint", ["max", None], ids=["hint", "no-hint"])
def test_llama3_heads_at_long_context_positions(device, hint):
    """The Llama-3-8B end-to-end configuration's attention shapes at its own
    positions: 32/8 heads; a 4,096-token prefix held once in shared blocks
    (prefix cache, kv_cache_manager.py:113-134); suffix prefill chunks of 512
    and 704 queries at offsets 24,096 and 28,196 (after the prefix and a
    suffix history); decodes at contexts 30,097, 32,997 and 33,280 (the
    longest prefix + suffix + output, 4,096 + 28,672 + 512). The whole
    cache is checked bit-exact after the write (the prefix blocks
    untouched); 120 sampled query rows (chunk edges, 32-row and 128-row
    boundaries, random rows, every decode) are checked against the oracle
    over their full visible ranges."""

    plan = [(20_000, 512), (28_900, 1), (24_100, 704), (26_000, 1), (29_183, 1)]
    q, k, v, cache, md, shared = shared_prefix_case(device, 4096, plan, 32, 8, seed=63)
    if hint is None:
        md = dataclasses.replace(md, max_query_len=None)
    assert int(md.context_lengths.max()) == 33_280
    prefix_before = cache[:, shared].clone()
    out = forward_checking_write(operator(), q, k, v, cache, md)
    assert torch.equal(cache[:, shared].view(torch.int16), prefix_before.view(torch.int16))
    assert not torch.isnan(out).any()
    qsl = md.query_start_locations.cpu().tolist()
    rng = np.random.default_rng(63)
    rows = []
    for r, (_, n) in enumerate(plan):
        first = qsl[r]
        if n == 1:
            rows.append(first)
            continue
        edges = [0, 1, 31, 32, 63, 64, 127, 128, 255, 256, n - 2, n - 1]
        rows.extend(first + e for e in edges)
        rows.extend(first + int(x) for x in rng.choice(n, size=40, replace=False))
    rows, expected = sampled_rows_step(q, cache, md, rows)
    assert_attention_close(out[torch.as_tensor(rows, device=device)], expected, **TOL[torch.bfloat16])


@pytest.mark.parametrize("step_kernel", ["2", "0"])
def test_graph_replay_matches_eager(device, monkeypatch, step_kernel):
    q, k, v, cache, md = build_case(device, torch.bfloat16, [300, 1, 2000, 45], [1, 1, 1, 20], 16, 8, 128, 16, seed=5, nan_cache=False)
    # By default the mixed batch runs as one step kernel. With the step kernel
    # off and the hint given, the prefill runs on the library's second stream,
    # so the capture holds a fork and a join.
    monkeypatch.setenv("MVLLM_STEP_KERNEL", step_kernel)
    md = dataclasses.replace(md, max_query_len=20)
    op = operator()
    eager_cache = cache.clone()
    eager = op(q, k, v, eager_cache, md)
    torch.cuda.synchronize()
    graph_cache = cache.clone()
    op(q, k, v, graph_cache, md)  # warm up outside the graph
    graph_cache.copy_(cache)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = op(q, k, v, graph_cache, md)
    for _ in range(3):
        graph_cache.copy_(cache)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        assert torch.equal(graph_cache, eager_cache)
        # Eager work between replays.
        _ = (q.float() * 2).sum().item()


DECODE_VARIANTS = [
    {"MVLLM_DECODE_KERNEL": "general"},
    {"MVLLM_DECODE_KERNEL": "general", "MVLLM_DECODE_PREFETCH": "1", "MVLLM_DECODE_WAVES": "8"},
    {"MVLLM_DECODE_STAGES": "2", "MVLLM_DECODE_WAVES": "4"},
    {"MVLLM_DECODE_STAGES": "3", "MVLLM_DECODE_WAVES": "2"},
    {"MVLLM_DECODE_STAGES": "4", "MVLLM_DECODE_WAVES": "1"},
    {"MVLLM_DECODE_SPLIT": "64"},
    {"MVLLM_DECODE_SPLIT": "1024"},
    {"MVLLM_DECODE_SPLIT": "1536"},
    {"MVLLM_DECODE_SPLIT": "2048"},
    # Longer than the pipelined kernel takes: the general kernel, and the
    # work list's size buckets scaled to the split (contexts 3000 and 5003
    # leave partial splits of 2,992 and 911 keys).
    {"MVLLM_DECODE_SPLIT": "4096"},
]


@pytest.mark.parametrize("env", DECODE_VARIANTS, ids=lambda e: ",".join(f"{k[13:]}={v}" for k, v in e.items()))
@pytest.mark.parametrize("bs", [16, 32])
def test_decode_tuning_variants_agree_with_oracle(device, monkeypatch, env, bs):
    """Every decode kernel instantiation selectable by the launch tuning."""

    for key, val in env.items():
        monkeypatch.setenv(key, val)
    lengths = DECODE_LENGTHS
    q, k, v, cache, md = build_case(device, torch.bfloat16, lengths, [1] * len(lengths), 32, 8, 128, bs, seed=17)
    run_and_check(q, k, v, cache, md, torch.bfloat16)
