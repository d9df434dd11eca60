"""End-to-end greedy decoding with the HIP operator against the torch
restatement of the reference operator.

Random-init Qwen3- and Llama-shaped decoders generate with the
`mi355x_paged` operator under token budgets that force chunked prefill and
mixed steps. Every generated position is then re-derived teacher-forced with
the reference-semantics operator (`tests/_torch_reference.py`) on the same
weights, and the greedy tokens must be IDENTICAL, with no allowance.

Identity of greedy tokens is only decidable where the reference's top-2
logit gap exceeds the rounding noise between two correct bf16
implementations. The token tests therefore use the copy-head init of
`tests/_copy_model.py`: the attention of layer 0 picks the token at
t - 37 with a gap of several logit units. Each test asserts that premise
(the smallest gap is at least 4x the largest logit difference between the
two operators on the same sequences), reports the first divergent position
and its gap if there is one, and fails on it. Plain random-init models are
checked through their logits (no token claim): `test_random_init_logits_*`.
"""

from __future__ import annotations

import copy
import weakref

import numpy as np
import pytest
import torch

from _copy_model import make_copy_model
from _torch_reference import TorchReferenceAttention
from micro_vllm_amd.attention.operators.registry import get_attention_operator_class
from micro_vllm_amd.attention.spec import FullAttentionSpec
from micro_vllm_amd.harness import DecoderConfig, DecoderModel, GenerationEngine, Request
from micro_vllm_amd.worker.packing import pack_scheduler_output
from micro_vllm_amd.worker.scheduler_output import CacheGroupBlockTable, ScheduledRequest, SchedulerOutput

pytestmark = pytest.mark.gpu

VOCAB = 8192
COPY_OFFSET = 37
GAP_OVER_NOISE = 4.0   # smallest reference top-2 gap / largest logit difference


def make_requests(seed, count, lo, hi, max_tokens, vocab=VOCAB):
    rng = np.random.default_rng(seed)
    return [
        Request(f"r{i}", rng.integers(0, vocab, size=int(rng.integers(lo, hi + 1))).tolist(), max_tokens)
        for i in range(count)
    ]


@torch.inference_mode()
def teacher_forced_logits(model, sequences, device, last=None, chunk=None):
    """Logits of every position of each sequence (one prefill step); with
    ``last`` only those of each sequence's last ``last[i]`` positions. With
    ``chunk``, the sequences are prefilled ``chunk`` tokens at a time over
    the same caches (chunked prefill), which bounds the reference
    attention's score matrices on long sequences."""

    tables, block = [], 0
    for seq in sequences:
        nb = -(-len(seq) // 16)
        tables.append(tuple(range(block, block + nb)))
        block += nb
    caches = [
        torch.zeros((2, block + 1, 16, model.config.num_key_value_heads, 128), dtype=model.dtype, device=device)
        for _ in range(model.config.num_hidden_layers)
    ]
    last = last if last is not None else [len(seq) for seq in sequences]
    longest = max(len(seq) for seq in sequences)
    step = chunk or longest
    kept = [[] for _ in sequences]
    for c0 in range(0, longest, step):
        plan_items, spans = [], []
        for i, seq in enumerate(sequences):
            if c0 >= len(seq):
                continue
            n = min(step, len(seq) - c0)
            plan_items.append(
                ScheduledRequest(f"s{i}", tuple(seq[c0 : c0 + n]), c0, n, True, (CacheGroupBlockTable(tables[i]),))
            )
            spans.append((i, c0, n))
        packed = pack_scheduler_output(
            SchedulerOutput(tuple(plan_items)), specs=[FullAttentionSpec()], block_size=16, null_block_id=block,
            device=device,
        )
        hidden = model.forward(packed.input_ids, packed.positions, caches, packed.group_metadata[0])
        offset = 0
        for i, p0, n in spans:
            first = len(sequences[i]) - last[i]
            lo, hi = max(first, p0), p0 + n
            if hi > lo:
                kept[i].append(hidden[offset + lo - p0 : offset + hi - p0])
            offset += n
        del hidden
    del caches
    hidden = torch.cat([h for rows in kept for h in rows])
    return model.logits(hidden).float()


def check_against_reference(requests, hip_model, ref_model, device, group=None, chunk=None):
    """Teacher-forced check of every generated position (see module doc):
    identical greedy tokens, on a margin the test verifies. ``group`` bounds
    how many sequences are teacher-forced in one step, ``chunk`` how many
    tokens of each are prefilled at a time."""

    group = group or len(requests)
    max_diff = 0.0
    checked, min_gap, divergence = 0, float("inf"), None
    for g0 in range(0, len(requests), group):
        part = requests[g0 : g0 + group]
        sequences = [r.prompt_token_ids + r.output_token_ids[:-1] for r in part]
        last = [len(r.output_token_ids) for r in part]
        ref_logits = teacher_forced_logits(ref_model, sequences, device, last, chunk)
        hip_logits = teacher_forced_logits(hip_model, sequences, device, last, chunk)
        assert torch.isfinite(hip_logits).all()
        max_diff = max(max_diff, (hip_logits - ref_logits).abs().max().item())
        offset = 0
        for r, k in zip(part, last):
            rows = ref_logits[offset : offset + k]
            offset += k
            top2 = rows.topk(2, dim=-1)
            expected = top2.indices[:, 0].tolist()
            gap = (top2.values[:, 0] - top2.values[:, 1]).tolist()
            for i, (got, want, g) in enumerate(zip(r.output_token_ids, expected, gap)):
                checked += 1
                min_gap = min(min_gap, g)
                if got != want and divergence is None:
                    divergence = (r.request_id, i, got, want, g)
        del ref_logits, hip_logits
    print(f"{checked} positions; max |logit difference| {max_diff:.4f}; smallest reference top-2 gap {min_gap:.3f}")
    if divergence is not None:
        print("first divergence: request %s output %d: got %d, reference %d (reference gap %.4f)" % divergence)
    assert min_gap > GAP_OVER_NOISE * max_diff, "the init does not separate the top-2 logits beyond the noise"
    assert divergence is None, "greedy tokens differ from the reference-semantics operator"
    return checked


def models(device, seed=3, fused_layers=False, copy_head=True, dtype=torch.bfloat16, **overrides):
    """The HIP model and the reference-semantics model on the same weights."""

    base = overrides.pop("base", DecoderConfig.qwen3_0_6b)
    overrides.setdefault("num_hidden_layers", 2)
    overrides.setdefault("vocab_size", VOCAB)
    cfg = base(**overrides)
    hip_model = DecoderModel(
        cfg, get_attention_operator_class("mi355x_paged")(), device=device, seed=seed, fused_layers=fused_layers,
        dtype=dtype,
    )
    if copy_head:
        make_copy_model(hip_model, offset=COPY_OFFSET)
    ref_model = copy.copy(hip_model)  # the same weight tensors
    ref_model.operator = TorchReferenceAttention()
    ref_model.fused_layers = False
    return hip_model, ref_model


def test_greedy_decoding_matches_reference_attention(device):
    hip_model, ref_model = models(device)
    requests = make_requests(seed=1, count=8, lo=40, hi=200, max_tokens=12)
    engine = GenerationEngine(hip_model, num_blocks=256, max_num_batched_tokens=160, max_num_seqs=6, max_model_len=512)
    result = engine.generate(requests)
    assert result.output_tokens == 8 * 12
    assert result.steps > 12  # chunked prefill and mixed steps happened
    assert check_against_reference(requests, hip_model, ref_model, device) == 8 * 12


def test_greedy_decoding_with_decode_graphs_matches_reference_attention(device):
    hip_model, ref_model = models(device, seed=5)
    requests = make_requests(seed=2, count=7, lo=40, hi=150, max_tokens=16)
    engine = GenerationEngine(
        hip_model, num_blocks=256, max_num_batched_tokens=512, max_num_seqs=8, max_model_len=512, decode_graphs=True
    )
    result = engine.generate(requests)
    assert result.output_tokens == 7 * 16
    assert set(engine.graphs.entries) >= {8}  # decode steps ran as graphs
    check_against_reference(requests, hip_model, ref_model, device)
    # The captured graphs go with the engine's last reference, not with a
    # later cyclic collection (which may fall inside another capture).
    graphs = weakref.ref(engine.graphs)
    del engine, result
    assert graphs() is None


@pytest.mark.parametrize("qk_norm", [True, False], ids=["qwen3", "llama3-style"])
def test_fused_layer_kernels_match_reference_decoding(device, qk_norm):
    """The fused residual/RMSNorm, q/k-norm + rotary + cache-write and SwiGLU
    kernels, with decode steps as graphs, against the torch layers and the
    reference-semantics operator."""

    hip_model, ref_model = models(device, seed=9, fused_layers=True, qk_norm=qk_norm)
    requests = make_requests(seed=6, count=7, lo=40, hi=160, max_tokens=12)
    engine = GenerationEngine(
        hip_model, num_blocks=256, max_num_batched_tokens=200, max_num_seqs=8, max_model_len=512, decode_graphs=True
    )
    result = engine.generate(requests)
    assert result.output_tokens == 7 * 12
    check_against_reference(requests, hip_model, ref_model, device)


def test_fused_layer_kernels_match_reference_decoding_in_fp16(device):
    """The same in float16: the fused layer kernels, the embedding lookup, the
    decode graphs with the fp16 attention kernels and the argmax, against the
    torch layers and the reference-semantics operator in float16."""

    hip_model, ref_model = models(device, seed=12, fused_layers=True, dtype=torch.float16)
    requests = make_requests(seed=8, count=7, lo=40, hi=160, max_tokens=12)
    engine = GenerationEngine(
        hip_model, num_blocks=256, max_num_batched_tokens=200, max_num_seqs=8, max_model_len=512, decode_graphs=True
    )
    result = engine.generate(requests)
    assert result.output_tokens == 7 * 12
    check_against_reference(requests, hip_model, ref_model, device)


def test_pipelined_decode_matches_synchronous_decode(device):
    """With the host one graph step ahead (placeholders for tokens still on
    the GPU), every request's tokens equal the synchronous engine's, with
    chunked prefill, mixed steps, a finishing request and graph buckets
    changing size in between."""

    hip_model, _ = models(device, seed=11, fused_layers=True)
    outputs = []
    for pipeline in (False, True):
        requests = make_requests(seed=8, count=9, lo=10, hi=170, max_tokens=14)
        requests[2].max_tokens = 3  # finishes early: the graph bucket shrinks
        engine = GenerationEngine(
            hip_model,
            num_blocks=256,
            max_num_batched_tokens=180,
            max_num_seqs=6,
            max_model_len=512,
            decode_graphs=True,
            pipeline=pipeline,
        )
        result = engine.generate(requests)
        assert all(t >= 0 for r in requests for t in r.output_token_ids)  # no placeholder left
        outputs.append(result.outputs)
    assert outputs[0] == outputs[1]


def test_pipelined_decode_with_preemption_matches_synchronous_decode(device):
    """A block pool too small for every request forces preemption; a victim
    may hold a token that is still on the GPU (a placeholder) and later
    recomputes its whole sequence. Tokens must equal the synchronous
    engine's."""

    hip_model, _ = models(device, seed=12)
    outputs, preemptions = [], []
    for pipeline in (False, True):
        requests = make_requests(seed=9, count=6, lo=40, hi=90, max_tokens=40)
        engine = GenerationEngine(
            hip_model,
            num_blocks=30,  # 29 usable blocks of 16 tokens for 6 requests of up to 130 tokens
            max_num_batched_tokens=512,
            max_num_seqs=6,
            max_model_len=256,
            decode_graphs=True,
            pipeline=pipeline,
        )
        result = engine.generate(requests)
        assert result.output_tokens == 6 * 40
        assert all(t >= 0 for r in requests for t in r.output_token_ids)
        outputs.append(result.outputs)
        preemptions.append(result.preemptions)
    assert preemptions[0] > 0 and preemptions[0] == preemptions[1]
    assert outputs[0] == outputs[1]


@pytest.mark.parametrize("prefix_cache", [False, True], ids=["plain", "prefix-cache"])
def test_fast_decode_steps_match_the_planned_steps(device, prefix_cache):
    """Synchronous decode-only steps taken by the engine's fast path (arrays
    instead of plan objects, token-independent bookkeeping while the GPU
    runs) against the same engine with every step planned by schedule():
    identical tokens, the same steps, and the same block pool afterwards
    (free list order, reference counts, prefix-cache index). The requests
    cross block boundaries, finish at different steps, arrive while others
    decode, and one round runs short of blocks (preemption: the fast path
    must hand such steps to schedule())."""

    hip_model, _ = models(device, seed=13, fused_layers=True)
    runs = []
    for fast in (False, True):
        requests = make_requests(seed=13, count=10, lo=20, hi=90, max_tokens=30)
        for i, r in enumerate(requests):
            r.max_tokens = 20 + 4 * i
        engine = GenerationEngine(
            hip_model, num_blocks=30, max_num_batched_tokens=128, max_num_seqs=6, max_model_len=256,
            decode_graphs=True, enable_prefix_cache=prefix_cache,
        )
        engine.fast_decode = fast
        result = engine.generate(requests)
        pool = engine.pool
        runs.append((result.outputs, result.steps, result.decode_steps, result.preemptions,
                     list(pool._free), list(pool._ref), dict(pool._index), result.fast_decode_steps))
    slow, fast = runs
    assert fast[7] > 10 and slow[7] == 0
    assert slow[3] > 0  # preemption happened
    assert fast[:7] == slow[:7]


def test_decode_graph_replays_match_eager_on_the_same_buffers(device):
    """Every replay of a captured decode step equals an eager forward on the
    same static buffers, bit for bit, with eager work between replays."""

    hip_model, _ = models(device, seed=7)
    engine = GenerationEngine(
        hip_model, num_blocks=128, max_num_batched_tokens=1024, max_num_seqs=8, max_model_len=256, decode_graphs=True
    )
    for r in make_requests(seed=4, count=5, lo=30, hi=90, max_tokens=8):
        engine.add_request(r)
    plan = engine.schedule()  # the prompts, in one step
    engine._update(plan, engine.execute(plan))
    plan = engine.schedule()  # a decode step of 5 requests
    assert engine.graphs.accepts(plan)
    entry = engine.graphs.capture(engine.graphs.bucket(len(plan.scheduled_requests)))
    engine.graphs._pack(plan, entry.buffers)
    torch.cuda.synchronize()
    with torch.inference_mode():
        eager_logits, eager_tokens = engine.graphs.forward(entry.buffers)
    eager_logits, eager_tokens = eager_logits.clone(), eager_tokens.clone()
    with torch.inference_mode():
        for _ in range(3):
            entry.logits.zero_()
            torch.cuda.synchronize()
            entry.graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(entry.logits, eager_logits)
            assert torch.equal(entry.tokens, eager_tokens)
            _ = (eager_logits.float() * 2).sum().item()  # eager work between replays


QWEN3_VOCAB = 151_936


def test_qwen3_0_6b_shape_greedy_tokens_match_reference(device):
    """The end-to-end Qwen3-0.6B configuration's model at its real shape (28
    layers, hidden 1024, 16/8 heads of 128, qk-norm, MLP 3072, vocab
    151,936, tied embeddings) through the bench's engine path: fused layer
    kernels, chunked prefill under a 2,048-token budget, HIP-graph decode
    steps, host one step ahead. 12 requests with prompts U[64, 1024] and 32
    greedy tokens each; every token must equal the reference-semantics
    operator's teacher-forced greedy choice (tests/integration/
    test_real_model_engine.py:183-207 asks the same of the real model)."""

    hip_model, ref_model = models(device, seed=21, fused_layers=True, num_hidden_layers=28, vocab_size=QWEN3_VOCAB)
    requests = make_requests(seed=21, count=12, lo=64, hi=1024, max_tokens=32, vocab=QWEN3_VOCAB)
    engine = GenerationEngine(
        hip_model,
        num_blocks=2048,
        max_num_batched_tokens=2048,
        max_num_seqs=8,
        max_model_len=1100,
        decode_graphs=True,
        pipeline=True,
    )
    result = engine.generate(requests)
    assert result.output_tokens == 12 * 32
    assert check_against_reference(requests, hip_model, ref_model, device) == 12 * 32


def test_qwen3_0_6b_config_scheduler_greedy_tokens_match_reference(device):
    """The end-to-end Qwen3-0.6B configuration's model AND scheduler settings:
    28 layers, hidden 1024, 16/8 heads of 128, qk-norm, MLP 3072, vocab
    151,936; 256 requests with prompts U[64, 1024]; max_num_batched_tokens
    8,192 and max_num_seqs 256, so prefill steps pack many prompts and mix
    with decodes; HIP-graph decode steps with the host one step ahead. Output
    lengths U[16, 40] make the running set shrink, so the decode graphs of
    buckets 256, 128 and 64 (and the smaller ones) are all replayed. Every
    one of the ~7,000 generated tokens must equal the reference-semantics
    operator's teacher-forced greedy choice."""

    hip_model, ref_model = models(device, seed=23, fused_layers=True, num_hidden_layers=28, vocab_size=QWEN3_VOCAB)
    requests = make_requests(seed=23, count=256, lo=64, hi=1024, max_tokens=16, vocab=QWEN3_VOCAB)
    rng = np.random.default_rng(24)
    for r in requests:
        r.max_tokens = int(rng.integers(16, 41))
    engine = GenerationEngine(
        hip_model,
        num_blocks=256 * 67 + 1,
        max_num_batched_tokens=8192,
        max_num_seqs=256,
        max_model_len=67 * 16,
        decode_graphs=True,
        pipeline=True,
    )
    result = engine.generate(requests)
    expected_tokens = sum(r.max_tokens for r in requests)
    assert result.output_tokens == expected_tokens
    assert {64, 128, 256} <= set(engine.graphs.entries), sorted(engine.graphs.entries)
    assert result.decode_steps >= 16
    del engine
    torch.cuda.empty_cache()
    assert check_against_reference(requests, hip_model, ref_model, device, group=32) == expected_tokens


def test_random_init_logits_agree_at_qwen3_0_6b_shape(device):
    """Plain random init (no copy head) at the real Qwen3-0.6B shape: the
    teacher-forced logits of the HIP path (fused layer kernels, HIP
    attention) and of the reference-semantics path (torch layers, torch
    reference attention) on six sequences of U[64, 1024] tokens. Logits have
    a standard deviation of ~0.6 here; bf16 rounding of the two paths may
    differ by a few units in the last place of a logit (0.0039-0.0156 at
    these magnitudes), so the bound is 0.25 on the largest difference and
    0.01 on the mean."""

    hip_model, ref_model = models(
        device, seed=22, fused_layers=True, copy_head=False, num_hidden_layers=28, vocab_size=QWEN3_VOCAB
    )
    rng = np.random.default_rng(22)
    sequences = [rng.integers(0, QWEN3_VOCAB, size=int(rng.integers(64, 1025))).tolist() for _ in range(6)]
    ref = teacher_forced_logits(ref_model, sequences, device)
    hip = teacher_forced_logits(hip_model, sequences, device)
    diff = (hip - ref).abs()
    flips = (hip.argmax(-1) != ref.argmax(-1)).sum().item()
    print(
        f"logit std {ref.std().item():.3f}; max |diff| {diff.max().item():.4f}; mean {diff.mean().item():.5f}; "
        f"greedy flips {flips} of {ref.shape[0]} positions (no token claim at this init)"
    )
    assert torch.isfinite(hip).all()
    assert diff.max().item() < 0.25
    assert diff.mean().item() < 0.01


LLAMA3_VOCAB = 128_256


def test_llama3_shared_prefix_with_preemption_greedy_tokens_match_reference(device):
    """The Llama-3-8B end-to-end configuration's pattern at reduced depth: the
    Llama-3-8B layer shape (hidden 4096, 32/8 heads of 128, MLP 14,336, vocab
    128,256), 2 layers. Six requests share a 4,096-token random prefix, each
    followed by its own suffix of U[100, 500] tokens; prefix caching on
    (config.py:112), so the prefix is computed once and every later request
    is admitted at the computed offset 4,096 on the same physical blocks
    (kv_cache_manager.py:113-134); a 512-token budget chunks every prefill;
    a 359-block pool cannot hold every running request, so older requests
    preempt newer ones (scheduler.py:100-113), which are later re-admitted
    onto the shared prefix. 64 greedy tokens per request, each equal to the
    reference-semantics operator's."""

    hip_model, ref_model = models(
        device, seed=31, fused_layers=True, base=DecoderConfig.llama3_8b, num_hidden_layers=2, vocab_size=LLAMA3_VOCAB
    )
    rng = np.random.default_rng(31)
    prefix = rng.integers(0, LLAMA3_VOCAB, size=4096).tolist()
    requests = [
        Request(f"r{i}", prefix + rng.integers(0, LLAMA3_VOCAB, size=int(rng.integers(100, 501))).tolist(), 64)
        for i in range(6)
    ]
    engine = GenerationEngine(
        hip_model,
        num_blocks=360,
        max_num_batched_tokens=512,
        max_num_seqs=8,
        max_model_len=8192,
        decode_graphs=True,
        pipeline=True,
        enable_prefix_cache=True,
        cache_namespace="llama3-shape",
    )
    result = engine.generate(requests)
    print(f"steps {result.steps}, preemptions {result.preemptions}, prefix-cache hit tokens {result.prefix_hit_tokens}")
    assert result.output_tokens == 6 * 64
    assert result.preemptions > 0
    assert result.prefix_hit_tokens >= (5 + result.preemptions) * 4096
    assert check_against_reference(requests, hip_model, ref_model, device) == 6 * 64


def test_llama3_config5_context_lengths_greedy_tokens_match_reference(device):
    """The Llama-3-8B end-to-end configuration at its own context lengths:
    the Llama-3-8B layer shape (hidden 4096, 32/8 heads of 128, MLP 14,336,
    vocab 128,256), 4 layers; four requests share a 4,096-token random
    prefix, each followed by its own suffix drawn from U[4096, 28672] with the
    longest forced to 28,672, so contexts reach 32,784 tokens. Prefix cache
    on, max_num_batched_tokens 8,192 (every prompt is chunked), HIP-graph
    decode steps with the host one step ahead; 16 greedy tokens per request,
    each equal to the reference-semantics operator's, teacher-forced in
    prefill chunks of 4,096."""

    hip_model, ref_model = models(
        device, seed=35, fused_layers=True, base=DecoderConfig.llama3_8b, num_hidden_layers=4, vocab_size=LLAMA3_VOCAB
    )
    rng = np.random.default_rng(35)
    prefix = rng.integers(0, LLAMA3_VOCAB, size=4096).tolist()
    suffixes = [28672] + [int(x) for x in rng.integers(4096, 28673, size=3)]
    requests = [
        Request(f"r{i}", prefix + rng.integers(0, LLAMA3_VOCAB, size=n).tolist(), 16) for i, n in enumerate(suffixes)
    ]
    blocks_per_request = -(-(4096 + max(suffixes) + 16) // 16)
    engine = GenerationEngine(
        hip_model,
        num_blocks=4 * blocks_per_request + 64,
        max_num_batched_tokens=8192,
        max_num_seqs=4,
        max_model_len=blocks_per_request * 16,
        decode_graphs=True,
        pipeline=True,
        enable_prefix_cache=True,
        cache_namespace="llama3-config5",
    )
    result = engine.generate(requests)
    print(f"steps {result.steps}, prefix-cache hit tokens {result.prefix_hit_tokens}, suffixes {suffixes}")
    assert result.output_tokens == 4 * 16
    assert result.prefix_hit_tokens >= 3 * 4096
    del engine
    torch.cuda.empty_cache()
    assert check_against_reference(requests, hip_model, ref_model, device, group=1, chunk=4096) == 4 * 16


def test_duplicate_prompts_share_canonical_blocks_through_the_device_block_table(device):
    """Two identical prompts admitted in the same step compute their blocks
    twice; the prefix cache then switches the second request to the first
    one's blocks (cache_group_manager.py:98-132) and the device-resident
    block table receives only those replaced entries. Decoding continues on
    the shared blocks (graphs, pipelined): both requests produce the same
    tokens, equal to the reference's."""

    hip_model, ref_model = models(device, seed=41, fused_layers=True)
    rng = np.random.default_rng(41)
    prompt = rng.integers(0, VOCAB, size=300).tolist()
    other = rng.integers(0, VOCAB, size=200).tolist()
    requests = [Request("a", list(prompt), 24), Request("b", list(prompt), 24), Request("c", other, 24)]
    engine = GenerationEngine(
        hip_model, num_blocks=128, max_num_batched_tokens=1024, max_num_seqs=4, max_model_len=512,
        decode_graphs=True, pipeline=True, enable_prefix_cache=True,
    )
    result = engine.generate(requests)
    assert result.outputs["a"] == result.outputs["b"]
    assert engine.pool.num_cached_blocks >= 300 // 16
    check_against_reference(requests, hip_model, ref_model, device)
