"""Pins tests/_torch_reference.py to the oracle before it is trusted.

The end-to-end greedy-token tests compare the HIP path with
``TorchReferenceAttention`` (a torch restatement of
ReferenceAttentionOperator.forward, src/micro_vllm/attention/operators/
reference.py:14-138). Here that checker is run on the CPU against the pinned
numpy oracle (``oracle.reference_forward``, itself checked against the
reference tests' vectors and a float64 dense closed form in
tests/test_oracle.py), on:

* the reference tests' golden attention cases (visibility start -> 25.0,
  fp16 single key == value; test_reference.py:114-139, 552-575);
* ragged GQA batches under the full, sliding-window and chunked-local specs
  (prefill chunks at offsets, decodes, a first-token prefill), with stale
  values everywhere the batch must not read;
* a shared prefix: two requests whose block tables start with the same
  physical blocks (test_reference.py:923-968);
* a graph-padded batch: slot -1 writes nothing, tokens outside every request
  come back zero (model_runner.py:78-122).

The bar: the cache after the write is bit-identical to the oracle's, and the
fp32 outputs agree to 1e-6 (fp16/bf16 outputs to one unit in the last place).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from _golden import GOLDEN, batch_from_case, cache_from_case

torch = pytest.importorskip("torch")

from _torch_reference import TorchReferenceAttention  # noqa: E402
from micro_vllm_amd.attention import AttentionMetadata  # noqa: E402

TORCH_DTYPE = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def _bits(t):
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _metadata(batch: oracle.Batch) -> AttentionMetadata:
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int64))  # noqa: E731
    return AttentionMetadata(
        query_positions=t(batch.query_positions),
        query_context_start_positions=t(batch.query_context_start_positions),
        query_start_locations=t(batch.query_start_locations),
        context_lengths=t(batch.context_lengths),
        block_table=t(batch.block_table),
        slot_mapping=t(batch.slot_mapping),
        block_size=batch.block_size,
    )


def run_both(q, k, v, cache, batch):
    """(checker cache, checker output, oracle cache, oracle fp32 output) on
    the same inputs; ``cache`` is a torch tensor that is not modified."""

    ref_cache = cache.clone()
    out = TorchReferenceAttention()(q, k, v, ref_cache, _metadata(batch))
    # The write in storage bits (bf16 as uint16), then fp32 attention over
    # the written cache.
    o_cache = _bits(cache).copy()
    oracle.write_kv_cache(_bits(k), _bits(v), o_cache, batch.slot_mapping)
    expected = oracle.reference_forward(
        oracle.to_f32(_bits(q)), oracle.to_f32(_bits(k)), oracle.to_f32(_bits(v)), oracle.to_f32(o_cache), batch
    )
    return ref_cache, out, o_cache, expected


def assert_matches_oracle(q, k, v, cache, batch):
    ref_cache, out, o_cache, expected = run_both(q, k, v, cache, batch)
    # Bit-identical cache, NaN sentinels included.
    got_cache = _bits(ref_cache)
    view = np.uint32 if got_cache.dtype == np.float32 else np.uint16
    assert np.array_equal(got_cache.view(view), o_cache.view(view))
    assert out.shape == q.shape and out.dtype == q.dtype
    got = out.float().numpy()
    if q.dtype == torch.float32:
        np.testing.assert_allclose(got, expected, atol=1e-6, rtol=1e-6)
    else:
        # The fp32 results may round to neighbouring 16-bit values.
        ulp = 2.0**-10 if q.dtype == torch.float16 else 2.0**-7
        np.testing.assert_allclose(got, expected, atol=1e-6, rtol=ulp)
    return out


@pytest.mark.parametrize("c", GOLDEN["attention_cases"], ids=lambda c: c["name"])
def test_checker_matches_the_golden_attention_cases(c):
    dtype = TORCH_DTYPE[c["dtype"]]
    np_dtype = np.float16 if c["dtype"] == "float16" else np.float32
    cache = torch.from_numpy(cache_from_case(c, np_dtype))
    batch = batch_from_case(c)
    t = lambda x: torch.tensor(x, dtype=dtype)  # noqa: E731
    out = assert_matches_oracle(t(c["query"]), t(c["key"]), t(c["value"]), cache, batch)
    np.testing.assert_allclose(out.double().numpy(), np.array(c["expect_output"]), atol=c["tolerance"], rtol=0)


def ragged_case(seed, lengths, qlens, hq, hkv, d, bs, spec, dtype):
    """Requests whose blocks come from a shuffled pool; request r's new tokens
    end at position lengths[r] - 1. The cache holds random stale values in
    every slot (history included), so the write and the gather are both
    exercised."""

    rng = np.random.default_rng(seed)
    need = [-(-L // bs) for L in lengths]
    pool = rng.permutation(sum(need) + 3)
    tables, cursor = [], 0
    for n in need:
        tables.append(pool[cursor : cursor + n].tolist())
        cursor += n
    num_blocks = len(pool) + 1
    positions = [list(range(L - q, L)) for L, q in zip(lengths, qlens)]
    batch = oracle.make_batch(positions, tables, block_size=bs, null_block_id=num_blocks - 1, spec=spec)
    gen = torch.Generator().manual_seed(seed)
    n = sum(qlens)
    q, k, v = (torch.randn((n, h, d), generator=gen).to(dtype) for h in (hq, hkv, hkv))
    cache = torch.randn((2, num_blocks, bs, hkv, d), generator=gen).to(dtype)
    return q, k, v, cache, batch


SPECS = [(oracle.FULL, 0), (oracle.SLIDING_WINDOW, 5), (oracle.SLIDING_WINDOW, 33), (oracle.CHUNKED_LOCAL, 8)]


@pytest.mark.parametrize("spec", SPECS, ids=["full", "window5", "window33", "chunked8"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_checker_matches_oracle_on_ragged_gqa_batches(spec, dtype):
    """A 40-token chunk at offset 20, two decodes, a 3-token chunk, a
    first-token prefill; 16 q / 4 KV heads (group 4), head_dim 32, block 4."""

    q, k, v, cache, batch = ragged_case(
        7, [60, 9, 33, 5, 1], [40, 1, 1, 3, 1], 16, 4, 32, 4, spec, TORCH_DTYPE[dtype]
    )
    assert_matches_oracle(q, k, v, cache, batch)


def test_checker_matches_oracle_with_a_shared_prefix():
    """Two requests share their first three blocks (a 12-token prefix) and
    continue through their own blocks: one with a 6-token chunk, one with a
    decode; a third request shares only the first block."""

    rng = np.random.default_rng(11)
    hq, hkv, d, bs = 8, 2, 16, 4
    shared = [5, 0, 7]
    tables = [shared + [2, 9], shared + [4], shared[:1] + [1, 8]]
    positions = [list(range(14, 20)), [15], list(range(9, 12))]
    num_blocks = 11
    batch = oracle.make_batch(positions, tables, block_size=bs, null_block_id=num_blocks - 1)
    gen = torch.Generator().manual_seed(11)
    n = sum(len(p) for p in positions)
    q, k, v = (torch.randn((n, h, d), generator=gen) for h in (hq, hkv, hkv))
    cache = torch.from_numpy(rng.standard_normal((2, num_blocks, bs, hkv, d)).astype(np.float32))
    ref_cache, out, _, _ = run_both(q, k, v, cache, batch)
    assert_matches_oracle(q, k, v, cache, batch)
    # The shared blocks before position 12 were not written.
    assert torch.equal(ref_cache[:, shared], cache[:, shared])


def test_checker_matches_oracle_on_a_graph_padded_batch():
    """Graph padding (model_runner.py:78-122): two real requests, then a
    padded request with context length 0 and a padded token whose slot is
    -1. The padded token's output is zero and its slot writes nothing."""

    hq, hkv, d, bs = 4, 2, 8, 4
    gen = torch.Generator().manual_seed(13)
    q, k, v = (torch.randn((5, h, d), generator=gen) for h in (hq, hkv, hkv))
    cache = torch.randn((2, 6, bs, hkv, d), generator=gen)
    batch = oracle.Batch(
        query_positions=np.array([4, 5, 6, 2, 0]),
        query_context_start_positions=np.zeros(5, np.int64),
        query_start_locations=np.array([0, 3, 4, 4]),
        context_lengths=np.array([7, 3, 0]),
        block_table=np.array([[3, 1], [4, 5], [5, 5]]),
        slot_mapping=np.array([4, 5, 6, 18, -1]),  # block 1 rows 0-2, block 4 row 2
        block_size=bs,
    )
    ref_cache, out, _, _ = run_both(q, k, v, cache, batch)
    assert_matches_oracle(q, k, v, cache, batch)
    assert not out[4].any()
    assert torch.equal(ref_cache[:, 0], cache[:, 0]) and torch.equal(ref_cache[:, 2], cache[:, 2])
