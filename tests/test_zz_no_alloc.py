"""GPU parity of the allocation-free entry point.

``mvllm_attention_forward_noalloc`` takes its workspace from a library-owned
device array instead of a caller argument. Called through the C ABI, it must
give the same cache and the same output as ``mvllm_attention_forward`` with
a caller workspace (the same kernels over the same work lists: bit for bit),
on two calls in a row, the second with a smaller batch, so that whatever the
first call left in the array cannot leak into the second.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import pytest
import torch

from micro_vllm_amd import _native, workloads
from micro_vllm_amd.attention.operators.mi355x_paged import batch_descriptor

pytestmark = pytest.mark.gpu


def mixed_batch(device, *, chunks, chunk_tokens, decodes, decode_range, seed, hint):
    rng = np.random.default_rng(seed)
    offsets = rng.integers(0, 1024, size=chunks)
    decode_lengths = rng.integers(decode_range[0], decode_range[1] + 1, size=decodes)
    lengths = np.concatenate([offsets + chunk_tokens, decode_lengths])
    queries = np.concatenate([np.full(chunks, chunk_tokens), np.ones(decodes, dtype=np.int64)])
    needed = int(((lengths + 15) // 16).sum())
    w = workloads.build(
        f"noalloc_{seed}",
        context_lengths=lengths,
        query_lengths=queries,
        num_q_heads=32,
        num_kv_heads=8,
        head_dim=128,
        block_size=16,
        pool_blocks=needed + 64,
        dtype=torch.bfloat16,
        value_scale=1.0,
        seed=seed,
        device=device,
        rng=rng,
    )
    if not hint:
        w.metadata = dataclasses.replace(w.metadata, max_query_len=None)
    return w


def run(w, cache, noalloc):
    lib = _native.load()
    device = w.query.device
    batch, keep = batch_descriptor(w.metadata, device)
    out = torch.full_like(w.query, float("nan"))
    args = (
        _native.tensor3(w.query),
        _native.tensor3(w.key),
        _native.tensor3(w.value),
        _native.kv_cache(cache),
        batch,
        _native.tensor3(out),
        1.0 / math.sqrt(w.head_dim),
    )
    stream = _native.stream_handle(device)
    need = lib.mvllm_attention_workspace_bytes(batch, w.num_q_heads, w.head_dim)
    assert 0 < need <= _native.NOALLOC_SCRATCH_BYTES
    print(f"  {'noalloc' if noalloc else 'workspace'}: {w.name}, {w.query.shape[0]} tokens, "
          f"{len(w.context_lengths)} requests, workspace {need} B", flush=True)
    if noalloc:
        status = lib.mvllm_attention_forward_noalloc(*args, stream)
        _native.check(status, "mvllm_attention_forward_noalloc")
    else:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
        status = lib.mvllm_attention_forward(*args, workspace.data_ptr(), need, stream)
        _native.check(status, "mvllm_attention_forward")
    torch.cuda.synchronize()
    del keep
    return out


def test_noalloc_entry_point_matches_the_workspace_entry_point(device):
    calls = [
        # 4 prefill chunks beside 120 decodes (the prefill kernel on the
        # caller's stream), then a smaller batch without the hint.
        dict(chunks=4, chunk_tokens=384, decodes=120, decode_range=(64, 6000), seed=31, hint=True),
        dict(chunks=1, chunk_tokens=100, decodes=30, decode_range=(16, 900), seed=32, hint=False),
    ]
    for spec in calls:
        w = mixed_batch(device, **spec)
        cache_ref = w.cache.clone()
        cache_new = w.cache.clone()
        ref = run(w, cache_ref, noalloc=False)
        got = run(w, cache_new, noalloc=True)
        assert torch.equal(cache_new.view(torch.int16), cache_ref.view(torch.int16))
        assert not torch.isnan(ref).any()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
        del w, cache_ref, cache_new
