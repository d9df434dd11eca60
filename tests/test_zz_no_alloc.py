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
import subprocess
import sys
import textwrap
from pathlib import Path

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


def noalloc_args(w, cache, out):
    batch, keep = batch_descriptor(w.metadata, w.query.device)
    args = (
        _native.tensor3(w.query),
        _native.tensor3(w.key),
        _native.tensor3(w.value),
        _native.kv_cache(cache),
        batch,
        _native.tensor3(out),
        1.0 / math.sqrt(w.head_dim),
    )
    return args, keep


def test_noalloc_entry_point_captured_in_a_graph_replays_bit_exact(device):
    """After a warm call on the device, the allocation-free forward captures
    into a HIP graph; every replay (eager work between them) gives the eager
    call's output and cache bit for bit."""

    lib = _native.load()
    w = mixed_batch(device, chunks=2, chunk_tokens=200, decodes=40, decode_range=(16, 3000), seed=33, hint=True)
    eager_cache = w.cache.clone()
    eager_out = torch.full_like(w.query, float("nan"))
    args, keep = noalloc_args(w, eager_cache, eager_out)
    _native.check(lib.mvllm_attention_forward_noalloc(*args, _native.stream_handle(device)), "noalloc eager")
    torch.cuda.synchronize()
    assert not torch.isnan(eager_out).any()

    graph_cache = w.cache.clone()
    graph_out = torch.full_like(w.query, float("nan"))
    gargs, gkeep = noalloc_args(w, graph_cache, graph_out)
    graph = torch.cuda.CUDAGraph()
    statuses = []
    with torch.cuda.graph(graph):
        statuses.append(lib.mvllm_attention_forward_noalloc(*gargs, _native.stream_handle(device)))
    assert statuses == [0], lib.mvllm_last_error()
    for _ in range(3):
        graph_cache.copy_(w.cache)
        graph_out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out.view(torch.int16), eager_out.view(torch.int16))
        assert torch.equal(graph_cache.view(torch.int16), eager_cache.view(torch.int16))
        _ = (w.query.float() * 2).sum().item()  # eager work between replays
    del keep, gkeep


FIRST_CALL_UNDER_CAPTURE = textwrap.dedent(
    """
    import math, sys
    sys.path[:0] = [sys.argv[1], sys.argv[1] + "/micro-vllm_amd", sys.argv[1] + "/tests"]
    import torch
    from micro_vllm_amd import _native, workloads
    from micro_vllm_amd.attention.operators.mi355x_paged import batch_descriptor
    lib = _native.load()
    dev = torch.device("cuda", 0)
    w = workloads.small_mixed(dev, dtype=torch.bfloat16)
    out = torch.zeros_like(w.query)
    batch, keep = batch_descriptor(w.metadata, dev)
    args = (_native.tensor3(w.query), _native.tensor3(w.key), _native.tensor3(w.value),
            _native.kv_cache(w.cache), batch, _native.tensor3(out), 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        first = lib.mvllm_attention_forward_noalloc(*args, _native.stream_handle(dev))
    print("first", first, (lib.mvllm_last_error() or b"").decode(), flush=True)
    warm = lib.mvllm_attention_forward_noalloc(*args, _native.stream_handle(dev))
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        captured = lib.mvllm_attention_forward_noalloc(*args, _native.stream_handle(dev))
    g2.replay()
    torch.cuda.synchronize()
    print("warm", warm, "captured", captured, "finite", bool(torch.isfinite(out).all()), flush=True)
    """
)


def test_noalloc_first_call_under_capture_is_refused_then_capture_works(device):
    """In a fresh process, the first allocation-free call on the device made
    under stream capture is refused with MVLLM_ERR_INVALID (its workspace
    lookup stays out of the capture); after one call outside capture the
    same call captures and replays."""

    root = Path(__file__).resolve().parents[1]
    result = subprocess.run(
        [sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE, str(root)],
        capture_output=True, text=True, timeout=300,
    )
    print(result.stdout, result.stderr[-2000:])
    assert result.returncode == 0
    lines = dict(line.split(" ", 1) for line in result.stdout.splitlines() if " " in line)
    first = lines["first"].split(" ", 1)
    assert int(first[0]) == _native.ERR_INVALID and "under stream capture" in first[1]
    assert lines["warm"].split() == ["0", "captured", "0", "finite", "True"]

