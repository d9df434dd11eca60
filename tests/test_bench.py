"""Host-side checks of the benchmark harness (no GPU needed)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_committed_traffic_summaries_parse():
    for workload in ("qwen3_decode", "llama3_mixed"):
        traffic = bench.measured_traffic(workload)
        assert isinstance(traffic, int) and traffic > 10**9, workload
    assert bench.measured_traffic("unknown") is None


def test_decode_kernel_bytes_counts_every_visible_row_once():
    # Two sequences of 17 and 32 tokens, one query each, 2 KV heads x 4 dims
    # in bf16, 4 query heads, block 16.
    w = SimpleNamespace(
        query=SimpleNamespace(element_size=lambda: 2),
        context_lengths=np.array([17, 32]),
        query_lengths=np.array([1, 1]),
        num_kv_heads=2,
        num_q_heads=4,
        head_dim=4,
        block_size=16,
    )
    kv = (17 + 32) * 2 * 4 * 2 * 2
    qo = 2 * 2 * 4 * 4 * 2
    table = (2 + 2) * 8
    meta = 2 * 8 * 2 + 8 + 2 * 8 * 2
    assert bench.decode_kernel_bytes(w) == kv + qo + table + meta


def test_step_roofline_takes_the_larger_floor():
    # One decode of 1,000 tokens and one 100-token prefill chunk at offset
    # 400: 2 KV heads x 4 dims in bf16, 4 query heads, block 16.
    w = SimpleNamespace(
        query=SimpleNamespace(element_size=lambda: 2),
        context_lengths=np.array([1000, 500]),
        query_lengths=np.array([1, 100]),
        num_kv_heads=2,
        num_q_heads=4,
        head_dim=4,
        block_size=16,
    )
    sys.path.insert(0, str(ROOT / "micro-vllm_amd"))
    from micro_vllm_amd import workloads

    flops = 4 * 4 * 4 * (100 * 400 + 100 * 101 // 2)
    assert workloads.prefill_flops(w) == flops
    step_bytes = workloads.decode_bytes(w)
    hbm_ms = step_bytes / 8e12 * 1e3
    mfma_ms = flops / 2.5e15 * 1e3
    r = bench.step_roofline(w, 2 * max(hbm_ms, mfma_ms))
    assert r["bound"] == ("hbm" if hbm_ms >= mfma_ms else "mfma")
    assert abs(r["floor_ms"] - max(hbm_ms, mfma_ms)) < 1e-5
    assert r["frac"] == 0.5


def test_more_than_one_gpu_is_refused_with_a_message():
    result = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
        capture_output=True,
        text=True,
        timeout=120,
    )
    assert result.returncode == 2
    assert "one GPU" in result.stderr


def _oracle_case(dtype):
    import torch

    sys.path.insert(0, str(ROOT / "micro-vllm_amd"))
    from micro_vllm_amd import workloads

    from _oracle_bridge import oracle_step, to_oracle

    w = workloads.small_mixed("cpu", dtype=dtype)
    want_cache, want = oracle_step(w.query, w.key, w.value, w.cache, w.metadata)
    got = bench.torch_gathered_attention(w.query, w.key, w.value, w.cache, w.metadata, 1.0 / np.sqrt(128))
    return w, got, want, want_cache, to_oracle


def test_torch_baseline_matches_the_oracle_fp32():
    w, got, want, want_cache, to_oracle = _oracle_case(__import__("torch").float32)
    assert np.array_equal(to_oracle(w.cache), want_cache)  # the write is bit-exact
    np.testing.assert_allclose(got.numpy(), want, atol=2e-5, rtol=1e-5)


def test_torch_baseline_matches_the_oracle_bf16():
    import torch

    w, got, want, want_cache, to_oracle = _oracle_case(torch.bfloat16)
    assert np.array_equal(to_oracle(w.cache), want_cache)
    # bf16 products (inputs rounded as the oracle's are) and bf16 output.
    np.testing.assert_allclose(got.float().numpy(), want, atol=2e-2, rtol=1e-2)


def test_torch_baseline_leaves_tokens_outside_requests_zero_and_empty_rows_nan():
    import torch

    sys.path.insert(0, str(ROOT / "micro-vllm_amd"))
    from micro_vllm_amd import workloads

    w = workloads.small_mixed("cpu", dtype=torch.float32)
    md = w.metadata
    # Drop the last request from the batch: its token is outside every request.
    md2 = type(md)(
        query_positions=md.query_positions,
        query_context_start_positions=md.query_context_start_positions.clone(),
        query_start_locations=md.query_start_locations[:-1].clone(),
        context_lengths=md.context_lengths[:-1].clone(),
        block_table=md.block_table[:-1].clone(),
        slot_mapping=md.slot_mapping,
        block_size=md.block_size,
        max_query_len=md.max_query_len,
    )
    # Request 1 (a decode at position 63): its visible range starts past its position.
    md2.query_context_start_positions[17] = 64
    out = bench.torch_gathered_attention(w.query, w.key, w.value, w.cache, md2, 1.0 / np.sqrt(128))
    assert torch.all(out[-1] == 0)
    assert torch.isnan(out[17]).all()
    assert torch.isfinite(out[18]).all()


def test_cpu_baseline_runs_the_reference_cpu_path_on_every_host_thread():
    import torch

    sys.path.insert(0, str(ROOT / "micro-vllm_amd"))
    from micro_vllm_amd import workloads

    w = workloads.small_mixed("cpu", dtype=torch.bfloat16)
    before = w.cache.clone()
    r = bench.cpu_baseline(w, sample_requests=4, repeats=2, warmups=1)
    assert r["kind"] == "port" and r["unit"] == "GB/s" and r["value"] > 0
    assert r["cores"] == bench.host_threads() >= 1
    assert "4 of 4 sequences" in r["sample"] and r["cpu_model"]
    assert torch.equal(w.cache, before)  # the baseline works on a host copy


def test_cpu_prefill_baseline_times_only_the_prefill_chunks():
    import torch

    sys.path.insert(0, str(ROOT / "micro-vllm_amd"))
    from micro_vllm_amd import workloads

    w = workloads.small_mixed("cpu", dtype=torch.bfloat16)
    r = bench.cpu_prefill_baseline(w, repeats=2, warmups=1)
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s" and r["value"] > 0
    assert "all 1 prefill chunks (17 queries" in r["sample"]
    # 17 causal queries from position 0: 17 * 18 / 2 visible pairs, 4 * Hq * D flops each.
    assert f"{4 * 16 * 128 * 153 / 1e9:.1f} GFLOP" in r["sample"]
