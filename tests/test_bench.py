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


def test_more_than_one_gpu_is_refused_with_a_message():
    result = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
        capture_output=True,
        text=True,
        timeout=120,
    )
    assert result.returncode == 2
    assert "one GPU" in result.stderr
