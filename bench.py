"""Benchmark of the ragged paged-attention path on one MI355X.

A step is one pass of the hot path over one synthetic batch: the
``mi355x_paged`` operator's forward (KV-cache write + split-KV decode +
combine; + MFMA prefill for multi-query requests). The default workload is
the Qwen3-0.6B-head decode batch: 256 sequences, contexts U[128, 4096]
(seed 0), 16 query / 8 KV heads, head_dim 128, block 16, bf16, blocks drawn
from a shuffled 70,000-block pool, values N(0,1)*0.5.

Each timed measurement first runs untimed forwards for ``--settle-ms`` of wall
time, then its ``--warmup`` untimed steps, then ``--steps`` timed ones: a GPU
that was idle runs its first ~50 back-to-back forwards up to 3-4% slower
while its clock ramps (``settle`` in the line records how many ran).

Reported (one JSON line on stdout):
* ``value``: algorithmic HBM bytes of the step / step time, in GB/s;
* ``roofline``: the decode kernel's algorithmic bytes per launch / its mean
  duration measured with HIP events recorded around its launch, against
  the 8 TB/s HBM peak;
* ``prefill``: the prefill kernel on the Llama-3-head mixed batch (8 chunks
  of 512 + 248 decodes): causal-visible FLOPs / its mean duration, against
  the 2.5 PFLOP/s bf16 peak (serial pass), and the mixed step's time with
  the decode and prefill workgroups in one step kernel, also as a fraction
  of its floor max(step bytes / HBM peak, prefill FLOPs / bf16 peak)
  (``prefill.mixed_step_roofline``); ``prefill.fp16`` times the prefill
  kernel on the same batch in fp16, the reference Triton backend's dtype;
  ``prefill.library`` times the same chunks through PyTorch-ROCm's flash
  attention (variable-length, one launch) and a square bf16 GEMM through
  hipBLASLt on the same GPU;
* ``kv_write``: the KV-cache write alone (one copy kernel) over the mixed
  batch's tokens: K/V bytes read and written / its mean duration, against the
  8 TB/s HBM peak (the shipped forward fuses the copy into its prologue);
* ``e2e``: Qwen3-0.6B-shaped end-to-end output tok/s, synchronized steps
  summed (the reference's method) and, as ``value_pipelined``, with the host
  one graph step ahead;
* ``e2e_llama3``: Llama-3-8B-shaped end-to-end output tok/s (64 requests
  sharing a 4,096-token prefix through the prefix cache, suffixes
  U[4096, 28672], 512 greedy tokens each, ~200 GB KV cache), synchronized
  steps summed, with the prefix-cache hit tokens and preemptions;
* ``config1``: the reference's CPU-runnable case (contexts [17, 64, 130,
  255]) through the HIP forward (fp32 and bf16) and the reference
  operator's CPU path;
* ``prefill.cpu_baseline``: the mixed batch's prefill chunks through the
  reference operator's CPU path, in TFLOP/s;
* ``gpu_baseline``: the same step in plain torch (block-table gather and
  matmuls) timed on the same GPU, and the HIP path's speedup over it;
* ``cpu_baseline``: the reference operator's CPU path (torch, bf16 cache,
  fp32 math, every available host core) on the same batch.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--settle-ms 150] [--workload qwen3_decode] [--quick]

Other workloads: ``llama3_mixed``, ``llama3_long_decode``, ``llama3_long_prefill``
(8 chunks of 512 at offsets U[14336, 16384]), ``llama3_causal_prefill`` (8
causal chunks of 4,096 from position 0) (attention steps),
``qwen3_e2e`` and ``llama3_e2e`` (end-to-end generation; the Llama-3-8B one
shares a 4,096-token prefix through the prefix cache and holds a ~200 GB KV
cache), and ``small_mixed`` (the ``config1`` record alone).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "micro-vllm_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "decode paged-attn HBM GB/s (% peak); e2e output tok/s, Qwen3-0.6B bf16"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PREFILL_WORKLOADS = ("llama3_mixed", "llama3_long_prefill", "llama3_causal_prefill")


class HipEvents:
    """hipEvent_t handles through the HIP runtime torch has loaded."""

    def __init__(self):
        import torch

        lib_dir = Path(torch.__file__).resolve().parent / "lib"
        candidates = [lib_dir / "libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so"]
        for name in candidates:
            try:
                self.hip = ctypes.CDLL(str(name))
                break
            except OSError:
                continue
        else:
            raise RuntimeError("cannot locate the HIP runtime library")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, count: int) -> list[int]:
        events = []
        for _ in range(count):
            handle = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(handle)) != 0:
                raise RuntimeError("hipEventCreate failed")
            events.append(handle.value)
        return events

    def elapsed_ms(self, start: int, stop: int) -> float:
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(start), ctypes.c_void_p(stop)) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, events: list[int]) -> None:
        for e in events:
            self.hip.hipEventDestroy(ctypes.c_void_p(e))


def decode_kernel_bytes(w) -> int:
    """Algorithmic bytes one decode-kernel launch must move: every visible
    K and V row once, Q read, O written, the block-table entries walked and
    the per-request metadata."""

    es = w.query.element_size()
    rows = int(w.context_lengths.sum())
    kv = rows * w.num_kv_heads * w.head_dim * 2 * es
    n = int(w.query_lengths.sum())
    qo = 2 * n * w.num_q_heads * w.head_dim * es
    table = int(((w.context_lengths + w.block_size - 1) // w.block_size).sum()) * 8
    meta = len(w.context_lengths) * 8 * 2 + 8 + n * 8 * 2
    return kv + qo + table + meta


TRAFFIC_PROFILES = {
    "qwen3_decode": ROOT / "profiles" / "decode_qwen3_256seq_traffic.md",
    "llama3_mixed": ROOT / "profiles" / "decode_llama3_mixed_traffic.md",
    "llama3_long_decode": ROOT / "profiles" / "decode_llama3_long_kernel_stats.md",
}


def measured_traffic(workload: str) -> int | None:
    """HBM bytes per decode-kernel launch on this workload, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (each counter scaled by what it
    reads for a plain elementwise kernel of known traffic); None if absent."""

    path = TRAFFIC_PROFILES.get(workload)
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def host_threads() -> int:
    """Host threads for the CPU baseline: every core this process may use,
    capped by OMP_NUM_THREADS when it is set (this process's CPU share)."""

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        cores = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        cores = min(cores, int(env))
    return max(1, cores)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_forward_seconds(w, chosen, repeats: int, warmups: int = 2) -> tuple[float, int]:
    """Median seconds of the reference operator's CPU path
    (``oracle.reference_cpu``: the steps of reference.py:14-138 in torch,
    the workload's cache dtype, fp32 math) over the requests ``chosen`` of
    the batch, on every host core this process may use: their blocks are
    copied into a compact host cache and the step's own K/V rows are written
    by the forward. Returns (seconds, threads)."""

    import numpy as np
    import torch

    from oracle import reference_cpu

    threads = host_threads()
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        blocks = [w.block_lists[r] for r in chosen]
        ids = np.concatenate(blocks)
        compact = w.cache[:, torch.as_tensor(ids, device=w.cache.device)].cpu()
        cache = torch.cat([compact, torch.zeros_like(compact[:, :1])], dim=1)
        null = len(ids)
        width = max(len(b) for b in blocks)
        table = torch.full((len(chosen), width), null, dtype=torch.int64)
        cursor = 0
        positions, qsl, lengths = [], [0], []
        for i, (r, b) in enumerate(zip(chosen, blocks)):
            table[i, : len(b)] = torch.arange(cursor, cursor + len(b))
            cursor += len(b)
            L, q = int(w.context_lengths[r]), int(w.query_lengths[r])
            positions.extend(range(L - q, L))
            qsl.append(qsl[-1] + q)
            lengths.append(L)
        pos = torch.tensor(positions, dtype=torch.int64)
        starts = torch.zeros_like(pos)
        req = torch.repeat_interleave(torch.arange(len(chosen)), torch.tensor(np.diff(qsl)))
        slots = table[req, pos // w.block_size] * w.block_size + pos % w.block_size
        full_qsl = w.metadata.query_start_locations.cpu().numpy()
        rows = np.concatenate([np.arange(full_qsl[r], full_qsl[r + 1]) for r in chosen])
        rows_t = torch.as_tensor(rows, device=w.query.device)
        q, k, v = (t[rows_t].cpu() for t in (w.query, w.key, w.value))
        qsl_t, len_t = torch.tensor(qsl, dtype=torch.int64), torch.tensor(lengths, dtype=torch.int64)

        def run():
            start = time.perf_counter()
            reference_cpu.reference_forward(q, k, v, cache, pos, starts, qsl_t, len_t, table, slots, w.block_size)
            return time.perf_counter() - start

        for _ in range(warmups):
            run()
        times = [run() for _ in range(repeats)]
    finally:
        torch.set_num_threads(previous)
    return statistics.median(times), threads


def cpu_baseline(w, sample_requests: int, repeats: int, warmups: int = 2) -> dict:
    """The reference operator's CPU path on ``sample_requests`` sequences of
    a decode batch (evenly spaced), as HBM-equivalent GB/s: the same
    algorithmic bytes the GPU step is credited with, over the CPU time."""

    import numpy as np

    order = np.arange(len(w.context_lengths))
    step = max(1, len(order) // sample_requests)
    chosen = order[::step][:sample_requests]
    seconds, threads = cpu_forward_seconds(w, chosen, repeats, warmups)
    sample_bytes = _subset_bytes(w, chosen)
    return {
        "value": round(sample_bytes / seconds / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": (
            f"{len(chosen)} of {len(w.context_lengths)} sequences "
            f"({int(w.context_lengths[chosen].sum())} context tokens) through the reference operator's CPU path "
            f"(torch, {threads} threads, bf16 cache, fp32 math), median of {repeats} runs after {warmups}: "
            f"{seconds:.3f} s per forward"
        ),
    }


def cpu_prefill_baseline(w, repeats: int = 3, warmups: int = 1) -> dict:
    """The reference operator's CPU path on the batch's multi-query requests
    (the prefill chunks), as TFLOP/s over the same causal-visible FLOPs the
    GPU prefill kernel is credited with."""

    import numpy as np

    from micro_vllm_amd import workloads

    chosen = np.nonzero(w.query_lengths > 1)[0]
    seconds, threads = cpu_forward_seconds(w, chosen, repeats, warmups)
    flops = workloads.prefill_flops(w)
    return {
        "value": round(flops / seconds / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": (
            f"all {len(chosen)} prefill chunks ({int(w.query_lengths[chosen].sum())} queries, "
            f"{flops / 1e9:.1f} GFLOP causal-visible) through the reference operator's CPU path "
            f"(torch, {threads} threads, bf16 cache, fp32 math), median of {repeats} runs after {warmups}: "
            f"{seconds:.3f} s per forward"
        ),
    }


def small_mixed_record(hip: "HipEvents", device, steps: int = 200, warmup: int = 20) -> dict:
    """The reference's CPU-runnable case on both sides: contexts
    [17, 64, 130, 255] (a 17-token prefill and three decodes), 16 q / 8 KV
    heads, head_dim 128, block 16, seed 0. The HIP forward is timed between
    HIP events (mean over ``steps`` launches) in fp32 (the any-shape kernel)
    and bf16 (the step kernel); the reference operator's CPU path in fp32 on
    every host core (median of 7 runs after 3)."""

    import numpy as np
    import torch

    from micro_vllm_amd import workloads
    from micro_vllm_amd.attention.operators.mi355x_paged import hip_paged_attention

    hip.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    stream = torch.cuda.current_stream(device).cuda_stream
    record = {
        "workload": (
            "small_mixed: contexts [17, 64, 130, 255] (one 17-token prefill + 3 decodes), 16 q / 8 kv heads, "
            "head_dim 128, block 16, 64-block pool, seed 0"
        )
    }
    for dtype, name in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        w = workloads.small_mixed(device, dtype=dtype)
        events = hip.create(2)
        for _ in range(warmup):
            hip_paged_attention(w.query, w.key, w.value, w.cache, w.metadata)
        torch.cuda.synchronize()
        hip.hip.hipEventRecord(ctypes.c_void_p(events[0]), ctypes.c_void_p(stream))
        for _ in range(steps):
            hip_paged_attention(w.query, w.key, w.value, w.cache, w.metadata)
        hip.hip.hipEventRecord(ctypes.c_void_p(events[1]), ctypes.c_void_p(stream))
        torch.cuda.synchronize()
        record[f"hip_us_{name}"] = round(hip.elapsed_ms(events[0], events[1]) * 1e3 / steps, 2)
        hip.destroy(events)
        if dtype == torch.float32:
            seconds, threads = cpu_forward_seconds(w, np.arange(4), repeats=7, warmups=3)
            record["cpu_baseline"] = {
                "us": round(seconds * 1e6, 1),
                "cores": threads,
                "kind": "port",
                "cpu_model": cpu_model(),
                "sample": f"the whole batch through the reference operator's CPU path (torch, {threads} threads, fp32), "
                "median of 7 runs after 3",
            }
    record["note"] = "latency-bound (20 query tokens); the HIP times include the forward's launches"
    return record


def torch_gathered_attention(query, key, value, cache, md, scale: float):
    """The operator's semantics in plain torch, as a baseline on the same GPU.

    Writes K/V into the cache (``index_copy_`` on the flat slot view, padded
    slots skipped), then per request gathers the keys of
    [context start of its first query, context length) through the block
    table and computes masked attention, as reference.py:14-138 does: key p
    is visible to query t when cstart(t) <= p <= pos(t). Products run as bf16
    (or input-dtype) ``matmul`` with the right operand made contiguous,
    softmax in fp32. Single-query requests are batched (padded to the longest
    context); multi-query requests run one at a time. Tokens outside every
    request stay zero; a row with no visible key is NaN, as in the reference.
    """

    import torch

    nb, bs, hkv, d = cache.shape[1:]
    flat = cache.view(2, nb * bs, hkv, d)
    slots = md.slot_mapping
    keep = slots >= 0
    idx = slots[keep]
    flat[0].index_copy_(0, idx, key[keep])
    flat[1].index_copy_(0, idx, value[keep])
    n, hq, _ = query.shape
    g = hq // hkv
    out = torch.zeros_like(query)
    qsl = md.query_start_locations.cpu()
    lengths = md.context_lengths.cpu()
    qlen = qsl[1:] - qsl[:-1]
    table = md.block_table
    dev = query.device

    def gather(rows: torch.Tensor, pos: torch.Tensor):
        # Slots of key positions pos[s, j] of requests rows[s]; invalid -> (0, masked).
        blk = table[rows[:, None], (pos // bs).clamp(max=table.shape[1] - 1)]
        ok = (blk >= 0) & (blk < nb)
        slot = torch.where(ok, blk * bs + pos % bs, torch.zeros_like(blk))
        return flat[0][slot], flat[1][slot], ok

    single = torch.nonzero(qlen == 1).flatten()
    if single.numel():
        rows = single.to(dev)
        tok = md.query_start_locations[rows]
        lmax = int(lengths[single].max())
        pos = torch.arange(lmax, device=dev)[None, :].expand(rows.numel(), lmax)
        kg, vg, ok = gather(rows, pos)
        vis = ok & (pos >= md.query_context_start_positions[tok][:, None]) & (pos <= md.query_positions[tok][:, None])
        vis &= pos < md.context_lengths[rows][:, None]
        q = query[tok].view(-1, hkv, g, d)
        kt = kg.permute(0, 2, 3, 1).contiguous()  # [S, Hkv, D, L]
        s = torch.matmul(q, kt).float() * scale    # [S, Hkv, G, L]
        s = s.masked_fill(~vis[:, None, None, :], float("-inf"))
        p = torch.softmax(s, dim=-1).to(query.dtype)
        o = torch.matmul(p, vg.permute(0, 2, 1, 3).contiguous())  # [S, Hkv, G, D]
        out[tok] = o.reshape(-1, hq, d)
    for r in torch.nonzero(qlen > 1).flatten().tolist():
        t0, t1, length = int(qsl[r]), int(qsl[r + 1]), int(lengths[r])
        first = int(md.query_context_start_positions[t0])
        pos = torch.arange(max(first, 0), length, device=dev)[None, :]
        rows = torch.tensor([r], device=dev)
        kg, vg, ok = gather(rows, pos)
        cst = md.query_context_start_positions[t0:t1][:, None]
        qp = md.query_positions[t0:t1][:, None]
        vis = ok & (pos >= cst) & (pos <= qp)  # [n, L]
        q = query[t0:t1].view(t1 - t0, hkv, g, d).permute(1, 2, 0, 3)  # [Hkv, G, n, D]
        kt = kg[0].permute(1, 2, 0).contiguous()  # [Hkv, D, L]
        s = torch.matmul(q, kt[:, None]).float() * scale  # [Hkv, G, n, L]
        s = s.masked_fill(~vis[None, None], float("-inf"))
        p = torch.softmax(s, dim=-1).to(query.dtype)
        o = torch.matmul(p, vg[0].permute(1, 0, 2).contiguous()[:, None])  # [Hkv, G, n, D]
        out[t0:t1] = o.permute(2, 0, 1, 3).reshape(t1 - t0, hq, d)
    return out


def torch_baseline(w, reference_out, steps: int = 5, warmup: int = 2) -> dict:
    """Time ``torch_gathered_attention`` on the same batch and GPU."""

    import math

    import torch

    from micro_vllm_amd import workloads

    scale = 1.0 / math.sqrt(w.head_dim)
    out = None
    for _ in range(warmup):
        out = torch_gathered_attention(w.query, w.key, w.value, w.cache, w.metadata, scale)
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        out = torch_gathered_attention(w.query, w.key, w.value, w.cache, w.metadata, scale)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - start) * 1e3 / steps
    diff = (out.float() - reference_out.float()).abs().nan_to_num(0.0).max().item()
    return {
        "value": round(workloads.decode_bytes(w) / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms, 4),
        "kind": "torch gathered attention (index_copy_ write, block-table gather, bf16 matmul, fp32 softmax)",
        "max_abs_diff_vs_hip": diff,
        "steps": steps,
    }


def library_prefill_baseline(w, hip_out, steps: int = 10, warmup: int = 3) -> dict:
    """The batch's prefill chunks through PyTorch-ROCm's flash attention on the
    same GPU, and a square bf16 GEMM through ``torch.matmul`` (hipBLASLt) as the
    library's own MFMA rate on this part, both timed between CUDA events on
    torch's stream (medians).

    The attention call is ``aten._flash_attention_forward`` in its
    variable-length form: one launch over every chunk, each chunk's queries
    against its whole context gathered into contiguous K/V (the gathers are
    outside the timed region), causal with the mask aligned to the end of the
    context (query i of a chunk of q tokens in a context of L sees keys
    0..L-q+i, the paged kernels' rule), GQA by head grouping. Its output is
    compared with the HIP path's."""

    import math

    import torch

    from micro_vllm_amd import workloads

    def median_ms(fn, warm: int) -> float:
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(steps):
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            fn()
            stop.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(stop))
        return statistics.median(times)

    out: dict = {}
    n = 8192
    a = torch.randn(n, n, device=w.query.device, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=w.query.device, dtype=torch.bfloat16)
    # Twenty untimed products first: the part's clock settles under a long MFMA load.
    ms = median_ms(lambda: torch.matmul(a, b), warm=20)
    gemm_tflops = 2 * n**3 / (ms * 1e-3) / 1e12
    out["gemm"] = {
        "kind": f"torch.matmul {n}x{n}x{n} bf16 (hipBLASLt)",
        "achieved": round(gemm_tflops, 1),
        "frac": round(gemm_tflops / BF16_PEAK_TFLOPS, 4),
    }
    del a, b

    md = w.metadata
    qsl = md.query_start_locations.tolist()
    rows_q, keys, values = [], [], []
    cum_q, cum_k = [0], [0]
    for r, (length, q) in enumerate(zip(w.context_lengths.tolist(), w.query_lengths.tolist())):
        if q <= 1:
            continue
        pos = torch.arange(length, device=w.query.device)
        blocks = md.block_table[r, pos // w.block_size]
        keys.append(w.cache[0, blocks, pos % w.block_size])
        values.append(w.cache[1, blocks, pos % w.block_size])
        rows_q.append((qsl[r], qsl[r + 1]))
        cum_q.append(cum_q[-1] + q)
        cum_k.append(cum_k[-1] + length)
    query = torch.cat([w.query[s:e] for s, e in rows_q]).contiguous()
    key = torch.cat(keys).contiguous()
    value = torch.cat(values).contiguous()
    del keys, values
    cq = torch.tensor(cum_q, dtype=torch.int32, device=w.query.device)
    ck = torch.tensor(cum_k, dtype=torch.int32, device=w.query.device)
    max_q = max(e - s for s, e in rows_q)
    max_k = max(cum_k[i + 1] - cum_k[i] for i in range(len(rows_q)))
    scale = 1.0 / math.sqrt(w.head_dim)

    def run():
        return torch.ops.aten._flash_attention_forward(
            query, key, value, cq, ck, max_q, max_k, 0.0, True, False, scale=scale
        )[0]

    try:
        result = run()
        ms = median_ms(run, warm=warmup)
    except (RuntimeError, AttributeError) as exc:  # no such operator in this torch build, or it refuses the shapes
        out["flash_attention"] = {"unavailable": str(exc)[:160]}
    else:
        mine = torch.cat([hip_out[s:e] for s, e in rows_q]).float()
        tflops = workloads.prefill_flops(w) / (ms * 1e-3) / 1e12
        out["flash_attention"] = {
            "kind": "torch aten._flash_attention_forward, variable-length, causal (end-aligned), GQA",
            "us": round(ms * 1e3, 1),
            "achieved": round(tflops, 1),
            "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "max_abs_diff_vs_hip": (result.float() - mine).abs().max().item(),
        }
    del query, key, value
    torch.cuda.empty_cache()
    return out


def _subset_bytes(w, chosen) -> int:
    es = w.query.element_size()
    L = w.context_lengths[chosen]
    n = int(w.query_lengths[chosen].sum())
    return int(L.sum()) * w.num_kv_heads * w.head_dim * 2 * es + 2 * n * w.num_q_heads * w.head_dim * es


E2E_CONFIGS = {
    # The Qwen3-0.6B end-to-end configuration: 256 random prompts U[64, 1024],
    # 256 greedy tokens each, 8,192-token budget, up to 256 sequences.
    "qwen3_e2e": dict(model="qwen3_0_6b", requests=256, prompt=(64, 1024), prefix=0, max_tokens=256,
                      max_num_seqs=256, prefix_cache=False, kv_bytes=None),
    # The Llama-3-8B end-to-end configuration: 64 requests sharing a
    # 4,096-token random prefix, each with its own suffix U[4096, 28672],
    # 512 greedy tokens each, KV cache of ~200 GB, prefix cache on.
    "llama3_e2e": dict(model="llama3_8b", requests=64, prompt=(4096, 28672), prefix=4096, max_tokens=512,
                       max_num_seqs=64, prefix_cache=True, kv_bytes=200e9),
}


def run_generation(device, workload: str, *, modes=("sync",), requests: int | None = None,
                   max_tokens: int | None = None, unfused: bool = False, seed: int = 0,
                   full_block_lists: bool = False) -> dict:
    """Greedy generation with a random-init decoder through the harness
    engine. ``modes``: "sync" times synchronized steps and sums them (the
    reference's method, benchmarks/benchmark_engine.py:305-315: each step is
    schedule + execute + synchronize + update); "pipelined" lets the host run
    one graph step ahead and times the loop's wall clock; "eager" runs sync
    without HIP graphs. Returns one record per mode."""

    import numpy as np
    import torch

    from micro_vllm_amd.attention.operators.registry import get_attention_operator_class
    from micro_vllm_amd.harness import DecoderConfig, DecoderModel, GenerationEngine, Request

    spec = dict(E2E_CONFIGS[workload])
    if requests is not None:
        spec["requests"] = requests
    if max_tokens is not None:
        spec["max_tokens"] = max_tokens
    cfg = getattr(DecoderConfig, spec["model"])()
    model = DecoderModel(cfg, get_attention_operator_class("mi355x_paged")(), device=device, seed=seed,
                         fused_layers=not unfused)
    rng = np.random.default_rng(seed)
    lo, hi = spec["prompt"]
    lengths = rng.integers(lo, hi + 1, size=spec["requests"])
    prefix = rng.integers(0, cfg.vocab_size, size=spec["prefix"]).tolist()
    prompts = [prefix + rng.integers(0, cfg.vocab_size, size=int(n)).tolist() for n in lengths]
    block_size = 16
    longest = spec["prefix"] + int(lengths.max()) + spec["max_tokens"]
    per_request = -(-longest // block_size)
    if spec["kv_bytes"] is not None:
        block_bytes = cfg.num_hidden_layers * 2 * block_size * cfg.num_key_value_heads * cfg.head_dim * 2
        num_blocks = int(spec["kv_bytes"] // block_bytes)
    else:
        num_blocks = per_request * spec["requests"] + 1
    max_model_len = per_request * block_size

    # Warm-up: a few short requests through a small engine (kernel loading, allocator).
    warm = GenerationEngine(model, num_blocks=4 * 8 + 1, max_num_batched_tokens=8192, max_num_seqs=256)
    warm.generate([Request(f"w{i}", prompts[i][:64], max_tokens=4) for i in range(min(4, len(prompts)))])
    del warm
    torch.cuda.synchronize(device)

    records = {}
    for mode in modes:
        engine = GenerationEngine(
            model,
            num_blocks=num_blocks,
            max_num_batched_tokens=8192,
            max_num_seqs=spec["max_num_seqs"],
            max_model_len=max_model_len,
            decode_graphs=mode != "eager",
            pipeline=mode == "pipelined",
            enable_prefix_cache=spec["prefix_cache"],
            cache_namespace=spec["model"],
            incremental_block_table=not full_block_lists,
        )
        if engine.graphs is not None:
            # Capture every bucket before timing (the reference captures at
            # start-up, model_runner.py:344-497).
            for size in engine.graphs.BUCKETS:
                if size <= spec["max_num_seqs"]:
                    engine.graphs.capture(size)
        print(f"[bench] {workload} {mode}: generating", file=sys.stderr, flush=True)
        result = engine.generate(
            [Request(f"r{i}", p, max_tokens=spec["max_tokens"]) for i, p in enumerate(prompts)], progress_seconds=20.0
        )
        records[mode] = {
            "output_tok_s": round(result.output_tokens_per_second, 2),
            "steps": result.steps,
            "step_seconds": round(result.step_seconds, 4),
            "timing": (
                "wall time of the generation loop (steps overlap)"
                if mode == "pipelined"
                else "synchronized steps summed"
            ),
            "decode_steps": result.decode_steps,
            "decode_step_ms": round(result.decode_seconds / max(result.decode_steps, 1) * 1e3, 3),
            "other_steps": result.steps - result.decode_steps,
            "other_step_ms": round(
                (result.step_seconds - result.decode_seconds) / max(result.steps - result.decode_steps, 1) * 1e3, 3
            ),
            "preemptions": result.preemptions,
            "prefix_hit_tokens": result.prefix_hit_tokens,
            "host_pack_ms_per_step": round(result.pack_seconds / max(result.steps, 1) * 1e3, 4),
            # Synchronous decode steps on the engine's fast path, and their
            # host phases per step: schedule (the step's arrays and blocks),
            # pack (payload copy + pack launch), replay (graph launch and the
            # tokens' copy issued), overlap (bookkeeping while the GPU runs),
            # wait (until the step's tokens are on the host), append.
            "fast_decode_steps": result.fast_decode_steps,
            "fast_phase_ms": {
                k: round(v / max(result.fast_decode_steps, 1) * 1e3, 4) for k, v in result.fast_phase_seconds.items()
            },
            "output_tokens": result.output_tokens,
            "prompt_tokens": result.prompt_tokens,
        }
        del engine
        torch.cuda.synchronize(device)
        torch.cuda.empty_cache()
    c = cfg
    description = (
        f"{workload}: {spec['model']}-shaped decoder ({c.num_hidden_layers} layers, hidden {c.hidden_size}, "
        f"{c.num_attention_heads}/{c.num_key_value_heads} heads of {c.head_dim}, MLP {c.intermediate_size}, "
        f"vocab {c.vocab_size}{', qk-norm' if c.qk_norm else ''}), random init seed {seed}, bf16; "
        f"{spec['requests']} requests with random prompts "
        + (f"of a shared {spec['prefix']}-token prefix + " if spec["prefix"] else "")
        + f"U[{lo},{hi}] tokens, {spec['max_tokens']} greedy tokens each, max_num_batched_tokens 8192, "
        f"max_num_seqs {spec['max_num_seqs']}, block 16, {num_blocks} KV blocks"
        + (", prefix cache on" if spec["prefix_cache"] else "")
        + ("; torch layers" if unfused else "; fused HIP layer kernels")
        + ("; full block lists sent every step" if full_block_lists else "; device-resident block table (deltas)")
    )
    return {"workload": description, "parameters": model.parameter_count(), "modes": records}


def attention_workload(name: str, device):
    from micro_vllm_amd import workloads

    if name == "qwen3_decode":
        return workloads.qwen3_decode(device), (
            "qwen3_decode: 256 decode sequences, contexts U[128,4096] seed 0, 16 q / 8 kv heads, "
            "head_dim 128, block 16, bf16, 70k-block shuffled pool, values N(0,1)*0.5"
        )
    if name == "llama3_long_decode":
        return workloads.llama3_long_decode(device), (
            "llama3_long_decode: 64 decode sequences, contexts U[8192,33280] seed 0, 32 q / 8 kv heads, "
            "head_dim 128, block 16, bf16, values N(0,1)"
        )
    if name == "llama3_causal_prefill":
        return workloads.llama3_mixed(device, chunk_tokens=4096, offset_range=(0, 0), num_decodes=0), (
            "llama3_causal_prefill: 8 prefill chunks x 4096 from position 0 (causal square, no decodes), "
            "32 q / 8 kv heads, head_dim 128, block 16, bf16"
        )
    if name == "llama3_long_prefill":
        return workloads.llama3_mixed(device, offset_range=(14336, 16384), num_decodes=0), (
            "llama3_long_prefill: 8 prefill chunks x 512 at offsets U[14336,16384] (no decodes), "
            "32 q / 8 kv heads, head_dim 128, block 16, bf16"
        )
    return workloads.llama3_mixed(device), (
        "llama3_mixed: 8 prefill chunks x 512 at offsets U[0,2048] + 248 decodes U[256,8192], "
        "32 q / 8 kv heads, head_dim 128, block 16, bf16"
    )


def settle(run, settle_ms: float) -> int:
    """Untimed forwards for ``settle_ms`` of wall time (synchronized every 8)
    before a measurement's warm-up steps: a GPU that was idle runs its first
    ~50 back-to-back forwards up to 3-4% slower while its clock ramps, and
    five warm-up steps leave the timed ones inside that ramp. Returns the
    number of forwards run."""

    import torch

    n = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        run()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def time_kv_write(w, hip: HipEvents, device, steps: int, warmup: int, settle_ms: float = 0.0) -> dict:
    """The KV-cache write on its own (``mvllm_kv_write``: one launch of
    ``kv_write_rows_kernel``) over the batch's tokens, timed between HIP events
    on the launch stream. The shipped forward fuses this copy into its
    prologue launch; this is the copy kernel's own HBM rate."""

    import torch

    from micro_vllm_amd.attention.operators.mi355x_paged import hip_write_kv_cache

    events = hip.create(2 * steps)
    stream = torch.cuda.current_stream(device).cuda_stream
    hip.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    settle(lambda: hip_write_kv_cache(w.key, w.value, w.cache, w.metadata), settle_ms)
    for _ in range(warmup):
        hip_write_kv_cache(w.key, w.value, w.cache, w.metadata)
    torch.cuda.synchronize()
    for i in range(steps):
        hip.hip.hipEventRecord(ctypes.c_void_p(events[2 * i]), ctypes.c_void_p(stream))
        hip_write_kv_cache(w.key, w.value, w.cache, w.metadata)
        hip.hip.hipEventRecord(ctypes.c_void_p(events[2 * i + 1]), ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    ms = statistics.mean(hip.elapsed_ms(events[2 * i], events[2 * i + 1]) for i in range(steps))
    tokens = int(w.key.shape[0])
    row_bytes = int(w.key.shape[1] * w.key.shape[2] * w.key.element_size())
    moved = tokens * 2 * row_bytes * 2  # K and V rows, read and written
    achieved = moved / (ms * 1e-3) / 1e9
    return {
        "kernel": "kv_write_rows_kernel",
        "bound": "hbm",
        "tokens": tokens,
        "bytes": moved,
        "kernel_us": round(ms * 1e3, 2),
        "achieved": round(achieved, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "note": "standalone copy; the shipped forward fuses it into the prologue launch",
    }


def time_attention(
    w, hip: HipEvents, device, steps: int, warmup: int, concurrent: bool = True, settle_ms: float = 0.0
) -> dict:
    """``settle_ms`` of untimed forwards (``settle``) and ``warmup`` untimed
    forwards, then ``steps`` timed ones between HIP
    events on the launch stream. ``concurrent`` True times the shipped step:
    for a batch with prefill work that is the one-launch step kernel (decode
    and prefill workgroups in one grid), and the library's decode events
    bracket it. ``concurrent`` False asks for the prefill kernel's own events
    as well, which makes the library launch the prefill and decode kernels
    separately on the caller's stream: the per-kernel rooflines come from
    that pass."""

    import torch

    from micro_vllm_amd import _native
    from micro_vllm_amd.attention.operators.mi355x_paged import hip_paged_attention

    marks = hip.create(2)
    decode_events = hip.create(2 * steps)
    prefill_events = hip.create(2 * steps)
    stream = torch.cuda.current_stream(device).cuda_stream
    hip.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    saved = {k: os.environ.get(k) for k in ("MVLLM_PREFILL_CONCURRENT", "MVLLM_STEP_KERNEL")}
    if not concurrent:
        # Separate launches on the caller's stream, warm-up steps included.
        os.environ["MVLLM_PREFILL_CONCURRENT"] = "0"
        os.environ["MVLLM_STEP_KERNEL"] = "0"

    def step(i: int | None):
        timing = None
        if i is not None:
            timing = _native.Timing()
            timing.decode_start, timing.decode_stop = decode_events[2 * i], decode_events[2 * i + 1]
            if not concurrent:
                timing.prefill_start, timing.prefill_stop = prefill_events[2 * i], prefill_events[2 * i + 1]
        return hip_paged_attention(w.query, w.key, w.value, w.cache, w.metadata, timing=timing)

    try:
        settled = settle(lambda: step(None), settle_ms)
        for _ in range(warmup):
            step(None)
        torch.cuda.synchronize()
        hip.hip.hipEventRecord(ctypes.c_void_p(marks[0]), ctypes.c_void_p(stream))
        for i in range(steps):
            step(i)
        hip.hip.hipEventRecord(ctypes.c_void_p(marks[1]), ctypes.c_void_p(stream))
        torch.cuda.synchronize()
        out = {
            "settle_forwards": settled,
            "ms_per_step": hip.elapsed_ms(marks[0], marks[1]) / steps,
            "decode_ms": statistics.mean(hip.elapsed_ms(decode_events[2 * i], decode_events[2 * i + 1]) for i in range(steps)),
        }
        out["prefill_ms"] = None
        if not concurrent and (w.metadata.max_query_len or 0) > 1:
            try:
                out["prefill_ms"] = statistics.mean(
                    hip.elapsed_ms(prefill_events[2 * i], prefill_events[2 * i + 1]) for i in range(steps)
                )
            except RuntimeError:
                # No prefill launch was recorded (the generic kernel ran); the
                # failed query leaves a HIP error behind: clear it.
                hip.hip.hipGetLastError()
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        hip.destroy(marks + decode_events + prefill_events)
    return out


def step_roofline(w, step_ms: float) -> dict:
    """A step against its own floor: the larger of its algorithmic bytes at
    the HBM peak and its prefill FLOPs at the bf16 peak, over its time."""

    from micro_vllm_amd import workloads

    hbm_ms = workloads.decode_bytes(w) / (HBM_PEAK_GBS * 1e9) * 1e3
    mfma_ms = workloads.prefill_flops(w) / (BF16_PEAK_TFLOPS * 1e12) * 1e3
    floor_ms = max(hbm_ms, mfma_ms)
    return {
        "bound": "hbm" if hbm_ms >= mfma_ms else "mfma",
        "floor_ms": round(floor_ms, 5),
        "frac": round(floor_ms / step_ms, 4),
    }


def prefill_record(w, timing: dict) -> dict:
    from micro_vllm_amd import workloads

    flops = workloads.prefill_flops(w)
    if timing.get("prefill_ms") is None:
        return {"flops": int(flops), "kernel_us": None, "note": "prefill ran on the generic kernel"}
    tflops = flops / (timing["prefill_ms"] * 1e-3) / 1e12
    return {
        "kernel": "prefill_kernel<bf16>",
        "bound": "mfma",
        "flops": int(flops),
        "kernel_us": round(timing["prefill_ms"] * 1e3, 2),
        "achieved": round(tflops, 2),
        "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
    }


def e2e_line(args, device) -> dict:
    """One JSON line for an end-to-end workload: the value is output tok/s of
    the first timing mode (synchronized steps summed unless asked)."""

    if args.e2e_eager:
        modes = ("eager",)
    elif args.e2e_pipelined:
        modes = ("pipelined",)
    else:
        modes = ("sync",)
    run = run_generation(
        device, args.workload, modes=modes, requests=args.e2e_requests, max_tokens=args.e2e_max_tokens,
        unfused=args.e2e_unfused, full_block_lists=args.e2e_full_block_lists,
    )
    rec = run["modes"][modes[0]]
    return {
        "metric": METRIC,
        "value": rec["output_tok_s"],
        "unit": "output tok/s",
        "n_gpus": 1,
        "steps": rec["steps"],
        "warmup": 1,
        "ms_per_step": round(rec["step_seconds"] / rec["steps"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": run["workload"], "parameters": run["parameters"], **rec, "parallelism": "single GPU"},
        "roofline": None,
        "cpu_baseline": None,
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument(
        "--settle-ms",
        type=float,
        default=150.0,
        help="untimed forwards for this long before each measurement's warm-up steps (0: none)",
    )
    parser.add_argument(
        "--workload",
        default="qwen3_decode",
        choices=[
            "qwen3_decode",
            "llama3_mixed",
            "llama3_long_prefill",
            "llama3_causal_prefill",
            "llama3_long_decode",
            "qwen3_e2e",
            "llama3_e2e",
            "small_mixed",
        ],
    )
    parser.add_argument(
        "--quick",
        action="store_true",
        help="qwen3_decode without the mixed-batch prefill roofline and the Qwen3-0.6B end-to-end run",
    )
    parser.add_argument("--e2e-requests", type=int, default=None, help="requests of an end-to-end workload")
    parser.add_argument("--e2e-max-tokens", type=int, default=None, help="greedy output tokens per request")
    parser.add_argument("--e2e-eager", action="store_true", help="end-to-end steps eagerly (no HIP graphs)")
    parser.add_argument(
        "--e2e-unfused", action="store_true", help="end-to-end with the torch layers instead of the fused HIP layer kernels"
    )
    parser.add_argument(
        "--e2e-pipelined",
        action="store_true",
        help="end-to-end with the host one graph step ahead (the loop's wall time instead of summed steps)",
    )
    parser.add_argument(
        "--e2e-full-block-lists",
        action="store_true",
        help="end-to-end packing that re-sends every request's block list each step (no device-resident table)",
    )
    parser.add_argument(
        "--no-hint",
        action="store_true",
        help="attention metadata without the max_query_len hint (the reference's AttentionMetadata fields only)",
    )
    parser.add_argument("--cpu-sample", type=int, default=256, help="sequences timed by the CPU baseline")
    parser.add_argument("--cpu-repeats", type=int, default=5)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument(
        "--no-llama3-e2e", action="store_true", help="skip the Llama-3-8B end-to-end run of the default workload"
    )
    parser.add_argument(
        "--no-torch-baseline", action="store_true", help="skip the torch gathered-attention baseline on the same GPU"
    )
    parser.add_argument(
        "--copy-calibration-mib",
        type=int,
        default=0,
        help="after the timed steps, run one elementwise kernel that reads and writes this many MiB "
        "(a plain copy of known traffic, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)",
    )
    args = parser.parse_args()

    if args.gpus != 1:
        print(
            f"bench.py runs on one GPU: --gpus {args.gpus} is not supported "
            "(the multi-GPU sharding of the path is described, not implemented).",
            file=sys.stderr,
        )
        return 2

    import torch

    from micro_vllm_amd import _native, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a visible GPU", file=sys.stderr)
        return 1
    _native.load()
    device = torch.device("cuda", 0)
    if args.workload in E2E_CONFIGS:
        print(json.dumps(e2e_line(args, device)), flush=True)
        return 0
    if args.workload == "small_mixed":
        # The config-1 record alone (fp32 and bf16 forwards, the CPU path beside them).
        line = {"metric": "forward latency, contexts [17, 64, 130, 255]", "unit": "us", "higher_is_better": False,
                "n_gpus": 1, "data": "synthetic"}
        line.update(small_mixed_record(HipEvents(), device))
        print(json.dumps(line), flush=True)
        return 0

    w, description = attention_workload(args.workload, device)
    if args.no_hint:
        import dataclasses

        w.metadata = dataclasses.replace(w.metadata, max_query_len=None)
        description += "; metadata without the max_query_len hint"
    torch.cuda.synchronize()
    hip = HipEvents()
    timing = time_attention(w, hip, device, args.steps, args.warmup, settle_ms=args.settle_ms)
    ms_per_step, decode_ms = timing["ms_per_step"], timing["decode_ms"]
    overlap = None
    if args.workload in PREFILL_WORKLOADS:
        # The library runs a mixed batch as one launch whose grid holds the
        # decode and the prefill workgroups. The step above is that shipped
        # one; each kernel's roofline comes from a second pass with the two
        # kernels launched separately, one after the other.
        serial = time_attention(w, hip, device, args.steps, args.warmup, concurrent=False, settle_ms=args.settle_ms)
        decode_ms = serial["decode_ms"]
        overlap = {
            "ms_per_step_serial": round(serial["ms_per_step"], 5),
            "note": "decode and prefill workgroups in one step kernel; kernel rooflines from the serial pass",
        }

    step_bytes = workloads.decode_bytes(w)
    kernel_bytes = decode_kernel_bytes(w)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = kernel_bytes / (decode_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {
            "ms": args.settle_ms,
            "forwards": timing["settle_forwards"],
            "note": "untimed forwards before the warm-up steps, so that the timed steps run at the clock the "
            "part settles at under this load",
        },
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": description,
            "num_sequences": int(len(w.context_lengths)),
            "num_tokens": int(w.query_lengths.sum()),
            "context_tokens": int(w.context_lengths.sum()),
            "step_bytes": int(step_bytes),
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "decode_split_lds_kernel<bf16, 2>",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.workload),
            "kernel_us": round(decode_ms * 1e3, 2),
            "kernel_bytes": int(kernel_bytes),
        },
    }
    if args.workload == "llama3_long_decode":
        # Host cost of caching every request's full blocks after one decode
        # step (prefix-cache digests), the reference's from-scratch chains
        # against incremental ones, for this batch's contexts.
        from micro_vllm_amd.harness.prefix_hash import measure_step_cost

        result["control_plane"] = {"prefix_hash": measure_step_cost(w.context_lengths.tolist(), steps=3)}
    if overlap is not None:
        result["overlap"] = overlap
    if args.workload in PREFILL_WORKLOADS:
        result["prefill"] = prefill_record(w, serial)
        if not bool((w.query_lengths == 1).any()) and result["prefill"].get("kernel_us"):
            # No decode request: the decode launch finds no work, so the
            # step is priced by its FLOPs and the prefill kernel is the
            # roofline.
            flops = result["prefill"]["flops"]
            result["unit"] = "TFLOP/s"
            result["value"] = round(flops / (ms_per_step * 1e-3) / 1e12, 2)
            result["roofline"] = {k: result["prefill"][k] for k in
                                  ("kernel", "bound", "achieved", "peak", "unit", "frac", "kernel_us", "flops")}
            result["roofline"]["traffic"] = None
        if not args.no_cpu_baseline:
            result["prefill"]["cpu_baseline"] = cpu_prefill_baseline(w)
        from micro_vllm_amd.attention.operators.mi355x_paged import hip_paged_attention

        hip_out = hip_paged_attention(w.query, w.key, w.value, w.cache, w.metadata)
        result["prefill"]["library"] = library_prefill_baseline(w, hip_out)
        del hip_out
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_torch_baseline:
        from micro_vllm_amd.attention.operators.mi355x_paged import hip_paged_attention

        hip_out = hip_paged_attention(w.query, w.key, w.value, w.cache, w.metadata)
        torch.cuda.synchronize()
        result["gpu_baseline"] = torch_baseline(w, hip_out)
        result["gpu_baseline"]["hip_speedup"] = round(result["gpu_baseline"]["ms_per_step"] / ms_per_step, 2)
        del hip_out
        torch.cuda.empty_cache()
    result["cpu_baseline"] = None if args.no_cpu_baseline else cpu_baseline(w, args.cpu_sample, args.cpu_repeats)

    if args.workload == "qwen3_decode" and not args.quick:
        # The other targets on their own configurations, in the same line:
        # the reference's CPU-runnable case on both sides, the prefill kernel
        # on the Llama-3 mixed batch (bf16 MFMA roofline), Qwen3-0.6B and
        # Llama-3-8B end-to-end output tok/s.
        del w
        torch.cuda.empty_cache()
        result["config1"] = small_mixed_record(hip, device)
        mixed, mixed_description = attention_workload("llama3_mixed", device)
        shipped = time_attention(mixed, hip, device, args.steps, args.warmup, settle_ms=args.settle_ms)
        serial = time_attention(mixed, hip, device, args.steps, args.warmup, concurrent=False, settle_ms=args.settle_ms)
        record = prefill_record(mixed, serial)
        record["workload"] = mixed_description
        record["mixed_step_ms"] = round(shipped["ms_per_step"], 5)
        record["mixed_step_ms_serial"] = round(serial["ms_per_step"], 5)
        record["decode_part_frac"] = round(decode_kernel_bytes(mixed) / (serial["decode_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        record["mixed_step_roofline"] = step_roofline(mixed, shipped["ms_per_step"])
        from micro_vllm_amd.attention.operators.mi355x_paged import hip_paged_attention

        mixed_out = hip_paged_attention(mixed.query, mixed.key, mixed.value, mixed.cache, mixed.metadata)
        record["library"] = library_prefill_baseline(mixed, mixed_out)
        del mixed_out
        if not args.no_cpu_baseline:
            record["cpu_baseline"] = cpu_prefill_baseline(mixed)
        # The same batch in fp16, the only dtype of the reference's Triton
        # backend (dense fp16 MFMA peak = the bf16 one).
        mixed16 = workloads.llama3_mixed(device, dtype=torch.float16)
        serial16 = time_attention(
            mixed16, hip, device, args.steps, args.warmup, concurrent=False, settle_ms=args.settle_ms
        )
        fp16 = prefill_record(mixed16, serial16)
        record["fp16"] = {
            "kernel": "prefill_kernel<fp16>",
            "kernel_us": fp16.get("kernel_us"),
            "achieved": fp16.get("achieved"),
            "frac": fp16.get("frac"),
        }
        del mixed16
        torch.cuda.empty_cache()
        result["prefill"] = record
        kv = time_kv_write(mixed, hip, device, args.steps, args.warmup, settle_ms=args.settle_ms)
        kv["workload"] = f"llama3_mixed: the step's {kv['tokens']:,} tokens (8 KV heads, head_dim 128, bf16)"
        result["kv_write"] = kv
        del mixed
        torch.cuda.empty_cache()
        run = run_generation(device, "qwen3_e2e", modes=("sync", "pipelined"))
        sync, pipelined = run["modes"]["sync"], run["modes"]["pipelined"]
        result["e2e"] = {
            "workload": run["workload"],
            "value": sync["output_tok_s"],
            "unit": "output tok/s",
            "timing": "synchronized engine steps summed (benchmarks/benchmark_engine.py:305-315)",
            "value_pipelined": pipelined["output_tok_s"],
            "sync": sync,
            "pipelined": pipelined,
        }
        del run
        torch.cuda.empty_cache()
        if not args.no_llama3_e2e:
            run = run_generation(device, "llama3_e2e", modes=("sync",))
            sync = run["modes"]["sync"]
            result["e2e_llama3"] = {
                "workload": run["workload"],
                "parameters": run["parameters"],
                "value": sync["output_tok_s"],
                "unit": "output tok/s",
                "timing": "synchronized engine steps summed (benchmarks/benchmark_engine.py:305-315)",
                "sync": sync,
            }
            del run
            torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
