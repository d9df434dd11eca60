"""The reference operator's CPU path in torch (TEST INFRASTRUCTURE ONLY).

The CPU baseline that ``bench.py`` times on the GPU host's own cores, and
nothing else: the HIP library never calls it. It performs the same steps as
``ReferenceAttentionOperator.forward`` (src/micro_vllm/attention/operators/
reference.py:14-81, with ``write_kv_cache`` :84-98 and ``gather_kv_cache``
:101-138), which is what makes it the reference's cost on a CPU:

* the step's K/V rows are copied into their slots of the flat cache view
  (``index_copy_``);
* per request, the slots of positions [context start of its first query,
  context length) are formed from the block table and gathered with
  ``index_select``;
* GQA: the gathered heads are expanded to the query heads with
  ``repeat_interleave``;
* scores = einsum over fp32 copies, masked where a key lies before the
  query's context start or after its position, softmax(scores * D^-1/2) in
  fp32, times fp32 values, written into the output in the query's dtype.

Per-request ``.item()`` reads mirror the reference's host loop. Parity with
the numpy oracle (``oracle.paged_attention``) is checked in
``tests/test_oracle.py``.
"""

from __future__ import annotations

import math

import torch


def write_kv_cache(key, value, cache, slot_mapping) -> None:
    planes = cache.view(2, -1, *cache.shape[3:])
    planes[0].index_copy_(0, slot_mapping, key)
    planes[1].index_copy_(0, slot_mapping, value)


def gather_kv_cache(cache, query_positions, context_starts, query_start_locations, context_lengths, block_table, block_size):
    planes = cache.view(2, -1, *cache.shape[3:])
    histories = []
    for r in range(context_lengths.numel()):
        first = int(context_starts[int(query_start_locations[r])].item())
        length = int(context_lengths[r].item())
        pos = torch.arange(first, length, dtype=torch.int64)
        slots = block_table[r][pos // block_size] * block_size + pos % block_size
        histories.append((planes[0].index_select(0, slots), planes[1].index_select(0, slots)))
    return histories


def reference_forward(query, key, value, cache, query_positions, context_starts, query_start_locations,
                      context_lengths, block_table, slot_mapping, block_size) -> torch.Tensor:
    """One forward of the reference operator on CPU tensors; ``cache`` is
    written in place and a new output tensor is returned."""

    write_kv_cache(key, value, cache, slot_mapping)
    histories = gather_kv_cache(
        cache, query_positions, context_starts, query_start_locations, context_lengths, block_table, block_size
    )
    group = query.shape[1] // key.shape[1]
    scale = 1.0 / math.sqrt(query.shape[-1])
    out = torch.empty_like(query)
    for r, (k, v) in enumerate(histories):
        q0 = int(query_start_locations[r].item())
        q1 = int(query_start_locations[r + 1].item())
        if group > 1:
            k = k.repeat_interleave(group, dim=1)
            v = v.repeat_interleave(group, dim=1)
        scores = torch.einsum("qhd,khd->hqk", query[q0:q1].to(torch.float32), k.to(torch.float32))
        first = int(context_starts[q0].item())
        kpos = torch.arange(first, first + k.shape[0], dtype=torch.int64)
        hidden = (kpos[None, :] < context_starts[q0:q1, None]) | (kpos[None, :] > query_positions[q0:q1, None])
        scores.masked_fill_(hidden[None], -torch.inf)
        weights = torch.softmax(scores * scale, dim=-1, dtype=torch.float32)
        out[q0:q1].copy_(torch.einsum("hqk,khd->qhd", weights, v.to(torch.float32)))
    return out
