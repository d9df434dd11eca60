"""A torch (GPU) restatement of the reference attention operator, against
which end-to-end greedy decoding is compared (TEST INFRASTRUCTURE ONLY).

Same semantics as ReferenceAttentionOperator.forward
(src/micro_vllm/attention/operators/reference.py:14-138): write the step's
K/V into its slots, then per request gather the history from
start(first query) to the context length through the block table, expand the
KV heads over the query-head group, and compute masked softmax(q.k * D^-1/2).v
in float32, narrowed to the query dtype. Tokens outside every request are
zero.
"""

from __future__ import annotations

import math

import torch


class TorchReferenceAttention:
    def __call__(self, query, key, value, cache, md):
        num_kv = key.shape[1]
        d = query.shape[-1]
        group = query.shape[1] // num_kv
        flat = cache.view(2, -1, num_kv, d)
        slots = md.slot_mapping
        keep = slots >= 0
        flat[0].index_copy_(0, slots[keep], key[keep])
        flat[1].index_copy_(0, slots[keep], value[keep])
        out = torch.zeros_like(query)
        qsl = md.query_start_locations.tolist()
        lengths = md.context_lengths.tolist()
        starts = md.query_context_start_positions
        positions = md.query_positions
        bs = md.block_size
        for r in range(len(lengths)):
            qs, qe = qsl[r], qsl[r + 1]
            if qe <= qs:
                continue
            first = int(starts[qs])
            key_pos = torch.arange(first, lengths[r], device=query.device)
            row = md.block_table[r]
            slot_ids = row[key_pos // bs] * bs + key_pos % bs
            k = flat[0, slot_ids].float().repeat_interleave(group, dim=1).permute(1, 2, 0).contiguous()
            v = flat[1, slot_ids].float().repeat_interleave(group, dim=1).permute(1, 0, 2).contiguous()
            q = query[qs:qe].float().permute(1, 0, 2).contiguous()
            scores = torch.matmul(q, k) / math.sqrt(d)  # [H, nq, nk]
            masked = (key_pos[None, :] < starts[qs:qe, None]) | (key_pos[None, :] > positions[qs:qe, None])
            scores = scores.masked_fill(masked[None], float("-inf"))
            weights = torch.softmax(scores, dim=-1)
            out[qs:qe] = torch.matmul(weights, v).permute(1, 0, 2).to(query.dtype)
        return out
