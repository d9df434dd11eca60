"""Tensor operator contract shared by all attention semantics.

Same interface as the reference's src/micro_vllm/attention/operators/base.py:10-40:
positional-only ``(query, key, value, layer_kv_cache, metadata)``; the
operator writes the current K/V into ``layer_kv_cache`` in place and returns
a new tensor shaped, typed and placed like ``query``.
"""

from abc import ABC, abstractmethod

import torch

from micro_vllm_amd.attention.attention import AttentionMetadata


class AttentionOperator(ABC):
    """Compute attention from Q/K/V tensors and semantic metadata."""

    def __call__(
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        layer_kv_cache: torch.Tensor,
        metadata: AttentionMetadata,
        /,
    ) -> torch.Tensor:
        return self.forward(
            query,
            key,
            value,
            layer_kv_cache,
            metadata,
        )

    @abstractmethod
    def forward(
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        layer_kv_cache: torch.Tensor,
        metadata: AttentionMetadata,
        /,
    ) -> torch.Tensor:
        """Compute attention for one layer."""
