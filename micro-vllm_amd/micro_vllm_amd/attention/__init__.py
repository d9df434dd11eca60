"""Attention semantics, metadata and operators."""

from micro_vllm_amd.attention.attention import (  # noqa: F401
    Attention,
    AttentionMetadata,
    context_starts,
    map_cache_slots,
)
from micro_vllm_amd.attention.spec import (  # noqa: F401
    AttentionSpec,
    ChunkedLocalSpec,
    FullAttentionSpec,
    SlidingWindowSpec,
)
