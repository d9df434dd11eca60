"""Attention operator registry.

Same lookup contract as the reference's registry.py:24-50: a name maps to an
operator class; a backend whose native dependency is missing raises
``RuntimeError`` naming it; an unknown name raises ``ValueError`` listing
the supported names.
"""

from micro_vllm_amd.attention.operators.base import AttentionOperator

SUPPORTED_OPERATORS = ("mi355x_paged",)


def get_attention_operator_class(name: str) -> type[AttentionOperator]:
    """Return the registered attention operator class with the given name."""

    if name == "mi355x_paged":
        from micro_vllm_amd import _native

        try:
            _native.load()
        except _native.NativeLibraryError as error:
            raise RuntimeError(
                f"attention operator 'mi355x_paged' requires the HIP library: {error}"
            ) from error
        from micro_vllm_amd.attention.operators.mi355x_paged import (
            MI355XPagedAttentionOperator,
        )

        return MI355XPagedAttentionOperator

    raise ValueError(
        f"unsupported attention operator {name!r}; "
        f"supported operators: {list(SUPPORTED_OPERATORS)!r}"
    )
