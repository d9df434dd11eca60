"""Storage-type helpers for the oracle (TEST INFRASTRUCTURE ONLY).

The oracle holds tensors as numpy arrays. float32 and float16 arrays are used
as is. bfloat16 has no numpy type, so a bfloat16 tensor is carried as its raw
16-bit patterns in a ``np.uint16`` array; ``to_f32`` widens it exactly and
``from_f32`` rounds back with round-to-nearest-even, which is what
``torch.Tensor.to(torch.bfloat16)`` does (and what the reference relies on when
``output.copy_(attention)`` narrows fp32 results, reference.py:79).
"""

from __future__ import annotations

import numpy as np

BF16 = "bfloat16"
F16 = "float16"
F32 = "float32"


def storage_kind(array: np.ndarray) -> str:
    """Name the element type an oracle array stands for."""

    if array.dtype == np.float32:
        return F32
    if array.dtype == np.float16:
        return F16
    if array.dtype == np.uint16:
        return BF16
    raise TypeError(f"unsupported oracle storage dtype {array.dtype}")


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening: a bfloat16 is the top half of an IEEE float32."""

    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(
        np.float32
    )


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 bit patterns, nearest-even, NaN kept quiet."""

    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    is_nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        rounded = (u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    out = rounded.astype(np.uint16)
    if np.any(is_nan):
        out[is_nan] = ((u[is_nan] >> np.uint32(16)) | np.uint32(0x40)).astype(
            np.uint16
        )
    return out


def to_f32(array: np.ndarray) -> np.ndarray:
    """Widen any oracle storage array to float32 exactly."""

    kind = storage_kind(array)
    if kind == BF16:
        return bf16_bits_to_f32(array)
    return array.astype(np.float32)


def from_f32(values: np.ndarray, kind: str) -> np.ndarray:
    """Narrow float32 values to the named storage type (nearest-even)."""

    if kind == F32:
        return np.asarray(values, dtype=np.float32)
    if kind == F16:
        return np.asarray(values, dtype=np.float32).astype(np.float16)
    if kind == BF16:
        return f32_to_bf16_bits(values)
    raise TypeError(f"unsupported storage kind {kind!r}")
