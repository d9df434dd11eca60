"""CPU checks of the drop-in boundary (no compute calls).

* the C-ABI library loads and exports every function ``include/*.h``
  declares, and the ctypes binding names exactly that set;
* the Python mirror of the reference interface keeps its names and error
  conventions (registry: ValueError for unknown names; operator: RuntimeError
  for tensors off the GPU; frozen metadata; spec validation).
"""

from __future__ import annotations

import ctypes
import re
from dataclasses import FrozenInstanceError
from pathlib import Path

import pytest
import torch

from micro_vllm_amd import _native
from micro_vllm_amd.attention import (
    Attention,
    AttentionMetadata,
    ChunkedLocalSpec,
    FullAttentionSpec,
    SlidingWindowSpec,
    map_cache_slots,
)
from micro_vllm_amd.attention.operators.base import AttentionOperator
from micro_vllm_amd.attention.operators.registry import get_attention_operator_class

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(mvllm_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_and_binding_declare_the_same_functions():
    assert declared_functions() == set(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(_native.LIBRARY_PATH))
    missing = [name for name in sorted(declared_functions()) if not hasattr(lib, name)]
    assert not missing
    lib = _native.load()
    assert lib.mvllm_abi_version() == _native.ABI_VERSION
    assert lib.mvllm_last_error() == b""


def test_struct_sizes_match_the_header_layout():
    # 8-byte pointer + 2 x int32 + int64 fields, no implicit padding.
    assert ctypes.sizeof(_native.Tensor3) == 8 + 8 + 6 * 8
    assert ctypes.sizeof(_native.KVCache) == 8 + 8 + 4 * 8 + 5 * 8
    assert ctypes.sizeof(_native.Batch) == 6 * 8 + 3 * 8 + 2 * 8 + 8 + 8
    assert ctypes.sizeof(_native.PackArgs) == 3 * 8 + 5 * 8 + 8 + 4 * 8 + 8 * 8
    assert ctypes.sizeof(_native.Timing) == 4 * 8
    assert ctypes.sizeof(_native.BlockRows) == 8 + 2 * 8 + 8 + 8


def test_library_rejects_bad_arguments_without_a_device():
    lib = _native.load()
    assert lib.mvllm_pack_batch(None, None) == _native.ERR_INVALID
    assert lib.mvllm_pack_batch_rows(None, None, None) == _native.ERR_INVALID
    assert b"rows" in lib.mvllm_last_error()
    assert b"null" in lib.mvllm_last_error()
    assert lib.mvllm_context_starts(None, 4, 7, 0, None, None) == _native.ERR_INVALID
    assert b"spec" in lib.mvllm_last_error()
    assert lib.mvllm_kv_write(None, None, None, None, 0, None) == _native.ERR_INVALID
    assert lib.mvllm_attention_workspace_bytes(None, 16, 128) == 0
    assert lib.mvllm_attention_plan(None, 16, None, None, 0, None) == _native.ERR_INVALID
    assert b"cache" in lib.mvllm_last_error()
    assert lib.mvllm_paged_attention_planned(None, None, None, None, 1.0, None, 0, None) == _native.ERR_INVALID


def test_registry_returns_the_hip_operator():
    cls = get_attention_operator_class("mi355x_paged")
    assert issubclass(cls, AttentionOperator)


def test_registry_rejects_unknown_names():
    with pytest.raises(ValueError, match=r"unsupported attention operator 'unknown'.*mi355x_paged"):
        get_attention_operator_class("unknown")


def test_operator_rejects_cpu_tensors():
    token = torch.zeros((1, 1, 16), dtype=torch.bfloat16)
    cache = torch.zeros((2, 1, 1, 1, 16), dtype=torch.bfloat16)
    metadata = AttentionMetadata(
        query_positions=torch.tensor((0,)),
        query_context_start_positions=torch.tensor((0,)),
        query_start_locations=torch.tensor((0, 1)),
        context_lengths=torch.tensor((1,)),
        block_table=torch.tensor(((0,),)),
        slot_mapping=torch.tensor((0,)),
        block_size=1,
    )
    operator = get_attention_operator_class("mi355x_paged")()
    with pytest.raises(RuntimeError, match="requires GPU tensors"):
        operator(token, token, token, cache, metadata)
    with pytest.raises(RuntimeError, match="GPU"):
        Attention(FullAttentionSpec(), "mi355x_paged").build_metadata(
            query_positions=metadata.query_positions,
            query_start_locations=metadata.query_start_locations,
            context_lengths=metadata.context_lengths,
            block_table=metadata.block_table,
            slot_mapping=metadata.slot_mapping,
            block_size=1,
        )


def test_metadata_is_frozen_and_counts_requests():
    metadata = AttentionMetadata(
        query_positions=torch.tensor((0, 1)),
        query_context_start_positions=torch.tensor((0, 0)),
        query_start_locations=torch.tensor((0, 1, 2)),
        context_lengths=torch.tensor((1, 2)),
        block_table=torch.tensor(((0,), (1,))),
        slot_mapping=torch.tensor((0, 5)),
        block_size=4,
    )
    assert metadata.num_requests == 2
    with pytest.raises(FrozenInstanceError):
        metadata.block_size = 8  # type: ignore[misc]


@pytest.mark.parametrize("cls,field", [(SlidingWindowSpec, "window_size"), (ChunkedLocalSpec, "chunk_size")])
@pytest.mark.parametrize("value", [0, -1, True, 1.5])
def test_bounded_specs_require_positive_integers(cls, field, value):
    with pytest.raises(ValueError, match=f"{field} must be a positive integer"):
        cls(value)


def test_map_cache_slots_matches_reference_vector():
    # tests/worker/test_model_runner.py:383-402: positions 3, 4 with blocks (2, 5), block 4.
    slots = map_cache_slots(torch.tensor([3, 4]), torch.tensor([2, 5]), 4)
    assert slots.tolist() == [11, 20]


def test_noalloc_entry_point_rejects_batches_beyond_its_workspace():
    """The allocation-free entry point checks the batch's workspace need
    against its fixed device array before it touches any pointer."""

    lib = _native.load()
    q = _native.Tensor3()
    q.dtype = _native.DTYPE_BF16
    q.size[0], q.size[1], q.size[2] = 4096, 32, 128
    b = _native.Batch()
    b.num_tokens, b.num_requests, b.block_table_width, b.block_size = 4096, 4096, 2048, 16
    need = lib.mvllm_attention_workspace_bytes(b, 32, 128)
    assert need > _native.NOALLOC_SCRATCH_BYTES
    status = lib.mvllm_attention_forward_noalloc(q, q, q, _native.KVCache(), b, q, 1.0, None)
    assert status == _native.ERR_WORKSPACE
    message = lib.mvllm_last_error()
    assert str(need).encode() in message and str(_native.NOALLOC_SCRATCH_BYTES).encode() in message
