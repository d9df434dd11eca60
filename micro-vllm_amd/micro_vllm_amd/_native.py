"""ctypes binding of the gfx950 HIP library (``_lib/libmvllm_amd.so``).

The structures below mirror ``include/mvllm_amd.h`` field for field. The
library is loaded after ``torch`` so that it binds to the HIP runtime torch
already loaded. There is no fallback: if the library is missing, every
entry point raises ``NativeLibraryError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "_lib" / "libmvllm_amd.so"

ABI_VERSION = 5

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

SPEC_FULL = 0
SPEC_SLIDING_WINDOW = 1
SPEC_CHUNKED_LOCAL = 2

PACK_FIELDS = 8

ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_WORKSPACE = -4

# Device workspace of mvllm_attention_forward_noalloc (MVLLM_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 * 1024 * 1024

# Every function declared in include/mvllm_amd.h.
EXPORTED_SYMBOLS = (
    "mvllm_kv_write",
    "mvllm_attention_workspace_bytes",
    "mvllm_paged_attention",
    "mvllm_attention_plan",
    "mvllm_paged_attention_planned",
    "mvllm_attention_forward",
    "mvllm_attention_forward_timed",
    "mvllm_attention_forward_noalloc",
    "mvllm_gather_kv",
    "mvllm_context_starts",
    "mvllm_pack_batch",
    "mvllm_pack_batch_rows",
    "mvllm_add_rms_norm",
    "mvllm_qk_norm_rope_kv_write",
    "mvllm_silu_mul",
    "mvllm_embed_rms_norm",
    "mvllm_argmax_rows",
    "mvllm_last_error",
    "mvllm_abi_version",
)

_TORCH_DTYPES = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
}

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


class Tensor3(ctypes.Structure):
    _fields_ = [
        ("data", _ptr),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("size", _i64 * 3),
        ("stride", _i64 * 3),
    ]


class KVCache(ctypes.Structure):
    _fields_ = [
        ("data", _ptr),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("num_blocks", _i64),
        ("block_size", _i64),
        ("num_kv_heads", _i64),
        ("head_dim", _i64),
        ("stride", _i64 * 5),
    ]


class Batch(ctypes.Structure):
    _fields_ = [
        ("query_positions", _ptr),
        ("query_context_start_positions", _ptr),
        ("query_start_locations", _ptr),
        ("context_lengths", _ptr),
        ("block_table", _ptr),
        ("slot_mapping", _ptr),
        ("num_tokens", _i64),
        ("num_requests", _i64),
        ("block_table_width", _i64),
        ("block_table_stride", _i64 * 2),
        ("block_size", _i64),
        ("max_query_len", _i64),
    ]


class PackArgs(ctypes.Structure):
    _fields_ = [
        ("request_info", _ptr),
        ("block_ids", _ptr),
        ("token_ids", _ptr),
        ("num_requests", _i64),
        ("num_tokens", _i64),
        ("num_block_ids", _i64),
        ("block_size", _i64),
        ("null_block_id", _i64),
        ("spec_kind", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("spec_parameter", _i64),
        ("token_capacity", _i64),
        ("request_capacity", _i64),
        ("block_table_width", _i64),
        ("input_ids", _ptr),
        ("positions", _ptr),
        ("context_starts", _ptr),
        ("query_start_locations", _ptr),
        ("context_lengths", _ptr),
        ("block_table", _ptr),
        ("slot_mapping", _ptr),
        ("sampling_rows", _ptr),
    ]


class BlockRows(ctypes.Structure):
    _fields_ = [
        ("rows", _ptr),
        ("num_slots", _i64),
        ("width", _i64),
        ("updates", _ptr),
        ("num_updates", _i64),
    ]


class Timing(ctypes.Structure):
    _fields_ = [
        ("decode_start", _ptr),
        ("decode_stop", _ptr),
        ("prefill_start", _ptr),
        ("prefill_stop", _ptr),
    ]


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or unusable."""


_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    p = ctypes.POINTER
    lib.mvllm_kv_write.argtypes = [p(Tensor3), p(Tensor3), p(KVCache), _ptr, _i64, _ptr]
    lib.mvllm_kv_write.restype = ctypes.c_int
    lib.mvllm_attention_workspace_bytes.argtypes = [p(Batch), _i64, _i64]
    lib.mvllm_attention_workspace_bytes.restype = _i64
    lib.mvllm_paged_attention.argtypes = [
        p(Tensor3), p(KVCache), p(Batch), p(Tensor3), ctypes.c_float, _ptr, _i64, _ptr,
    ]
    lib.mvllm_paged_attention.restype = ctypes.c_int
    lib.mvllm_attention_plan.argtypes = [p(Batch), _i64, p(KVCache), _ptr, _i64, _ptr]
    lib.mvllm_attention_plan.restype = ctypes.c_int
    lib.mvllm_paged_attention_planned.argtypes = [
        p(Tensor3), p(KVCache), p(Batch), p(Tensor3), ctypes.c_float, _ptr, _i64, _ptr,
    ]
    lib.mvllm_paged_attention_planned.restype = ctypes.c_int
    lib.mvllm_attention_forward.argtypes = [
        p(Tensor3), p(Tensor3), p(Tensor3), p(KVCache), p(Batch), p(Tensor3),
        ctypes.c_float, _ptr, _i64, _ptr,
    ]
    lib.mvllm_attention_forward.restype = ctypes.c_int
    lib.mvllm_attention_forward_timed.argtypes = [
        p(Tensor3), p(Tensor3), p(Tensor3), p(KVCache), p(Batch), p(Tensor3),
        ctypes.c_float, _ptr, _i64, p(Timing), _ptr,
    ]
    lib.mvllm_attention_forward_timed.restype = ctypes.c_int
    lib.mvllm_attention_forward_noalloc.argtypes = [
        p(Tensor3), p(Tensor3), p(Tensor3), p(KVCache), p(Batch), p(Tensor3), ctypes.c_float, _ptr,
    ]
    lib.mvllm_attention_forward_noalloc.restype = ctypes.c_int
    lib.mvllm_gather_kv.argtypes = [p(KVCache), p(Batch), _i64, _ptr, _ptr, _ptr]
    lib.mvllm_gather_kv.restype = ctypes.c_int
    lib.mvllm_context_starts.argtypes = [_ptr, _i64, ctypes.c_int32, _i64, _ptr, _ptr]
    lib.mvllm_context_starts.restype = ctypes.c_int
    lib.mvllm_pack_batch.argtypes = [p(PackArgs), _ptr]
    lib.mvllm_pack_batch.restype = ctypes.c_int
    lib.mvllm_pack_batch_rows.argtypes = [p(PackArgs), p(BlockRows), _ptr]
    lib.mvllm_pack_batch_rows.restype = ctypes.c_int
    lib.mvllm_add_rms_norm.argtypes = [_ptr, _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int32, _ptr]
    lib.mvllm_add_rms_norm.restype = ctypes.c_int
    lib.mvllm_qk_norm_rope_kv_write.argtypes = [
        p(Tensor3), p(Tensor3), p(Tensor3), _ptr, _ptr, _ptr, _ptr, _ptr, _i64, ctypes.c_float, _ptr, p(KVCache),
        _ptr, _ptr,
    ]
    lib.mvllm_qk_norm_rope_kv_write.restype = ctypes.c_int
    lib.mvllm_silu_mul.argtypes = [_ptr, _i64, _ptr, _i64, _i64, _i64, ctypes.c_int32, _ptr]
    lib.mvllm_silu_mul.restype = ctypes.c_int
    lib.mvllm_embed_rms_norm.argtypes = [
        _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64, _i64, ctypes.c_float, ctypes.c_int32,
        _ptr,
    ]
    lib.mvllm_embed_rms_norm.restype = ctypes.c_int
    lib.mvllm_argmax_rows.argtypes = [_ptr, _i64, _i64, _i64, ctypes.c_int32, _ptr, _ptr, _ptr]
    lib.mvllm_argmax_rows.restype = ctypes.c_int
    lib.mvllm_last_error.argtypes = []
    lib.mvllm_last_error.restype = ctypes.c_char_p
    lib.mvllm_abi_version.argtypes = []
    lib.mvllm_abi_version.restype = ctypes.c_int


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is absent or stale."""

    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.exists():
            raise NativeLibraryError(
                f"HIP library not found at {LIBRARY_PATH}; build it with "
                "`python micro-vllm_amd/build.py` (hipcc, gfx950)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as error:
            raise NativeLibraryError(f"cannot load {LIBRARY_PATH}: {error}") from error
        missing = [name for name in EXPORTED_SYMBOLS if not hasattr(lib, name)]
        if missing:
            raise NativeLibraryError(f"{LIBRARY_PATH} lacks symbols {missing}; rebuild it")
        _declare(lib)
        version = lib.mvllm_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(
                f"{LIBRARY_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
            )
        _library = lib
        return lib


def available() -> bool:
    try:
        load()
    except NativeLibraryError:
        return False
    return True


def check(status: int, what: str) -> None:
    """Map a negative status to an exception carrying the library's text."""

    if status == 0:
        return
    message = (load().mvllm_last_error() or b"").decode(errors="replace")
    if status == ERR_UNSUPPORTED:
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what} failed ({status}): {message}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DTYPES[dtype]
    except KeyError as error:
        raise ValueError(f"unsupported dtype {dtype}") from error


def tensor3(t: torch.Tensor) -> Tensor3:
    if t.dim() != 3:
        raise ValueError(f"expected a 3-D [tokens, heads, dim] tensor, got shape {tuple(t.shape)}")
    d = Tensor3()
    d.data = t.data_ptr() if t.numel() else None
    d.dtype = dtype_code(t.dtype)
    for i in range(3):
        d.size[i] = t.shape[i]
        d.stride[i] = t.stride(i)
    return d


def kv_cache(cache: torch.Tensor, block_size: int | None = None) -> KVCache:
    if cache.dim() != 5 or cache.shape[0] != 2:
        raise ValueError(
            "layer_kv_cache must be shaped (2, num_blocks, block_size, num_kv_heads, head_dim), "
            f"got {tuple(cache.shape)}"
        )
    d = KVCache()
    d.data = cache.data_ptr()
    d.dtype = dtype_code(cache.dtype)
    d.num_blocks, d.block_size, d.num_kv_heads, d.head_dim = cache.shape[1:]
    for i in range(5):
        d.stride[i] = cache.stride(i)
    return d


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
