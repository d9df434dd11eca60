"""Fused decoder-layer steps around the attention call, on the HIP library.

torch-facing wrappers of `mvllm_add_rms_norm`, `mvllm_qk_norm_rope_kv_write`,
`mvllm_silu_mul`, `mvllm_embed_rms_norm` and `mvllm_argmax_rows`
(include/mvllm_amd.h). They replace, for bf16/fp16 activations on the GPU:
* RMSNorm (src/micro_vllm/layers/normalization.py:7-22) and the residual
  adds of the decoder layer (models/qwen.py:136-156, llama.py:120-140);
* Qwen3's per-head q/k RMSNorm and the rotary embedding (models/qwen.py:
  89-91, layers/rotary_embedding.py:14-52) together with the paged-cache
  write (attention/operators/reference.py:84-98);
* the SwiGLU activation (layers/mlp.py:10-21);
* the token embedding with the first layer's input RMSNorm (models/qwen.py:
  227, :144);
* greedy sampling, the per-row argmax (sampling/sampler.py:24-31, 39-46).
There is no fallback: the HIP library must be present.
"""

from __future__ import annotations

import torch

from micro_vllm_amd import _native


def _dtype(t: torch.Tensor) -> int:
    if t.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"fused layer ops support bfloat16 and float16, got {t.dtype}")
    if t.device.type != "cuda":
        raise RuntimeError("fused layer ops require GPU tensors")
    return _native.dtype_code(t.dtype)


def add_rms_norm(
    x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None
) -> torch.Tensor:
    """RMSNorm of ``residual + x`` (``residual`` is updated in place) or of ``x``."""

    code = _dtype(x)
    if x.dim() != 2 or x.stride(1) != 1 or weight.shape != (x.shape[1],) or weight.dtype != x.dtype:
        raise ValueError("add_rms_norm expects x [rows, dim] with unit column stride and weight [dim]")
    if residual is not None and (residual.shape != x.shape or residual.stride(1) != 1 or residual.dtype != x.dtype):
        raise ValueError("residual must match x")
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    _native.check(
        _native.load().mvllm_add_rms_norm(
            x.data_ptr(),
            x.stride(0),
            residual.data_ptr() if residual is not None else None,
            residual.stride(0) if residual is not None else 0,
            weight.contiguous().data_ptr(),
            out.data_ptr(),
            out.stride(0),
            x.shape[0],
            x.shape[1],
            eps,
            code,
            _native.stream_handle(x.device),
        ),
        "mvllm_add_rms_norm",
    )
    return out


def qk_norm_rope_kv_write(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    q_weight: torch.Tensor | None,
    k_weight: torch.Tensor | None,
    cos: torch.Tensor | None,
    sin: torch.Tensor | None,
    eps: float,
    layer_kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    positions: torch.Tensor | None = None,
) -> torch.Tensor:
    """Normalised, rotated query [tokens, Hq, 128]; key/value go into the cache.

    Without ``positions`` the cos/sin tables hold one row per token; with
    them, one row per position (token t uses row ``positions[t]``; a position
    outside the table rotates to NaN)."""

    _dtype(query)
    rows = query.shape[0] if positions is None else (cos.shape[0] if cos is not None else 0)
    for name, t in (("cos", cos), ("sin", sin)):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or t.shape != (rows, 128)):
            raise ValueError(f"{name} must be a contiguous float32 [{'tokens' if positions is None else 'positions'}, 128] table")
    if positions is not None:
        if cos is None or positions.dtype != torch.int64 or positions.numel() != query.shape[0]:
            raise ValueError("positions need cos/sin tables and one int64 entry per token")
        positions = positions.contiguous()
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != query.shape[0]:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    q_out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    _native.check(
        _native.load().mvllm_qk_norm_rope_kv_write(
            _native.tensor3(query),
            _native.tensor3(key),
            _native.tensor3(value),
            q_weight.contiguous().data_ptr() if q_weight is not None else None,
            k_weight.contiguous().data_ptr() if k_weight is not None else None,
            cos.data_ptr() if cos is not None else None,
            sin.data_ptr() if sin is not None else None,
            positions.data_ptr() if positions is not None else None,
            rows if positions is not None else 0,
            eps,
            q_out.data_ptr(),
            _native.kv_cache(layer_kv_cache),
            slot_mapping.contiguous().data_ptr(),
            _native.stream_handle(query.device),
        ),
        "mvllm_qk_norm_rope_kv_write",
    )
    return q_out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for rows [gate | up]."""

    code = _dtype(gate_up)
    if gate_up.dim() != 2 or gate_up.stride(1) != 1 or gate_up.shape[1] % 4:
        raise ValueError("silu_mul expects [rows, 2 * intermediate] with unit column stride")
    inter = gate_up.shape[1] // 2
    out = torch.empty((gate_up.shape[0], inter), dtype=gate_up.dtype, device=gate_up.device)
    _native.check(
        _native.load().mvllm_silu_mul(
            gate_up.data_ptr(),
            gate_up.stride(0),
            out.data_ptr(),
            out.stride(0),
            gate_up.shape[0],
            inter,
            code,
            _native.stream_handle(gate_up.device),
        ),
        "mvllm_silu_mul",
    )
    return out


def embed_rms_norm(
    ids: torch.Tensor,
    embedding: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    last_tokens: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(embedding rows of ``ids``, their RMSNorm): the residual stream and the
    first layer's input. An id ``-(1 + r)`` stands for ``last_tokens[r]``;
    ids outside the vocabulary give zero rows."""

    code = _dtype(embedding)
    if ids.dtype != torch.int64 or ids.dim() != 1:
        raise ValueError("ids must be a 1-D int64 tensor")
    if embedding.dim() != 2 or embedding.stride(1) != 1 or weight.shape != (embedding.shape[1],) or weight.dtype != embedding.dtype:
        raise ValueError("embed_rms_norm expects embedding [vocab, dim] with unit column stride and weight [dim]")
    if last_tokens is not None and (last_tokens.dtype != torch.int64 or not last_tokens.is_contiguous()):
        raise ValueError("last_tokens must be a contiguous int64 tensor")
    n, dim = ids.shape[0], embedding.shape[1]
    residual = torch.empty((n, dim), dtype=embedding.dtype, device=embedding.device)
    out = torch.empty_like(residual)
    ids = ids.contiguous()
    _native.check(
        _native.load().mvllm_embed_rms_norm(
            ids.data_ptr(),
            n,
            last_tokens.data_ptr() if last_tokens is not None else None,
            last_tokens.numel() if last_tokens is not None else 0,
            embedding.data_ptr(),
            embedding.shape[0],
            embedding.stride(0),
            weight.contiguous().data_ptr(),
            residual.data_ptr(),
            residual.stride(0),
            out.data_ptr(),
            out.stride(0),
            dim,
            eps,
            code,
            _native.stream_handle(embedding.device),
        ),
        "mvllm_embed_rms_norm",
    )
    return residual, out


def argmax_rows(logits: torch.Tensor, copy_into: torch.Tensor | None = None) -> torch.Tensor:
    """``logits.argmax(dim=-1)`` for [rows, vocab] logits (int64 [rows]);
    ``copy_into[:rows]`` receives the same indices."""

    if logits.device.type != "cuda":
        raise RuntimeError("argmax_rows requires GPU tensors")
    if logits.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"argmax_rows supports bfloat16, float16 and float32, got {logits.dtype}")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("argmax_rows expects [rows, vocab] logits with unit column stride")
    rows = logits.shape[0]
    if copy_into is not None and (copy_into.dtype != torch.int64 or not copy_into.is_contiguous() or copy_into.numel() < rows):
        raise ValueError("copy_into must be a contiguous int64 tensor with a slot per row")
    out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    _native.check(
        _native.load().mvllm_argmax_rows(
            logits.data_ptr(),
            rows,
            logits.shape[1],
            logits.stride(0),
            _native.dtype_code(logits.dtype),
            out.data_ptr(),
            copy_into.data_ptr() if copy_into is not None else None,
            _native.stream_handle(logits.device),
        ),
        "mvllm_argmax_rows",
    )
    return out
