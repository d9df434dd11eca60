"""Random-init dense decoder with the Qwen3 / Llama layer structure.

Follows the reference models layer by layer (src/micro_vllm/models/qwen.py:
20-245, llama.py:20-190):
* pre-norm decoder layers: RMSNorm -> attention -> residual, RMSNorm ->
  SwiGLU MLP -> residual, final RMSNorm;
* attention: q/k/v projections, optional per-head q/k RMSNorm (Qwen3,
  qwen.py:89-90), rotary embedding, the paged-attention operator, o_proj;
* RMSNorm accumulates in float32 and multiplies the weight in the model
  dtype (layers/normalization.py:7-22);
* rotary embedding in float32 with the rotate-half convention
  (layers/rotary_embedding.py:14-52). Angles are computed with the same
  float32 operations from a per-model inverse-frequency table, once per
  step for all layers instead of once per layer; with fused layers, once
  per model for every position up to the engine's maximum length (the same
  elementwise operations give the same values) and gathered by position.

The q/k/v and gate/up projections are stored as single fused weights so that
each is one GEMM; every output column is the same dot product as in the
unfused layers. Weights are drawn from a seeded normal distribution (there is
no checkpoint to load).

With ``fused_layers=True`` the elementwise steps run as the HIP library's
fused kernels (`micro_vllm_amd.layers`): residual add + RMSNorm, q/k norm +
rotary embedding + paged-cache write, SwiGLU, followed by attention over the
cache (`hip_attention_over_cache`), and the embedding lookup fused with the
first input RMSNorm. The torch path stays the restatement the fused kernels
are checked against.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.nn import functional as F

from micro_vllm_amd.attention.attention import AttentionMetadata


@dataclass(frozen=True)
class DecoderConfig:
    """Architecture of the decoder (field names as in HF configs)."""

    num_hidden_layers: int
    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    qk_norm: bool
    rope_theta: float
    tie_word_embeddings: bool
    rms_norm_eps: float = 1e-6

    @staticmethod
    def qwen3_0_6b(**overrides) -> "DecoderConfig":
        """Qwen3-0.6B: 28 layers, hidden 1024, 16/8 heads of 128, qk-norm,
        MLP 3072, vocab 151,936, tied embeddings, rope theta 1e6."""

        values = dict(
            num_hidden_layers=28,
            hidden_size=1024,
            num_attention_heads=16,
            num_key_value_heads=8,
            head_dim=128,
            intermediate_size=3072,
            vocab_size=151_936,
            qk_norm=True,
            rope_theta=1_000_000.0,
            tie_word_embeddings=True,
        )
        values.update(overrides)
        return DecoderConfig(**values)

    @staticmethod
    def llama3_8b(**overrides) -> "DecoderConfig":
        """Llama-3-8B: 32 layers, hidden 4096, 32/8 heads of 128, MLP 14,336,
        vocab 128,256, rope theta 5e5, untied embeddings."""

        values = dict(
            num_hidden_layers=32,
            hidden_size=4096,
            num_attention_heads=32,
            num_key_value_heads=8,
            head_dim=128,
            intermediate_size=14_336,
            vocab_size=128_256,
            qk_norm=False,
            rope_theta=500_000.0,
            tie_word_embeddings=False,
        )
        values.update(overrides)
        return DecoderConfig(**values)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dimension (normalization.py:7-22)."""

    dtype = x.dtype
    x32 = x.to(torch.float32)
    variance = x32.pow(2).mean(dim=-1, keepdim=True)
    return weight * (x32 * torch.rsqrt(variance + eps)).to(dtype)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    first, second = x.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


class DecoderModel:
    """The decoder's weights and forward pass on one device."""

    def __init__(
        self,
        config: DecoderConfig,
        operator,
        *,
        device: torch.device | str,
        dtype: torch.dtype = torch.bfloat16,
        seed: int = 0,
        init_std: float = 0.02,
        lm_head_std: float | None = None,
        fused_layers: bool = False,
    ) -> None:
        self.config = config
        self.operator = operator
        self.fused_layers = fused_layers
        self.device = torch.device(device)
        self.dtype = dtype
        c = config
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def normal(*shape: int, std: float = init_std) -> torch.Tensor:
            return (torch.randn(shape, generator=gen, device=self.device, dtype=torch.float32) * std).to(dtype)

        def ones(n: int) -> torch.Tensor:
            return torch.ones(n, device=self.device, dtype=dtype)

        q_size = c.num_attention_heads * c.head_dim
        kv_size = c.num_key_value_heads * c.head_dim
        self.embed = normal(c.vocab_size, c.hidden_size)
        self.layers = []
        for _ in range(c.num_hidden_layers):
            self.layers.append(
                dict(
                    input_norm=ones(c.hidden_size),
                    # Weights are stored [out, in] like torch Linear; F.linear multiplies x @ W^T.
                    qkv=normal(q_size + 2 * kv_size, c.hidden_size),
                    q_norm=ones(c.head_dim),
                    k_norm=ones(c.head_dim),
                    o=normal(c.hidden_size, q_size),
                    post_norm=ones(c.hidden_size),
                    gate_up=normal(2 * c.intermediate_size, c.hidden_size),
                    down=normal(c.hidden_size, c.intermediate_size),
                )
            )
        self.final_norm = ones(c.hidden_size)
        if c.tie_word_embeddings and lm_head_std is None:
            self.lm_head = self.embed
        else:
            self.lm_head = normal(c.vocab_size, c.hidden_size, std=lm_head_std or init_std)
        indices = torch.arange(0, c.head_dim, 2, dtype=torch.float32, device=self.device)
        self.inverse_frequencies = 1.0 / (c.rope_theta ** (indices / c.head_dim))
        # cos/sin [positions, head_dim] for the fused path (build_rotary_table).
        self.rotary_cos: torch.Tensor | None = None
        self.rotary_sin: torch.Tensor | None = None

    def build_rotary_table(self, num_positions: int) -> None:
        """cos/sin of every position below ``num_positions`` (kept if the
        table already covers them): the fused path then gathers rows by
        position instead of computing a table each step."""

        if self.rotary_cos is not None and self.rotary_cos.shape[0] >= num_positions:
            return
        positions = torch.arange(num_positions, dtype=torch.int64, device=self.device)
        cosine, sine = self.rotary_tables(positions)
        self.rotary_cos = cosine.reshape(num_positions, self.config.head_dim).contiguous()
        self.rotary_sin = sine.reshape(num_positions, self.config.head_dim).contiguous()

    def parameter_count(self) -> int:
        tensors = [self.embed, self.final_norm, *(t for layer in self.layers for t in layer.values())]
        if self.lm_head is not self.embed:
            tensors.append(self.lm_head)
        return sum(t.numel() for t in tensors)

    def rotary_tables(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin of the rotary angles, [tokens, 1, head_dim] in float32."""

        frequencies = torch.outer(positions.to(torch.float32), self.inverse_frequencies)
        angles = torch.cat((frequencies, frequencies), dim=-1).unsqueeze(1)
        return angles.cos(), angles.sin()

    def forward(
        self,
        input_ids: torch.Tensor,
        positions: torch.Tensor,
        kv_caches: list[torch.Tensor],
        metadata: AttentionMetadata,
        placeholder_tokens: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Final hidden states [tokens, hidden] of the flattened batch. An
        input id ``-(1 + r)`` stands for ``placeholder_tokens[r]``."""

        if self.fused_layers:
            return self._forward_fused(input_ids, positions, kv_caches, metadata, placeholder_tokens)
        if placeholder_tokens is not None:
            index = (-input_ids - 1).clamp(min=0)
            input_ids = torch.where(input_ids < 0, placeholder_tokens.index_select(0, index), input_ids)
        c = self.config
        eps = c.rms_norm_eps
        n = input_ids.shape[0]
        q_size = c.num_attention_heads * c.head_dim
        kv_size = c.num_key_value_heads * c.head_dim
        cosine, sine = self.rotary_tables(positions)
        hidden = F.embedding(input_ids, self.embed)
        for layer, cache in zip(self.layers, kv_caches):
            x = rms_norm(hidden, layer["input_norm"], eps)
            qkv = F.linear(x, layer["qkv"])
            q = qkv[:, :q_size].view(n, c.num_attention_heads, c.head_dim)
            k = qkv[:, q_size : q_size + kv_size].view(n, c.num_key_value_heads, c.head_dim)
            v = qkv[:, q_size + kv_size :].view(n, c.num_key_value_heads, c.head_dim)
            if c.qk_norm:
                q = rms_norm(q, layer["q_norm"], eps)
                k = rms_norm(k, layer["k_norm"], eps)
            q32, k32 = q.to(torch.float32), k.to(torch.float32)
            q = (q32 * cosine + _rotate_half(q32) * sine).to(self.dtype)
            k = (k32 * cosine + _rotate_half(k32) * sine).to(self.dtype)
            attention = self.operator(q, k, v, cache, metadata)
            hidden = hidden + F.linear(attention.flatten(1), layer["o"])
            x = rms_norm(hidden, layer["post_norm"], eps)
            gate, up = F.linear(x, layer["gate_up"]).chunk(2, dim=-1)
            hidden = hidden + F.linear(F.silu(gate) * up, layer["down"])
        return rms_norm(hidden, self.final_norm, eps)

    def _forward_fused(
        self,
        input_ids: torch.Tensor,
        positions: torch.Tensor,
        kv_caches: list[torch.Tensor],
        metadata: AttentionMetadata,
        placeholder_tokens: torch.Tensor | None = None,
    ) -> torch.Tensor:
        from micro_vllm_amd import layers
        from micro_vllm_amd.attention.operators.mi355x_paged import AttentionPlan, hip_attention_over_cache

        c = self.config
        eps = c.rms_norm_eps
        n = input_ids.shape[0]
        q_size = c.num_attention_heads * c.head_dim
        kv_size = c.num_key_value_heads * c.head_dim
        if self.rotary_cos is not None:
            cosine, sine, table_positions = self.rotary_cos, self.rotary_sin, positions
        else:
            cosine, sine = self.rotary_tables(positions)
            cosine = cosine.reshape(n, c.head_dim).contiguous()
            sine = sine.reshape(n, c.head_dim).contiguous()
            table_positions = None
        residual, x = layers.embed_rms_norm(
            input_ids, self.embed, self.layers[0]["input_norm"], eps, last_tokens=placeholder_tokens
        )
        # Every layer sees the same batch: its work lists are built once.
        plan = AttentionPlan(metadata, c.num_attention_heads, kv_caches[0])
        for i, (layer, cache) in enumerate(zip(self.layers, kv_caches)):
            qkv = F.linear(x, layer["qkv"])
            q = qkv[:, :q_size].view(n, c.num_attention_heads, c.head_dim)
            k = qkv[:, q_size : q_size + kv_size].view(n, c.num_key_value_heads, c.head_dim)
            v = qkv[:, q_size + kv_size :].view(n, c.num_key_value_heads, c.head_dim)
            q = layers.qk_norm_rope_kv_write(
                q,
                k,
                v,
                layer["q_norm"] if c.qk_norm else None,
                layer["k_norm"] if c.qk_norm else None,
                cosine,
                sine,
                eps,
                cache,
                metadata.slot_mapping,
                positions=table_positions,
            )
            attention = hip_attention_over_cache(q, cache, metadata, plan=plan)
            x = layers.add_rms_norm(F.linear(attention.flatten(1), layer["o"]), layer["post_norm"], eps, residual)
            mlp = F.linear(layers.silu_mul(F.linear(x, layer["gate_up"])), layer["down"])
            next_norm = self.layers[i + 1]["input_norm"] if i + 1 < len(self.layers) else self.final_norm
            x = layers.add_rms_norm(mlp, next_norm, eps, residual)
        return x

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden, self.lm_head)
