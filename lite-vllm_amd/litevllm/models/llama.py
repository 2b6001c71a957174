"""Llama-family decoder (reference models/llama.py:18-224), serving-shaped:
q/k/v are one fused projection and gate/up another (checkpoint tensors are
stacked on load), attention runs through the paged HIP kernels, and the
LM head is applied only to the rows that are sampled."""

from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn as nn

from litevllm import ops
from litevllm.config import ModelConfig
from litevllm.layers.attention import Attention
from litevllm.layers.rotary_emb import RotaryEmbedding, apply_rotary_emb
from litevllm.models.base import BaseModelForCausalLM


# Rows up to which a projection runs on lv_linear (decode-sized batches);
# larger batches (prefill chunks) use the library GEMM.  0 disables it.
DECODE_GEMM_ROWS = int(os.environ.get("LV_DECODE_GEMM_ROWS", "256"))


class Linear(nn.Linear):
    """nn.Linear (the reference's ColumnParallelLinear / RowParallelLinear,
    layers/linear.py:15-65) whose decode-sized calls run on the lv_linear
    MFMA kernel; other shapes, biases and dtypes use the library GEMM."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        m = x.shape[0] if x.dim() == 2 else 0
        if (0 < m <= DECODE_GEMM_ROWS and self.bias is None and x.is_cuda
                and ops.linear_supported(m, self.out_features, self.in_features, x.dtype)):
            return ops.linear(x, self.weight)
        return super().forward(x)


class RMSNorm(nn.Module):
    """RMSNorm with the reference's rounding (fp32 statistics, normalised
    value cast to the weight dtype, then scaled; reference llama.py:18-27),
    run by lv_add_rms_norm.  With `residual`, the residual add of the decoder
    layer is fused in: residual += x (in place), returns (norm(residual),
    residual)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None):
        n = self.weight.shape[0]
        rows = x.reshape(-1, n)
        if residual is None:
            return ops.add_rms_norm(rows, self.weight, self.eps).view(x.shape)
        out = ops.add_rms_norm(rows, self.weight, self.eps, residual=residual)
        return out.view(x.shape), residual


class GatedMLP(nn.Module):
    """down(silu(gate(x)) * up(x)) with gate and up fused (reference llama.py:30-38)."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.intermediate_size = intermediate_size
        self.gate_up_proj = Linear(hidden_size, 2 * intermediate_size, bias=False)
        self.down_proj = Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        m = x.shape[0] if x.dim() == 2 else 0
        if (0 < m <= DECODE_GEMM_ROWS and x.is_cuda and self.gate_up_proj.bias is None
                and ops.linear_supported(m, self.intermediate_size,
                                         self.gate_up_proj.in_features, x.dtype, "silu_mul")):
            # decode-sized: gate|up projection with SiLU * up in its epilogue
            return self.down_proj(ops.linear(x, self.gate_up_proj.weight, activation="silu_mul"))
        return self.down_proj(ops.silu_mul(self.gate_up_proj(x)))


class DecoderAttention(nn.Module):
    """q/k/v projection (+ optional per-head q/k RMSNorm, Qwen3), RoPE,
    paged attention, output projection (reference llama.py:41-99,
    qwen3.py:24-93)."""

    def __init__(self, config: ModelConfig, use_qk_norm: bool) -> None:
        super().__init__()
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = Linear(config.hidden_size, self.q_size + 2 * self.kv_size,
                               bias=config.attention_bias)
        self.o_proj = Linear(self.q_size, config.hidden_size, bias=False)
        self.use_qk_norm = use_qk_norm
        if use_qk_norm:
            self.q_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
            self.k_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(self.head_dim, config.max_position_embeddings,
                                          config.rope_theta, config.rope_scaling)
        self.attn = Attention(self.num_heads, self.head_dim, self.num_kv_heads)

    def forward(self, hidden: torch.Tensor, positions: torch.Tensor, kv_cache, slot_mapping,
                block_table, context_lens, is_prefill, attn_metadata) -> torch.Tensor:
        T = hidden.shape[0]
        qkv = self.qkv_proj(hidden)
        if attn_metadata is not None and kv_cache is not None:
            # engine path: one fused prologue kernel (q/k norm, RoPE, K/V into
            # the paged cache), then attention over the cache
            key_cache, value_cache = kv_cache
            q = ops.qk_norm_rope_cache(
                qkv, self.num_heads, self.num_kv_heads, self.head_dim,
                self.rotary_emb.cos_cached, self.rotary_emb.sin_cached, positions, slot_mapping,
                key_cache, value_cache,
                q_norm_weight=self.q_norm.weight if self.use_qk_norm else None,
                k_norm_weight=self.k_norm.weight if self.use_qk_norm else None,
                eps=self.q_norm.eps if self.use_qk_norm else 1e-6)
            out = self.attn(q, None, None, key_cache, value_cache, block_table, None,
                            context_lens, is_prefill, attn_metadata=attn_metadata)
            return self.o_proj(out.reshape(T, self.q_size))
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = q.reshape(T, self.num_heads, self.head_dim)
        k = k.reshape(T, self.num_kv_heads, self.head_dim)
        v = v.reshape(T, self.num_kv_heads, self.head_dim)
        if self.use_qk_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)
        cos, sin = self.rotary_emb(positions)
        q = apply_rotary_emb(q, cos.unsqueeze(1), sin.unsqueeze(1))
        k = apply_rotary_emb(k, cos.unsqueeze(1), sin.unsqueeze(1))
        key_cache, value_cache = kv_cache if kv_cache is not None else (None, None)
        out = self.attn(q, k, v, key_cache, value_cache, block_table, slot_mapping, context_lens,
                        is_prefill, attn_metadata=attn_metadata)
        return self.o_proj(out.reshape(T, self.q_size))


class DecoderLayer(nn.Module):
    def __init__(self, config: ModelConfig, use_qk_norm: bool) -> None:
        super().__init__()
        self.self_attn = DecoderAttention(config, use_qk_norm)
        self.mlp = GatedMLP(config.hidden_size, config.intermediate_size)
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, hidden, residual, positions, kv_cache, slot_mapping, block_table,
                context_lens, is_prefill, attn_metadata):
        """Returns (mlp output, residual stream).  The reference's
        `residual + hidden` adds (qwen3.py:131-140) happen inside the next
        RMSNorm call, so the residual stream carries the same bf16 sums."""
        if residual is None:
            residual = hidden
            hidden = self.input_layernorm(hidden)
        else:
            hidden, residual = self.input_layernorm(hidden, residual)
        hidden = self.self_attn(hidden, positions, kv_cache, slot_mapping, block_table,
                                context_lens, is_prefill, attn_metadata)
        hidden, residual = self.post_attention_layernorm(hidden, residual)
        return self.mlp(hidden), residual


class DecoderModel(nn.Module):
    def __init__(self, config: ModelConfig, use_qk_norm: bool) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([DecoderLayer(config, use_qk_norm)
                                     for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, input_ids, positions, kv_caches, slot_mapping, block_tables, context_lens,
                is_prefill, attn_metadata):
        """Returns (last layer's MLP output, residual stream); the final
        residual add + norm is left to the caller so it can run on the
        sampled rows only."""
        hidden = self.embed_tokens(input_ids)
        residual = None
        for i, layer in enumerate(self.layers):
            kv = kv_caches[i] if kv_caches is not None else None
            hidden, residual = layer(hidden, residual, positions, kv, slot_mapping, block_tables,
                                     context_lens, is_prefill, attn_metadata)
        return hidden, residual


class LlamaForCausalLM(BaseModelForCausalLM):
    @staticmethod
    def _qk_norm(config: ModelConfig) -> bool:
        return False

    def __init__(self, config: ModelConfig) -> None:
        super().__init__(config)
        self.model = DecoderModel(config, self._qk_norm(config))
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids, positions, kv_caches=None, slot_mapping=None, block_tables=None,
                context_lens=None, is_prefill=True, attn_metadata=None, logits_indices=None):
        hidden, residual = self.model(input_ids, positions, kv_caches, slot_mapping,
                                      block_tables, context_lens, is_prefill, attn_metadata)
        if logits_indices is not None:   # norm and LM head on the sampled rows only
            hidden = hidden.index_select(0, logits_indices)
            residual = residual.index_select(0, logits_indices)
        hidden, _ = self.model.norm(hidden, residual)
        return self.lm_head(hidden)

    # -- checkpoint loading ------------------------------------------------
    _STACKED = {"q_proj": ("qkv_proj", 0), "k_proj": ("qkv_proj", 1), "v_proj": ("qkv_proj", 2),
                "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1)}

    @torch.no_grad()
    def load_weights(self, weights: dict[str, torch.Tensor]) -> None:
        """HF names -> fused parameters (q/k/v and gate/up stacked on dim 0)."""
        params = dict(self.named_parameters())
        pieces: dict[str, dict[int, torch.Tensor]] = {}
        for name, w in weights.items():
            name = name.replace(".linear.", ".")
            parts = name.split(".")
            if len(parts) >= 2 and parts[-2] in self._STACKED:
                fused, idx = self._STACKED[parts[-2]]
                key = ".".join(parts[:-2] + [fused, parts[-1]])
                pieces.setdefault(key, {})[idx] = w
            elif name in params and params[name].shape == w.shape:
                params[name].copy_(w)
        for key, parts in pieces.items():
            if key in params:
                stacked = torch.cat([parts[i] for i in sorted(parts)], dim=0)
                if stacked.shape == params[key].shape:
                    params[key].copy_(stacked)
