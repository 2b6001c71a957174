"""CPU restatement of the reference's per-layer elementwise ops (test
oracle for lv_add_rms_norm, lv_qk_norm_rope_cache and lv_silu_mul).

Each function runs the reference's own torch op sequence on CPU tensors of
the model dtype, so every intermediate is rounded where the reference
rounds it:
  rms_norm        LlamaRMSNorm.forward            models/llama.py:24-27
  add_rms_norm    residual add + RMSNorm          models/qwen3.py:131-140
  rope            apply_rotary_emb                layers/rotary_emb.py:104-117
  qk_norm_rope_cache  q/k norm + RoPE + cache write  models/qwen3.py:75-84,
                                                  layers/attention.py:79-84
  silu_mul        F.silu(gate) * up               models/llama.py:37-38
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    variance = x.float().pow(2).mean(-1, keepdim=True)
    y = x * torch.rsqrt(variance + eps)          # promoted to fp32
    return weight * y.to(weight.dtype)


def add_rms_norm(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor,
                 eps: float) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """(norm(s), s) with s = x + residual (model dtype), or s = x."""
    s = x if residual is None else residual + x
    return rms_norm(s, weight, eps), (None if residual is None else s)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., D]; cos/sin [..., D/2] broadcastable (rows of the cache)."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def qk_norm_rope_cache(qkv: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int,
                       cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                       positions: torch.Tensor, slot_mapping: torch.Tensor,
                       key_cache: torch.Tensor, value_cache: torch.Tensor,
                       q_norm_weight: Optional[torch.Tensor], k_norm_weight: Optional[torch.Tensor],
                       eps: float) -> torch.Tensor:
    """Returns q [T, H, D]; writes K/V rows into the caches ([N, bs, Hkv, D])
    at slot_mapping, skipping slots < 0."""
    H, Hkv, D = num_heads, num_kv_heads, head_dim
    T = qkv.shape[0]
    q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
    q, k, v = q.reshape(T, H, D), k.reshape(T, Hkv, D), v.reshape(T, Hkv, D)
    if q_norm_weight is not None:
        q = rms_norm(q, q_norm_weight, eps)
    if k_norm_weight is not None:
        k = rms_norm(k, k_norm_weight, eps)
    cos = cos_cache[positions].unsqueeze(1)
    sin = sin_cache[positions].unsqueeze(1)
    q = rope(q, cos, sin)
    k = rope(k, cos, sin)
    keep = slot_mapping >= 0
    flat_k = key_cache.view(-1, Hkv, D)
    flat_v = value_cache.view(-1, Hkv, D)
    flat_k[slot_mapping[keep]] = k[keep].to(key_cache.dtype)
    flat_v[slot_mapping[keep]] = v[keep]
    return q.to(qkv.dtype)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    gate, up = gate_up.chunk(2, dim=-1)
    return F.silu(gate) * up
