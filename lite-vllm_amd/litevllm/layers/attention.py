"""PagedAttention / Attention with the reference's call signatures
(layers/attention.py:14-151), running on the HIP kernels.

``Attention.forward(query, key, value, key_cache, value_cache, block_table,
slot_mapping, context_lens, is_prefill=True)`` keeps the reference meaning
when called without metadata: scatter the new K/V by slot_mapping, then
either causal attention over this forward's own tokens (prefill,
attention.py:141-151) or paged decode over the block tables (91-139).  The
engine passes ``attn_metadata`` instead, describing a mixed batch (decodes
first, then prefill chunks at any offset) that one lv_paged_attention call
serves.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn

from .. import ops


@dataclass
class AttentionMetadata:
    """Per-step batch description shared by every layer (built on the GPU by
    the packing kernel)."""
    block_tables: torch.Tensor   # int32 [B, max_blocks]
    context_lens: torch.Tensor   # int32 [B]
    cu_seqlens: torch.Tensor     # int32 [B+1]
    num_decodes: int             # leading 1-token sequences
    max_query_len: int
    workspace: Optional[torch.Tensor] = None   # attention scratch owned by a HIP graph
    # decode rows' shared prefixes, read once per group (lv_paged_attention_prefix)
    prefix: Optional[ops.PrefixPlan] = None
    prefix_workspace: Optional[torch.Tensor] = None


class PagedAttention:
    @staticmethod
    def write_to_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                       value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """key_cache[slot // bs, slot % bs] = key (reference attention.py:17-33)."""
        ops.kv_scatter(key, value, key_cache, value_cache, slot_mapping)


class Attention(nn.Module):
    def __init__(self, num_heads: int, head_dim: int, num_kv_heads: int,
                 scale: Optional[float] = None) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.num_kv_groups = num_heads // num_kv_heads
        self.scale = scale or (1.0 / (head_dim ** 0.5))

    def forward(self, query, key, value, key_cache, value_cache, block_table, slot_mapping,
                context_lens, is_prefill=True, attn_metadata: Optional[AttentionMetadata] = None):
        if slot_mapping is not None and key_cache is not None:
            ops.kv_scatter(key, value, key_cache, value_cache, slot_mapping)
        if attn_metadata is not None:
            m = attn_metadata
            return ops.paged_attention(query, key_cache, value_cache, m.block_tables,
                                       m.context_lens, scale=self.scale, cu_seqlens=m.cu_seqlens,
                                       num_decodes=m.num_decodes, max_query_len=m.max_query_len,
                                       workspace=m.workspace, prefix=m.prefix,
                                       prefix_workspace=m.prefix_workspace)
        if is_prefill:
            return self._prefill(query, key, value)
        return ops.paged_attention(query, key_cache, value_cache, block_table, context_lens,
                                   scale=self.scale)

    def _prefill(self, query, key, value):
        """Causal attention over this forward's T tokens only (one sequence at
        offset 0, the reference's _prefill semantics): the new K/V are laid
        out as a temporary paged cache of ceil(T/16) blocks."""
        T = query.shape[0]
        bs = 16
        nb = (T + bs - 1) // bs
        kt = torch.zeros((nb, bs, self.num_kv_heads, self.head_dim), dtype=key.dtype,
                         device=key.device)
        vt = torch.zeros_like(kt)
        kt.view(nb * bs, self.num_kv_heads, self.head_dim)[:T] = key
        vt.view(nb * bs, self.num_kv_heads, self.head_dim)[:T] = value
        dev = query.device
        bt = torch.arange(nb, dtype=torch.int32, device=dev).unsqueeze(0)
        ctx = torch.tensor([T], dtype=torch.int32, device=dev)
        cu = torch.tensor([0, T], dtype=torch.int32, device=dev)
        return ops.paged_attention(query, kt, vt, bt, ctx, scale=self.scale, cu_seqlens=cu,
                                   num_decodes=0, max_query_len=T)
