"""fp32 CPU restatement of the reference's paged attention (test oracle).

decode_attention restates Attention._decode_fast (reference
litevllm/layers/attention.py:91-139) op for op: gather K/V for
max_s = block_table.shape[1] * bs logical positions through the block table
(111-119), GQA view q -> (B, Hkv, G, D) (124), scores * scale (129),
mask pos < context_len -> -inf (132-133), fp32 softmax (135), P.V (138).
Run on fp32 tensors (the reference CPU path is fp32, config/config.py:120)
it is also the CPU baseline that bench.py times.

chunk_attention is the causal attention of a prefill chunk at an offset over
the paged cache.  The reference has no such path (its _prefill,
attention.py:141-151, attends only the forward's own tokens); it reduces to
_prefill at offset 0 and to _decode_fast for a 1-token chunk, which is how
the tests pin it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def decode_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                     block_table: torch.Tensor, context_lens: torch.Tensor,
                     scale: float) -> torch.Tensor:
    """query [B, H, D] -> out [B, H, D], all fp32 on the CPU."""
    B, H, D = query.shape
    block_size = key_cache.shape[1]
    H_kv = key_cache.shape[2]
    G = H // H_kv
    max_s = block_table.shape[1] * block_size
    positions = torch.arange(max_s).unsqueeze(0)
    b_idx = torch.gather(block_table.to(torch.long), 1, (positions // block_size).expand(B, max_s))
    b_off = (positions % block_size).expand(B, max_s)
    k_hist = key_cache[b_idx, b_off]          # (B, max_s, H_kv, D)
    v_hist = value_cache[b_idx, b_off]
    q = query.view(B, H_kv, G, D)
    k = k_hist.permute(0, 2, 1, 3).contiguous()
    v = v_hist.permute(0, 2, 1, 3).contiguous()
    attn = torch.einsum("bhgd,bhsd->bhgs", q, k) * scale
    mask = positions < context_lens.unsqueeze(1).to(positions.dtype)
    attn = attn.masked_fill(~mask.view(B, 1, 1, max_s), float("-inf"))
    attn = F.softmax(attn, dim=-1, dtype=torch.float32).to(query.dtype)
    out = torch.einsum("bhgs,bhsd->bhgd", attn, v)
    return out.reshape(B, H, D)


def gather_sequence(cache: torch.Tensor, block_row: torch.Tensor, n_tokens: int) -> torch.Tensor:
    """Tokens 0..n_tokens-1 of one sequence from a paged cache -> [n, Hkv, D]."""
    bs = cache.shape[1]
    pos = torch.arange(n_tokens)
    blocks = block_row.to(torch.long)[pos // bs]
    return cache[blocks, pos % bs]


def chunk_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    block_row: torch.Tensor, context_len: int, scale: float) -> torch.Tensor:
    """Causal attention of the last q = query.shape[0] positions of a sequence.

    query [q, H, D] holds positions context_len - q .. context_len - 1; each
    attends keys 0..its own position from the paged cache.  fp32 CPU.
    """
    q_len, H, D = query.shape
    H_kv = key_cache.shape[2]
    G = H // H_kv
    # inputs of any dtype are upcast; all arithmetic is fp32
    k = gather_sequence(key_cache, block_row, context_len).float()   # [c, Hkv, D]
    v = gather_sequence(value_cache, block_row, context_len).float()
    k = k.repeat_interleave(G, dim=1).permute(1, 0, 2)          # [H, c, D]
    v = v.repeat_interleave(G, dim=1).permute(1, 0, 2)
    qh = query.float().permute(1, 0, 2)                         # [H, q, D]
    scores = torch.matmul(qh, k.transpose(1, 2)) * scale        # [H, q, c]
    q_pos = torch.arange(context_len - q_len, context_len).unsqueeze(1)
    k_pos = torch.arange(context_len).unsqueeze(0)
    scores = scores.masked_fill((k_pos > q_pos).unsqueeze(0), float("-inf"))
    p = F.softmax(scores, dim=-1, dtype=torch.float32)
    return torch.matmul(p, v).permute(1, 0, 2).contiguous()     # [q, H, D]


def mixed_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    block_tables: torch.Tensor, cu_seqlens: torch.Tensor,
                    context_lens: torch.Tensor, scale: float) -> torch.Tensor:
    """Every sequence of a packed mixed batch through chunk_attention (fp32 out)."""
    out = torch.empty(query.shape, dtype=torch.float32)
    cu = cu_seqlens.tolist()
    ctx = context_lens.tolist()
    for i in range(len(ctx)):
        a, b = cu[i], cu[i + 1]
        out[a:b] = chunk_attention(query[a:b], key_cache, value_cache, block_tables[i], ctx[i],
                                   scale)
    return out
