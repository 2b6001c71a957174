"""Seeded synthetic inputs for the hot-path configurations.

All randomness comes from a CPU ``torch.Generator`` so the GPU run and the
CPU checks see identical bits; tensors are returned on the CPU and moved by
the caller.  Shapes follow the benchmark configurations: paged decode at the
Qwen3-0.6B attention shape (16 q heads, 8 kv heads, head_dim 128,
block_size 16), the mixed chunked-prefill step, and the fused sampler over a
151936-wide vocabulary.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class PagedBatch:
    query: torch.Tensor          # [T, H, D]
    key_cache: torch.Tensor      # [N, bs, Hkv, D]
    value_cache: torch.Tensor
    block_tables: torch.Tensor   # int32 [B, max_blocks]
    context_lens: torch.Tensor   # int32 [B]
    cu_seqlens: torch.Tensor     # int32 [B+1]
    num_decodes: int
    max_query_len: int
    scale: float

    def to(self, device) -> "PagedBatch":
        return PagedBatch(*(getattr(self, f).to(device) if isinstance(getattr(self, f), torch.Tensor)
                            else getattr(self, f) for f in self.__dataclass_fields__))

    def kv_bytes_read(self) -> int:
        """Algorithmic K+V bytes one decode pass reads (each live token once)."""
        hkv, d = self.key_cache.shape[2], self.key_cache.shape[3]
        es = self.key_cache.element_size()
        return int(self.context_lens.to(torch.int64).sum()) * hkv * d * es * 2


def paged_decode(seed: int = 0, num_seqs: int = 256, num_heads: int = 16, num_kv_heads: int = 8,
                 head_dim: int = 128, block_size: int = 16, ctx_lo: int = 128,
                 ctx_hi: int = 2048, dtype: torch.dtype = torch.bfloat16,
                 scale_inputs: bool = True, tail_fill: float | None = None,
                 ctx_head: list[int] | None = None) -> PagedBatch:
    """Config 2: B decodes, ctx ~ U[ctx_lo, ctx_hi], blocks = seeded permutation
    of a pool that exactly fits all sequences; q, k, v ~ N(0,1) (/sqrt(D) if
    scale_inputs).  tail_fill writes that value into every cache slot past a
    sequence's context (to prove masked slots are never read); ctx_head
    overrides the first context lengths (edge cases)."""
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (num_seqs,), generator=g)
    if ctx_head:
        ctx[:len(ctx_head)] = torch.tensor(ctx_head)
    nb = (ctx + block_size - 1) // block_size
    pool = int(nb.sum())
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    max_blocks = int(nb.max())
    tables = torch.zeros(num_seqs, max_blocks, dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb.tolist()):
        tables[i, :n] = perm[off:off + n]
        off += n
    s = 1.0 / math.sqrt(head_dim) if scale_inputs else 1.0
    q = (torch.randn(num_seqs, num_heads, head_dim, generator=g) * s).to(dtype)
    kc = (torch.randn(pool, block_size, num_kv_heads, head_dim, generator=g) * s).to(dtype)
    vc = (torch.randn(pool, block_size, num_kv_heads, head_dim, generator=g) * s).to(dtype)
    if tail_fill is not None:
        for i, c in enumerate(ctx.tolist()):
            last = int(tables[i, (c - 1) // block_size])
            r = c % block_size
            if r:
                kc[last, r:] = tail_fill
                vc[last, r:] = tail_fill
    return PagedBatch(q, kc, vc, tables, ctx.to(torch.int32),
                      torch.arange(num_seqs + 1, dtype=torch.int32), num_seqs, 1,
                      1.0 / math.sqrt(head_dim))


@dataclass
class MixedStep:
    """One mixed chunked-prefill step before packing/scatter."""
    batch: PagedBatch            # query/caches/tables/ctx/cu for the attention
    key: torch.Tensor            # [T, Hkv, D] new keys of this step
    value: torch.Tensor
    slot_mapping: torch.Tensor   # int64 [T]
    positions: torch.Tensor      # int64 [T]
    descs: torch.Tensor          # int32 [B, 6] lv_seq_desc rows
    block_ids: torch.Tensor      # int32 flat block tables
    token_ids: torch.Tensor      # int64 flat input ids


def mixed_step(seed: int = 0, num_decodes: int = 192, dec_lo: int = 256, dec_hi: int = 4096,
               num_chunks: int = 15, chunk_len: int = 512, off_lo: int = 0, off_hi: int = 3072,
               num_heads: int = 16, num_kv_heads: int = 8, head_dim: int = 128,
               block_size: int = 16, num_cache_slots: int = 200_000, vocab: int = 151936,
               dtype: torch.dtype = torch.bfloat16) -> MixedStep:
    """Config 3.  Blocks that receive this step's writes are distinct across
    sequences; read-only history blocks are drawn (with repetition) from the
    rest of the pool, since the cache cannot hold every history distinctly."""
    g = torch.Generator().manual_seed(seed)
    bs = block_size
    n_blocks = num_cache_slots // bs
    dec_ctx = torch.randint(dec_lo, dec_hi + 1, (num_decodes,), generator=g).tolist()
    offs = torch.randint(off_lo, off_hi + 1, (num_chunks,), generator=g).tolist()
    # (num_computed, query_len) per sequence, decodes first
    seqs = [(c - 1, 1) for c in dec_ctx] + [(o, chunk_len) for o in offs]
    write_sets = []
    for n, q in seqs:
        write_sets.append(list(range(n // bs, (n + q - 1) // bs + 1)))
    n_write = sum(len(w) for w in write_sets)
    perm = torch.randperm(n_blocks, generator=g)
    write_pool = perm[:n_write].tolist()
    hist_pool = perm[n_write:]
    tables, flat, cursor = [], [], 0
    for (n, q), ws in zip(seqs, write_sets):
        nb = (n + q + bs - 1) // bs
        row = hist_pool[torch.randint(0, len(hist_pool), (nb,), generator=g)].tolist()
        for lb in ws:
            row[lb] = write_pool[cursor]
            cursor += 1
        tables.append(row)
    B = len(seqs)
    max_blocks = max(len(r) for r in tables)
    bt = torch.zeros(B, max_blocks, dtype=torch.int32)
    descs = []
    tok_count = 0
    for i, ((n, q), row) in enumerate(zip(seqs, tables)):
        bt[i, :len(row)] = torch.tensor(row, dtype=torch.int32)
        descs.append([n, q, len(row), len(flat), tok_count, -1])
        flat.extend(row)
        tok_count += q
    T = tok_count
    qlens = torch.tensor([q for _, q in seqs])
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(qlens, 0)
    ctx = torch.tensor([n + q for n, q in seqs], dtype=torch.int32)
    positions = torch.cat([torch.arange(n, n + q) for n, q in seqs])
    seq_of = torch.repeat_interleave(torch.arange(B), qlens)
    blk = bt[seq_of, positions // bs].to(torch.int64)
    slots = blk * bs + positions % bs
    kc = torch.randn(n_blocks, bs, num_kv_heads, head_dim, generator=g).to(dtype)
    vc = torch.randn(n_blocks, bs, num_kv_heads, head_dim, generator=g).to(dtype)
    query = torch.randn(T, num_heads, head_dim, generator=g).to(dtype)
    key = torch.randn(T, num_kv_heads, head_dim, generator=g).to(dtype)
    value = torch.randn(T, num_kv_heads, head_dim, generator=g).to(dtype)
    token_ids = torch.randint(0, vocab, (T,), generator=g)
    batch = PagedBatch(query, kc, vc, bt, ctx, cu, num_decodes, chunk_len if num_chunks else 1,
                       1.0 / math.sqrt(head_dim))
    return MixedStep(batch, key, value, slots, positions,
                     torch.tensor(descs, dtype=torch.int32), torch.tensor(flat, dtype=torch.int32),
                     token_ids)


@dataclass
class SamplerBatch:
    logits: torch.Tensor       # [B, V]
    temperature: torch.Tensor  # float32 [B] (0 = greedy)
    uniform: torch.Tensor      # float32 [B]
    planted: torch.Tensor      # int64 [B] index of the planted maximum


def sampler_batch(seed: int = 0, rows: int = 256, vocab: int = 151936, std: float = 4.0,
                  margin: float = 0.5, dtype: torch.dtype = torch.bfloat16) -> SamplerBatch:
    """Config 4: logits ~ N(0, std^2) in dtype with a planted row maximum
    (row max excluding it + margin, after rounding); first half greedy, second
    half T ~ U[0.5, 1.0]; uniforms supplied."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, vocab, generator=g) * std).to(dtype)
    planted = torch.randint(0, vocab, (rows,), generator=g)
    xf = x.float()
    idx = torch.arange(rows)
    xf[idx, planted] = float("-inf")
    rowmax = xf.max(dim=1).values
    x[idx, planted] = (rowmax + margin).to(dtype)
    temp = torch.zeros(rows, dtype=torch.float32)
    half = rows // 2
    temp[half:] = 0.5 + 0.5 * torch.rand(rows - half, generator=g)
    uni = torch.rand(rows, generator=g)
    return SamplerBatch(x, temp, uni.to(torch.float32), planted)


# -- config 5: end-to-end serving -------------------------------------------

QWEN3_06B_SHAPE = dict(
    model_type="qwen3", vocab_size=151936, hidden_size=1024, num_hidden_layers=28,
    num_attention_heads=16, num_key_value_heads=8, head_dim=128, intermediate_size=3072,
    rope_theta=1e6, rms_norm_eps=1e-6, max_position_embeddings=40960,
    tie_word_embeddings=False)


def e2e_prompts(seed: int = 0, num_seqs: int = 256, len_lo: int = 100, len_hi: int = 1024,
                vocab: int = 151936, shared_len: int = 512, num_shared: int = 128,
                min_shared_total: int = 528) -> tuple[list[list[int]], list[int]]:
    """Config 5 prompts: lengths U[len_lo, len_hi], ids U[0, vocab); a seeded
    choice of num_shared sequences starts with one common shared_len-token
    prefix, and those get length max(drawn, min_shared_total) so that the
    prefix is followed by at least one block of their own.  Returns
    (prompts, indices of the sharing sequences)."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(len_lo, len_hi + 1, (num_seqs,), generator=g).tolist()
    shared = torch.randint(0, vocab, (shared_len,), generator=g).tolist()
    sharers = sorted(torch.randperm(num_seqs, generator=g)[:num_shared].tolist())
    is_sharer = set(sharers)
    prompts = []
    for i, n in enumerate(lens):
        if i in is_sharer:
            n = max(n, min_shared_total)
            tail = torch.randint(0, vocab, (n - shared_len,), generator=g).tolist()
            prompts.append(shared + tail)
        else:
            prompts.append(torch.randint(0, vocab, (n,), generator=g).tolist())
    return prompts, sharers
