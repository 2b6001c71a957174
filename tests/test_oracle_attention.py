"""Pins of the attention oracle (CPU): float64 brute force, torch SDPA,
closed-form special cases, chunk/decode/prefill consistency."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import chunk_attention, decode_attention, gather_sequence, mixed_attention


def _paged(rng_seed, B, H, Hkv, D, bs, ctx, extra_blocks=3):
    g = torch.Generator().manual_seed(rng_seed)
    nb = [(c + bs - 1) // bs for c in ctx]
    pool = sum(nb) + extra_blocks
    perm = torch.randperm(pool, generator=g)
    mb = max(nb)
    table = torch.zeros(B, mb, dtype=torch.int32)
    off = 0
    for i, n in enumerate(nb):
        table[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kc = torch.randn(pool, bs, Hkv, D, generator=g)
    vc = torch.randn(pool, bs, Hkv, D, generator=g)
    q = torch.randn(B, H, D, generator=g)
    return q, kc, vc, table, torch.tensor(ctx, dtype=torch.int32)


def _brute_force(q, kc, vc, table, ctx, scale):
    """float64 Python loops over tokens: softmax(q.k*scale) V per head."""
    B, H, D = q.shape
    bs, Hkv = kc.shape[1], kc.shape[2]
    G = H // Hkv
    out = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            kh = h // G
            scores = []
            for t in range(int(ctx[b])):
                blk = int(table[b, t // bs])
                k = kc[blk, t % bs, kh].double().numpy()
                scores.append(float(np.dot(q[b, h].double().numpy(), k)) * scale)
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            z = sum(w)
            for t, wt in enumerate(w):
                blk = int(table[b, t // bs])
                out[b, h] += (wt / z) * vc[blk, t % bs, kh].double().numpy()
    return out


@pytest.mark.parametrize("G", [1, 2, 4])
def test_decode_matches_float64_brute_force(G):
    Hkv, D, bs = 2, 16, 4
    ctx = [1, 3, 4, 5, 13]
    q, kc, vc, table, ctx_t = _paged(1, len(ctx), Hkv * G, Hkv, D, bs, ctx)
    scale = 1 / math.sqrt(D)
    got = decode_attention(q, kc, vc, table, ctx_t, scale).double().numpy()
    ref = _brute_force(q, kc, vc, table, ctx_t, scale)
    assert np.abs(got - ref).max() < 1e-5


def test_decode_matches_sdpa_per_sequence():
    H, Hkv, D, bs = 8, 4, 32, 16
    ctx = [1, 15, 16, 17, 100, 257]
    q, kc, vc, table, ctx_t = _paged(2, len(ctx), H, Hkv, D, bs, ctx)
    scale = 1 / math.sqrt(D)
    got = decode_attention(q, kc, vc, table, ctx_t, scale)
    for b, c in enumerate(ctx):
        k = gather_sequence(kc, table[b], c).repeat_interleave(H // Hkv, 1).permute(1, 0, 2)
        v = gather_sequence(vc, table[b], c).repeat_interleave(H // Hkv, 1).permute(1, 0, 2)
        ref = F.scaled_dot_product_attention(q[b].unsqueeze(1).double(), k.double(), v.double())
        assert torch.allclose(got[b].double(), ref.squeeze(1), atol=1e-5)


def test_decode_special_cases():
    H, Hkv, D, bs = 4, 2, 8, 4
    q, kc, vc, table, _ = _paged(3, 2, H, Hkv, D, bs, [1, 9])
    # ctx = 1 -> the single value row, exactly
    out = decode_attention(q, kc, vc, table, torch.tensor([1, 9], dtype=torch.int32), 0.3)
    for h in range(H):
        assert torch.equal(out[0, h], vc[table[0, 0], 0, h // 2])
    # identical keys -> uniform weights -> mean of the values
    kc2 = kc.clone()
    kc2[:] = kc2[0, 0]
    out = decode_attention(q, kc2, vc, table, torch.tensor([1, 9], dtype=torch.int32), 0.3)
    vals = gather_sequence(vc, table[1], 9)
    for h in range(H):
        assert torch.allclose(out[1, h], vals[:, h // 2].mean(0), atol=1e-6)
    # one dominant score -> that value row
    kc3 = torch.zeros_like(kc)
    blk, off = int(table[1, 1]), 2   # position 6
    kc3[blk, off] = q[1].view(Hkv, 2, D)[:, 0] * 100
    out = decode_attention(q, kc3, vc, table, torch.tensor([1, 9], dtype=torch.int32), 1.0)
    assert torch.allclose(out[1, 0], vc[blk, off, 0], atol=1e-4)


def test_chunk_reduces_to_prefill_sdpa_at_offset_zero():
    H, Hkv, D, bs, L = 4, 2, 16, 4, 11
    q, kc, vc, table, _ = _paged(4, 1, H, Hkv, D, bs, [L])
    g = torch.Generator().manual_seed(5)
    qc = torch.randn(L, H, D, generator=g)
    scale = 1 / math.sqrt(D)
    got = chunk_attention(qc, kc, vc, table[0], L, scale)
    k = gather_sequence(kc, table[0], L).repeat_interleave(2, 1).permute(1, 0, 2)
    v = gather_sequence(vc, table[0], L).repeat_interleave(2, 1).permute(1, 0, 2)
    ref = F.scaled_dot_product_attention(qc.permute(1, 0, 2).double(), k.double(), v.double(),
                                         is_causal=True).permute(1, 0, 2)
    assert torch.allclose(got.double(), ref, atol=1e-5)


def test_chunk_of_one_equals_decode_and_offsets_are_consistent():
    H, Hkv, D, bs, C = 4, 2, 16, 4, 23
    q, kc, vc, table, _ = _paged(6, 1, H, Hkv, D, bs, [C])
    g = torch.Generator().manual_seed(7)
    qfull = torch.randn(C, H, D, generator=g)
    scale = 0.25
    full = chunk_attention(qfull, kc, vc, table[0], C, scale)
    # a chunk covering positions o..C-1 equals those rows of the full prefill
    for o in (0, 5, 16, 22):
        part = chunk_attention(qfull[o:], kc, vc, table[0], C, scale)
        assert torch.allclose(part, full[o:], atol=1e-6)
    # the last row alone equals a decode with context C
    dec = decode_attention(qfull[-1:].clone(), kc, vc, table[:1], torch.tensor([C], dtype=torch.int32), scale)
    assert torch.allclose(dec[0], full[-1], atol=1e-6)


def test_mixed_batch_is_per_sequence():
    H, Hkv, D, bs = 4, 2, 16, 4
    ctx = [5, 9, 12]
    qlen = [1, 4, 12]
    _, kc, vc, table, ctx_t = _paged(8, 3, H, Hkv, D, bs, ctx)
    g = torch.Generator().manual_seed(9)
    T = sum(qlen)
    q = torch.randn(T, H, D, generator=g)
    cu = torch.tensor([0, 1, 5, 17], dtype=torch.int32)
    got = mixed_attention(q, kc, vc, table, cu, ctx_t, 0.3)
    ref_dec = decode_attention(q[0:1].clone(), kc, vc, table[:1], ctx_t[:1], 0.3)
    assert torch.allclose(got[0], ref_dec[0], atol=1e-6)
    assert torch.allclose(got[1:5], chunk_attention(q[1:5], kc, vc, table[1], 9, 0.3))
