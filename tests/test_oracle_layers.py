"""Pins of the layer-op oracle (CPU): library routines, closed forms and
invariants that a dropped term, a swapped half or a wrong sign would fail."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import layers as L


def test_rms_norm_matches_library_and_scale_invariance():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 96, generator=g)
    w = torch.rand(96, generator=g) + 0.5
    assert torch.allclose(L.rms_norm(x, w, 1e-6), F.rms_norm(x, (96,), w, eps=1e-6), atol=1e-6)
    # eps = 0: scaling the input by 4 leaves the output bit-identical
    assert torch.equal(L.rms_norm(4 * x, w, 0.0), L.rms_norm(x, w, 0.0))
    # bf16 input: fp32 statistics, output rounded to bf16, within 1 ulp of fp32
    xb, wb = x.bfloat16(), w.bfloat16()
    ref = F.rms_norm(xb.float(), (96,), wb.float(), eps=1e-6)
    got = L.rms_norm(xb, wb, 1e-6)
    assert got.dtype == torch.bfloat16
    assert ((got.float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-6).all()


def test_add_rms_norm_returns_sum_and_norm():
    x = torch.randn(3, 32)
    r = torch.randn(3, 32)
    w = torch.ones(32)
    out, s = L.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(s, x + r)
    assert torch.allclose(out.pow(2).mean(-1), torch.ones(3), atol=1e-4)
    out2, none = L.add_rms_norm(x, None, w, 1e-6)
    assert none is None and torch.allclose(out2.pow(2).mean(-1), torch.ones(3), atol=1e-4)


def _tables(D, P=64, theta=1e4):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
    f = torch.outer(torch.arange(P, dtype=torch.float64), inv)
    return f.cos().float(), f.sin().float()


def test_rope_identity_norm_relative_position_and_composition():
    D = 16
    cos, sin = _tables(D)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(D, generator=g)
    k = torch.randn(D, generator=g)
    assert torch.equal(L.rope(q, cos[0], sin[0]), q)
    r = L.rope(q, cos[9], sin[9])
    pair_norm = lambda v: v[:D // 2] ** 2 + v[D // 2:] ** 2
    assert torch.allclose(pair_norm(r), pair_norm(q), atol=1e-5)
    # <R(m) q, R(n) k> depends only on m - n
    s1 = L.rope(q, cos[12], sin[12]) @ L.rope(k, cos[5], sin[5])
    s2 = L.rope(q, cos[30], sin[30]) @ L.rope(k, cos[23], sin[23])
    assert abs(float(s1 - s2)) < 1e-4
    # R(a) R(b) = R(a + b); the first half pairs with the second half (not
    # adjacent elements): rotating (e_0) by 90 degrees of frequency 0 moves it
    # to e_{D/2}
    assert torch.allclose(L.rope(L.rope(q, cos[3], sin[3]), cos[4], sin[4]),
                          L.rope(q, cos[7], sin[7]), atol=1e-5)
    e0 = torch.zeros(D)
    e0[0] = 1.0
    quarter = torch.full((D // 2,), math.cos(math.pi / 2)), torch.full((D // 2,), 1.0)
    rot = L.rope(e0, *quarter)
    assert abs(float(rot[D // 2]) - 1.0) < 1e-6 and abs(float(rot[0])) < 1e-6


def test_qk_norm_rope_cache_writes_rows_and_skips_padding():
    H, Hkv, D, bs = 4, 2, 16, 4
    cos, sin = _tables(D)
    T = 5
    qkv = torch.randn(T, (H + 2 * Hkv) * D)
    kc = torch.full((6, bs, Hkv, D), 7.0)
    vc = torch.full((6, bs, Hkv, D), 7.0)
    pos = torch.tensor([0, 1, 2, 3, 9])
    slots = torch.tensor([5, 6, -1, 20, 0])
    q = L.qk_norm_rope_cache(qkv, H, Hkv, D, cos, sin, pos, slots, kc, vc, None, None, 1e-6)
    assert torch.equal(q[0], qkv[0, :H * D].view(H, D))           # position 0: no rotation
    v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
    flat_v = vc.view(-1, Hkv, D)
    for t, s in enumerate(slots.tolist()):
        if s >= 0:
            assert torch.equal(flat_v[s], v[t])
    assert (flat_v[[1, 2, 3, 4, 7, 8]] == 7.0).all()               # untouched, incl. padding
    k0 = qkv[0, H * D:(H + Hkv) * D].view(Hkv, D)
    assert torch.equal(kc.view(-1, Hkv, D)[5], k0)


def test_silu_mul_closed_form():
    g = torch.linspace(-6, 6, 50)
    u = torch.linspace(2, -1, 50)
    out = L.silu_mul(torch.cat([g, u]).view(1, 100))
    assert torch.allclose(out[0], g * torch.sigmoid(g) * u, atol=1e-6)
    assert float(L.silu_mul(torch.tensor([[0.0, 3.0]]))[0, 0]) == 0.0
