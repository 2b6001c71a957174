"""Pins of the sampler oracle (CPU): the reference's KATs, exp2_det accuracy,
distributional checks and special cases of the inverse-CDF definition."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import sampler

KATS = json.loads((Path(__file__).parent / "golden" / "reference_sampler_kats.json").read_text())


def test_reference_greedy_kat():
    x = np.array(KATS["greedy"]["logits"], dtype=np.float32)
    assert sampler.greedy(x).tolist() == KATS["greedy"]["expected"]
    assert sampler.sample(x, np.zeros(2, np.float32), np.zeros(2, np.float32)).tolist() == \
        KATS["greedy"]["expected"]


def test_reference_planted_max_kat():
    kat = KATS["top_k_planted"]
    x = np.zeros((1, kat["vocab"]), dtype=np.float32)
    x[0, kat["planted_index"]] = kat["planted_value"]
    # greedy and T=1 sampling both land on the planted token: the others
    # have probability 2^-144.3 each (subnormal in fp32, as exp(-100) is in
    # the reference's fp32 softmax), so every u above 7 * 2^-144.3 draws it
    assert sampler.sample(x, np.zeros(1, np.float32), np.zeros(1, np.float32)).tolist() == kat["expected"]
    for u in (1e-30, 0.5, 0.999999):
        assert sampler.sample(x, np.ones(1, np.float32), np.array([u], np.float32)).tolist() == kat["expected"]
    # u = 0 is the inverse CDF at 0: the first token of nonzero probability
    assert sampler.sample(x, np.ones(1, np.float32), np.zeros(1, np.float32)).tolist() == [0]


def test_greedy_first_index_on_ties():
    x = np.array([[1.0, 3.0, 3.0, 2.0], [-np.inf, -np.inf, 0.0, 0.0]], dtype=np.float32)
    assert sampler.sample(x, np.zeros(2, np.float32), np.zeros(2, np.float32)).tolist() == [1, 2]


def test_exp2_det_accuracy():
    # normal results: relative error against float64 exp2, including inputs
    # just below 0 (where t - floor(t) rounds to 1 and is clamped) and tiny
    # subnormal inputs
    t = np.concatenate([np.linspace(-125.0, 0.0, 400001, dtype=np.float32),
                        np.array([-1e-9, -2.0 ** -26, -2.0 ** -24, -1e-30, -1e-45, -0.0,
                                  -1.0, -0.5, -124.999], np.float32)])
    got = sampler.exp2_det(t).astype(np.float64)
    ref = np.exp2(t.astype(np.float64))
    assert (np.abs(got - ref) / ref).max() < 2.0 ** -22
    # exact powers of two below the normal range (P(0) = 1), gradual
    # underflow, and the inputs that give 0
    got = sampler.exp2_det(np.array([0.0, -126.0, -149.0, -150.0, -151.0, -200.0, -1e30,
                                     -np.inf, np.nan], np.float32)).tolist()
    assert got == [1.0, 2.0 ** -126, 2.0 ** -149, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]
    # between -150 and -126 the result is 2^t rounded to the subnormal grid
    t = np.float32(-140.3)
    assert abs(sampler.exp2_det(np.array([t]))[0] - 2.0 ** -140.3) <= 2.0 ** -150


def _softmax64(x, T):
    z = x.astype(np.float64) / T
    z -= z.max()
    p = np.exp(z)
    return p / p.sum()


def test_agrees_with_float64_inverse_cdf_away_from_bin_edges():
    rng = np.random.default_rng(0)
    V = 1300  # three segments, last one partial
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    T = np.float32(0.7)
    p = _softmax64(x, float(T))
    cdf = np.cumsum(p)
    us = rng.random(4000).astype(np.float32)
    got = sampler.sample(np.repeat(x[None], len(us), 0), np.full(len(us), T, np.float32), us)
    ref = np.searchsorted(cdf, us.astype(np.float64), side="right")
    edge = np.minimum(np.abs(cdf[np.clip(ref, 0, V - 1)] - us), np.abs(cdf[np.clip(ref - 1, 0, V - 1)] - us))
    far = edge > 2e-6
    assert far.mean() > 0.99
    assert np.array_equal(got[far], ref[far])


def test_chi_square_against_softmax():
    rng = np.random.default_rng(1)
    V = 40
    x = rng.standard_normal(V).astype(np.float32)
    T = np.float32(0.8)
    n = 20000
    us = rng.random(n).astype(np.float32)
    got = sampler.sample(np.repeat(x[None], n, 0), np.full(n, T, np.float32), us)
    counts = np.bincount(got, minlength=V)
    p = _softmax64(x, float(T))
    keep = p * n >= 5
    chi2 = (((counts[keep] - p[keep] * n) ** 2) / (p[keep] * n)).sum()
    # 99.9% quantile of chi-square with <= 39 dof is about 72
    assert chi2 < 80, chi2


def test_special_cases():
    rng = np.random.default_rng(2)
    V = 1000
    x = rng.standard_normal(V).astype(np.float32)
    one = lambda arr, t, u: int(sampler.sample(arr[None], np.array([t], np.float32),
                                               np.array([u], np.float32))[0])
    # u = 0 -> first index with positive weight; u -> 1 -> last such index
    assert one(x, 1.0, 0.0) == 0
    assert one(x, 1.0, np.nextafter(np.float32(1), np.float32(0))) == V - 1
    # -inf entries are never drawn, even at the extremes
    y = x.copy()
    y[:10] = -np.inf
    y[-7:] = -np.inf
    assert one(y, 1.0, 0.0) == 10
    assert one(y, 1.0, np.nextafter(np.float32(1), np.float32(0))) == V - 8
    # tiny temperature -> argmax; huge margin -> that token
    assert one(x, 1e-3, 0.5) == int(np.argmax(x))
    z = np.zeros(V, np.float32)
    z[517] = 110.0   # every other weight is 2^-158.7 -> exactly 0
    for u in (0.0, 0.3, 0.9999):
        assert one(z, 1.0, u) == 517
    for big in (100.0, 80.0):   # others keep 2^-144.3 (subnormal) / 2^-115.4 > 0:
        z[517] = big            # u = 0 picks the first of them
        assert one(z, 1.0, 0.0) == 0 and one(z, 1.0, 0.3) == 517
    # uniform logits: token = floor(u * V) away from edges
    flat = np.zeros(V, np.float32)
    for u in (0.1234, 0.5, 0.77777):
        assert one(flat, 1.0, u) == int(np.floor(u * V))


@pytest.mark.parametrize("V", [1, 7, 8, 511, 512, 513, 4096 + 3])
def test_odd_vocab_sizes_stay_in_range(V):
    rng = np.random.default_rng(V)
    x = rng.standard_normal((16, V)).astype(np.float32)
    t = np.full(16, 0.9, np.float32)
    u = rng.random(16).astype(np.float32)
    got = sampler.sample(x, t, u)
    assert np.all((got >= 0) & (got < V))
