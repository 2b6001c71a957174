"""Pins of the KV-scatter oracle (CPU): round trip and untouched slots."""

from __future__ import annotations

import numpy as np

from oracle.scatter import kv_scatter


def test_round_trip_and_sentinel():
    rng = np.random.default_rng(0)
    N, bs, Hkv, D, T = 20, 4, 2, 8, 30
    kc = np.full((N, bs, Hkv, D), 7.0, np.float32)
    vc = np.full((N, bs, Hkv, D), -7.0, np.float32)
    slots = rng.permutation(N * bs)[:T].astype(np.int64)
    slots[3] = -1  # padding slot: skipped
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    kv_scatter(k, v, kc, vc, slots)
    flat_k = kc.reshape(N * bs, Hkv, D)
    flat_v = vc.reshape(N * bs, Hkv, D)
    live = slots >= 0
    assert np.array_equal(flat_k[slots[live]], k[live])
    assert np.array_equal(flat_v[slots[live]], v[live])
    untouched = np.setdiff1d(np.arange(N * bs), slots[live])
    assert np.all(flat_k[untouched] == 7.0) and np.all(flat_v[untouched] == -7.0)
    # slot s lives at block s // bs, offset s % bs
    s = int(slots[0])
    assert np.array_equal(kc[s // bs, s % bs], k[0])
