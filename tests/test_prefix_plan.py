"""Host side of the shared-prefix attention plan (CPU): the work-item
layout lv_paged_attention_prefix reads (include/litevllm_hip.h) built from
groups of decode rows."""

from __future__ import annotations

import pytest

from litevllm import ops


def test_prefix_plan_arrays_layout():
    """Host plan: one item per (group, 128 // G member slice, 128-key
    split); padding items have leader -1; bad groups raise."""
    blocks, items, members = ops.prefix_plan_arrays(
        [([3, 4, 5], 9), (list(range(10, 80)), 16), ([90], 8), ([91, 92], 0)],
        num_decodes=100, group_size=2, max_items=8)
    assert blocks[3] == blocks[5] == 9 and blocks[10] == blocks[79] == 16
    assert blocks[90] == 0 and blocks[91] == 0 and blocks.sum() == 3 * 9 + 70 * 16
    assert members.tolist()[:3] == [3, 4, 5] and members.tolist()[3:] == list(range(10, 80))
    want = [(3, 0, 3, 0), (3, 0, 3, 1),            # 144 keys: two splits
            (10, 3, 64, 0), (10, 3, 64, 1),        # 70 rows, 64 per item (G = 2)
            (10, 67, 6, 0), (10, 67, 6, 1)]
    assert [tuple(r) for r in items[:6].tolist()] == want
    assert (items[6:, 0] == -1).all()
    with pytest.raises(ValueError):
        ops.prefix_plan_arrays([([1, 2], 129)], 10, 2)
    with pytest.raises(ValueError):
        ops.prefix_plan_arrays([([1, 2], 4), ([2, 3], 4)], 10, 2)
    with pytest.raises(ValueError):
        ops.prefix_plan_arrays([([1, 2], 4)] * 1, 10, 2, max_items=0)


# ---------------------------------------------------------------------------
# the engine's group finder
# ---------------------------------------------------------------------------

np = pytest.importorskip("numpy")
from litevllm.engine.model_runner import find_shared_prefixes  # noqa: E402


def _step(tables, ctx):
    """Decode descriptors (num_computed = ctx - 1, query_len 1) over the
    given block tables."""
    descs, flat = [], []
    for t, c in zip(tables, ctx):
        descs.append([c - 1, 1, len(t), len(flat), 0, -1])
        flat.extend(t)
    return np.asarray(descs, np.int32), np.asarray(flat, np.int32)


def _brute(tables, ctx, bs=16):
    """Rows grouped by equal first block; prefix = longest common run of the
    group's tables, at most 128 blocks and ctx // bs for every member."""
    by_first = {}
    for r, t in enumerate(tables):
        if t and ctx[r] // bs > 0:
            by_first.setdefault(t[0], []).append(r)
    out = {}
    for rows in by_first.values():
        if len(rows) < 2:
            continue
        cap = min(min(ctx[r] // bs, len(tables[r])) for r in rows)
        cap = min(cap, 128)
        n = 0
        while n < cap and all(tables[r][n] == tables[rows[0]][n] for r in rows):
            n += 1
        if n:
            out[tuple(rows)] = n
    return out


def test_find_shared_prefixes_matches_brute_force():
    rng = np.random.default_rng(0)
    for trial in range(60):
        B = int(rng.integers(2, 70))
        next_id = [1000]

        def fresh(k):
            ids = list(range(next_id[0], next_id[0] + k))
            next_id[0] += k
            return ids
        prefixes = [fresh(int(rng.integers(1, 140))) for _ in range(int(rng.integers(1, 5)))]
        tables, ctx = [], []
        for _ in range(B):
            c = int(rng.integers(1, 2500))
            nb = (c + 15) // 16
            if rng.random() < 0.7:
                p = prefixes[int(rng.integers(len(prefixes)))]
                k = min(int(rng.integers(0, len(p) + 1)), nb)
                t = p[:k] + fresh(nb - k)
            else:
                t = fresh(nb)
            tables.append(t)
            ctx.append(c)
        descs, flat = _step(tables, ctx)
        got = find_shared_prefixes(descs, flat, B, 16, 2, max_items=10 ** 6, min_saved=0)
        got = {tuple(int(r) for r in rows): n for rows, n in got}
        assert got == _brute(tables, ctx), trial


def test_find_shared_prefixes_threshold_and_item_budget():
    # 4 groups of 10 rows sharing 40 blocks: 9 * 40 = 360 saved each,
    # 4 items each (one 64-row slice x 5 splits of 128 keys = 5 items)
    tables, ctx = [], []
    for g in range(4):
        p = list(range(10_000 * (g + 1), 10_000 * (g + 1) + 40))
        for r in range(10):
            tables.append(p + [50_000 + 100 * len(tables) + i for i in range(3)])
            ctx.append(43 * 16)
    descs, flat = _step(tables, ctx)
    assert find_shared_prefixes(descs, flat, 40, 16, 2, min_saved=4 * 360 + 1) == []
    assert len(find_shared_prefixes(descs, flat, 40, 16, 2, min_saved=4 * 360)) == 4
    two = find_shared_prefixes(descs, flat, 40, 16, 2, max_items=11, min_saved=0)
    assert len(two) == 2 and all(n == 40 for _, n in two)


def test_find_shared_prefixes_caps_at_the_context():
    """A common run longer than a member's context stops at ctx // 16
    blocks (the decode's own block is never part of the prefix unless the
    context ends on a block boundary)."""
    p = list(range(100, 140))
    tables = [p[:10] + [1], p[:10] + [2], p]
    ctx = [10 * 16 + 5, 10 * 16 + 1, 40 * 16]
    descs, flat = _step(tables, ctx)
    got = find_shared_prefixes(descs, flat, 3, 16, 2, min_saved=0)
    assert [(list(map(int, r)), n) for r, n in got] == [([0, 1, 2], 10)]
    ctx = [10 * 16, 9 * 16 + 3, 40 * 16]
    descs, flat = _step(tables, ctx)
    got = find_shared_prefixes(descs, flat, 3, 16, 2, min_saved=0)
    assert [(list(map(int, r)), n) for r, n in got] == [([0, 1, 2], 9)]


def test_check_prefix_plan_rejects_inconsistent_plans():
    """check_prefix_plan accepts what prefix_plan_arrays builds and refuses
    each way a hand-made plan could leave a prefix row with a stale or
    doubled partial."""
    blocks, items, members = ops.prefix_plan_arrays(
        [([3, 4, 5], 9), (list(range(10, 80)), 16)], num_decodes=100, group_size=2,
        max_items=8)
    ops.check_prefix_plan(blocks, items, members, 2)

    def bad(mutate, match):
        b, it, m = blocks.copy(), items.copy(), members.copy()
        mutate(b, it, m)
        with pytest.raises(ValueError, match=match):
            ops.check_prefix_plan(b, it, m, 2)

    bad(lambda b, it, m: it.__setitem__((0, 0), -1), "exactly one item")   # item dropped
    bad(lambda b, it, m: it.__setitem__((1, 2), 65), "out of range")       # slice wider than 64
    bad(lambda b, it, m: it.__setitem__((1, 1), 200), "out of range")      # slice past members
    bad(lambda b, it, m: it.__setitem__((1, 3), 3), "past its leader")     # split past the prefix
    bad(lambda b, it, m: b.__setitem__(4, 8), "another prefix length")     # member disagrees
    bad(lambda b, it, m: b.__setitem__(50 + 30, 16), "exactly one item")   # row 80 uncovered
    bad(lambda b, it, m: it.__setitem__(6, it[5]), "exactly one item")     # doubled item
