"""Pins of the packing oracle (CPU): hand-worked fixture, literal restatement
vs descriptor expansion, closed-form invariants."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle.packing import (SeqRecord, descriptors_from_records, expand_descriptors,
                            prepare_inputs_literal)

KAT = json.loads((Path(__file__).parent / "golden" / "packing_kat.json").read_text())


def _records(case):
    return [SeqRecord(prompt_token_ids=s["prompt"], output_token_ids=s["output"],
                      num_computed_tokens=s["num_computed"], block_ids=s["blocks"])
            for s in case["seqs"]]


@pytest.mark.parametrize("case", KAT["cases"], ids=lambda c: c["name"])
def test_literal_restatement_matches_hand_worked_fixture(case):
    got = prepare_inputs_literal(_records(case), KAT["block_size"])
    for key, want in case["reference"].items():
        assert got[key] == want, key


@pytest.mark.parametrize("case", KAT["cases"], ids=lambda c: c["name"])
def test_descriptor_expansion_matches_hand_worked_fixture(case):
    descs, blocks, toks = descriptors_from_records(_records(case))
    packed = case["packed"]
    got = expand_descriptors(descs, blocks, toks, KAT["block_size"], packed["max_blocks"])
    ref = case["reference"]
    for key in ("input_ids", "positions", "slot_mapping"):
        assert got[key].tolist() == ref[key], key
    for key in ("cu_seqlens", "seq_start", "context_lens", "block_tables"):
        assert got[key].tolist() == packed[key], key


def _random_records(rng, n, block_size, decode_frac=0.5):
    recs = []
    next_block = 0
    for _ in range(n):
        plen = int(rng.integers(1, 40))
        prompt = rng.integers(0, 1000, plen).tolist()
        if rng.random() < decode_frac:
            out = rng.integers(0, 1000, int(rng.integers(1, 10))).tolist()
            nc = plen
            total = plen + len(out)
        else:
            out = []
            nc = int(rng.integers(0, plen))
            total = plen
        nb = (total + block_size - 1) // block_size
        # occasionally a short table, to exercise the slot-0 rule
        if rng.random() < 0.2 and nb > 1:
            nb -= 1
        blocks = (next_block + rng.permutation(nb * 3)[:nb]).tolist()
        next_block += nb * 3
        recs.append(SeqRecord(prompt, out, nc, blocks))
    return recs


@pytest.mark.parametrize("seed", range(6))
def test_expansion_equals_literal_on_reference_semantics(seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([4, 16]))
    recs = _random_records(rng, int(rng.integers(1, 12)), bs)
    lit = prepare_inputs_literal(recs, bs)
    descs, blocks, toks = descriptors_from_records(recs)
    mb = max(len(r.block_ids) for r in recs)
    got = expand_descriptors(descs, blocks, toks, bs, mb)
    for key in ("input_ids", "positions", "slot_mapping"):
        assert got[key].tolist() == lit[key], key
    if not lit["is_prefill"]:
        assert got["block_tables"].tolist() == lit["block_tables"]
        assert got["context_lens"].tolist() == lit["context_lens"]


@pytest.mark.parametrize("seed", range(4))
def test_expansion_invariants(seed):
    rng = np.random.default_rng(100 + seed)
    bs = 16
    recs = _random_records(rng, 30, bs)
    descs, blocks, toks = descriptors_from_records(recs)
    mb = max(len(r.block_ids) for r in recs)
    got = expand_descriptors(descs, blocks, toks, bs, mb)
    cu = got["cu_seqlens"]
    assert cu[0] == 0 and np.all(np.diff(cu) == descs[:, 1])
    for i, r in enumerate(recs):
        a, b = cu[i], cu[i + 1]
        pos = got["positions"][a:b]
        assert pos.tolist() == list(range(descs[i, 0], descs[i, 0] + descs[i, 1]))
        slots = got["slot_mapping"][a:b]
        for p, s in zip(pos, slots):
            if p // bs < len(r.block_ids):
                assert s // bs == r.block_ids[p // bs] and s % bs == p % bs
            else:
                assert s == 0
        row = got["block_tables"][i]
        assert row[:len(r.block_ids)].tolist() == r.block_ids
        assert np.all(row[len(r.block_ids):] == 0)
    assert np.all(got["context_lens"] == descs[:, 0] + descs[:, 1])


def test_device_token_indirection():
    descs = np.array([[5, 1, 1, 0, 0, 2], [0, 3, 1, 1, 0, -1]], dtype=np.int32)
    blocks = np.array([4, 7], dtype=np.int32)
    toks = np.array([100, 101, 102], dtype=np.int64)
    dev = np.array([9, 8, 777], dtype=np.int64)
    got = expand_descriptors(descs, blocks, toks, 16, 1, device_tokens=dev)
    assert got["input_ids"].tolist() == [777, 100, 101, 102]
    assert got["positions"].tolist() == [5, 0, 1, 2]
    assert got["slot_mapping"].tolist() == [4 * 16 + 5, 7 * 16, 7 * 16 + 1, 7 * 16 + 2]


# ---------------------------------------------------------------------------
# Pinned to the reference itself: 80 decode-only and prefill-only schedules
# whose packed arrays the reference's ModelRunner.prepare_inputs wrote
# (tests/golden/make_packing_fixtures.py, block tables from its BlockManager).
# ---------------------------------------------------------------------------

sys.path.insert(0, str(Path(__file__).parent / "golden"))
import packing_fixture  # noqa: E402

REF_CASES = packing_fixture.load_cases()


def test_reference_fixture_covers_both_batch_kinds_and_the_slot0_rule():
    kinds = {c["is_prefill"] for c in REF_CASES}
    assert kinds == {True, False} and len(REF_CASES) >= 50
    # some sequence of some case writes past its table (slot 0)
    assert any(any(len(s.block_ids) * c["block_size"] < s.total_len for s in c["seqs"])
               for c in REF_CASES)


@pytest.mark.parametrize("case", REF_CASES, ids=lambda c: c["name"])
def test_oracle_matches_reference_prepare_inputs(case):
    bs = case["block_size"]
    lit = prepare_inputs_literal(case["seqs"], bs)
    descs, blocks, toks = descriptors_from_records(case["seqs"])
    mb = max(len(s.block_ids) for s in case["seqs"])
    got = expand_descriptors(descs, blocks, toks, bs, mb)
    for key in ("input_ids", "positions", "slot_mapping"):
        assert lit[key] == case[key].tolist(), key
        assert np.array_equal(got[key], case[key]), key
    assert lit["is_prefill"] == case["is_prefill"]
    if not case["is_prefill"]:
        assert np.array_equal(got["block_tables"], case["block_tables"])
        assert np.array_equal(got["context_lens"], case["context_lens"])
        assert lit["block_tables"] == case["block_tables"].tolist()
        assert lit["context_lens"] == case["context_lens"].tolist()
