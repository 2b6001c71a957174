"""Reader of reference_packing.npz (written by make_packing_fixtures.py from
the reference's own ModelRunner.prepare_inputs, engine/model_runner.py:
180-260, and BlockManager, cache/block_manager.py:42-62): each case as
oracle.packing.SeqRecord inputs plus the reference's packed arrays."""

from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle.packing import SeqRecord

PATH = Path(__file__).resolve().parent / "reference_packing.npz"


def _split(flat, lens):
    out, at = [], 0
    for n in lens.tolist():
        out.append(flat[at:at + n].tolist())
        at += n
    return out


def load_cases() -> list[dict]:
    z = np.load(PATH, allow_pickle=False)
    cases = []
    for n in range(int(z["num_cases"])):
        g = lambda k: z[f"c{n}/{k}"]
        prompts = _split(g("prompt_ids"), g("prompt_lens"))
        outputs = _split(g("output_ids"), g("output_lens"))
        blocks = _split(g("block_ids"), g("block_lens"))
        recs = [SeqRecord(p, o, int(nc), b)
                for p, o, nc, b in zip(prompts, outputs, g("num_computed").tolist(), blocks)]
        is_prefill = bool(g("is_prefill"))
        case = {"name": f"c{n}_{'prefill' if is_prefill else 'decode'}_bs{int(g('block_size'))}",
                "block_size": int(g("block_size")), "is_prefill": is_prefill, "seqs": recs,
                "input_ids": g("input_ids").astype(np.int64),
                "positions": g("positions").astype(np.int64),
                "slot_mapping": g("slot_mapping").astype(np.int64)}
        if not is_prefill:
            case["block_tables"] = g("block_tables")
            case["context_lens"] = g("context_lens")
        cases.append(case)
    return cases
