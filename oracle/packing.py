"""CPU restatement of ragged-batch packing (test oracle).

prepare_inputs_literal restates ModelRunner.prepare_inputs (reference
litevllm/engine/model_runner.py:180-260) loop for loop on plain Python
sequence records; pure-Python loops, so only for small cases.

expand_descriptors is the same computation driven by per-sequence
descriptors (the lv_seq_desc layout of include/litevllm_hip.h), vectorised
with numpy.  The tests pin it against the literal restatement and the
hand-worked fixture tests/golden/packing_kat.json.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class SeqRecord:
    """The fields prepare_inputs reads from a Sequence (engine/sequence.py:36-107)."""
    prompt_token_ids: list[int]
    output_token_ids: list[int] = field(default_factory=list)
    num_computed_tokens: int = 0
    block_ids: list[int] = field(default_factory=list)

    @property
    def total_len(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    @property
    def is_prefill(self) -> bool:   # sequence.py:95-97
        return self.num_computed_tokens < len(self.prompt_token_ids)


def prepare_inputs_literal(seqs: list[SeqRecord], block_size: int) -> dict:
    """model_runner.py:186-250 on SeqRecords; returns Python lists / None."""
    input_ids, positions, slots, tables, ctx = [], [], [], [], []
    is_prefill = False
    for seq in seqs:
        bt = seq.block_ids
        if seq.is_prefill:                                   # 201-216
            is_prefill = True
            start, end = seq.num_computed_tokens, len(seq.prompt_token_ids)
            for i, tok in enumerate(seq.prompt_token_ids[start:end]):
                pos = start + i
                input_ids.append(tok)
                positions.append(pos)
                bi, bo = pos // block_size, pos % block_size
                slots.append(bt[bi] * block_size + bo if bi < len(bt) else 0)
        else:                                                # 217-232
            all_ids = seq.prompt_token_ids + seq.output_token_ids
            pos = seq.total_len - 1
            input_ids.append(all_ids[-1])
            positions.append(pos)
            bi, bo = pos // block_size, pos % block_size
            slots.append(bt[bi] * block_size + bo if bi < len(bt) else 0)
            ctx.append(seq.total_len)
            tables.append(list(bt))
    if is_prefill:                                           # 239-241
        block_tables = context_lens = None
    else:                                                    # 242-250
        mb = max((len(t) for t in tables), default=0)
        block_tables = [t + [0] * (mb - len(t)) for t in tables]
        context_lens = ctx
    return {"input_ids": input_ids, "positions": positions, "slot_mapping": slots,
            "block_tables": block_tables, "context_lens": context_lens,
            "is_prefill": is_prefill}


def descriptors_from_records(seqs: list[SeqRecord]):
    """Reference-semantics descriptors for SeqRecords (prefill feeds the
    whole remaining prompt, decode feeds the last token).

    Returns (descs int32 [B, 6], block_ids int32, token_ids int64).
    """
    descs, blocks, toks = [], [], []
    for seq in seqs:
        if seq.is_prefill:
            n = seq.num_computed_tokens
            q = len(seq.prompt_token_ids) - n
            ids = seq.prompt_token_ids[n:]
        else:
            n = seq.total_len - 1
            q = 1
            ids = [(seq.prompt_token_ids + seq.output_token_ids)[-1]]
        descs.append([n, q, len(seq.block_ids), len(blocks), len(toks), -1])
        blocks.extend(seq.block_ids)
        toks.extend(ids)
    return (np.asarray(descs, dtype=np.int32).reshape(-1, 6),
            np.asarray(blocks, dtype=np.int32), np.asarray(toks, dtype=np.int64))


def expand_descriptors(descs: np.ndarray, block_ids: np.ndarray, token_ids: np.ndarray,
                       block_size: int, max_blocks: int,
                       device_tokens: np.ndarray | None = None) -> dict[str, np.ndarray]:
    """The packed step arrays that lv_pack_inputs must produce (numpy)."""
    descs = np.asarray(descs, dtype=np.int64).reshape(-1, 6)
    nc, ql, nb, boff, toff, tidx = (descs[:, i] for i in range(6))
    B = descs.shape[0]
    cu = np.zeros(B + 1, dtype=np.int64)
    cu[1:] = np.cumsum(ql)
    T = int(cu[-1])
    seq_of = np.repeat(np.arange(B), ql)
    j = np.arange(T) - cu[seq_of]
    pos = nc[seq_of] + j
    from_dev = tidx[seq_of] >= 0
    ids = np.zeros(T, dtype=np.int64)
    host_idx = toff[seq_of] + j
    ids[~from_dev] = token_ids[host_idx[~from_dev]]
    if from_dev.any():
        ids[from_dev] = np.asarray(device_tokens)[tidx[seq_of][from_dev]]
    bi = pos // block_size
    has = bi < nb[seq_of]
    slot = np.zeros(T, dtype=np.int64)
    src = (boff[seq_of] + bi)[has]
    slot[has] = block_ids[src].astype(np.int64) * block_size + pos[has] % block_size
    tables = np.zeros((B, max_blocks), dtype=np.int32)
    for i in range(B):
        n = int(min(nb[i], max_blocks))
        tables[i, :n] = block_ids[boff[i]:boff[i] + n]
    return {
        "input_ids": ids, "positions": pos.astype(np.int64), "slot_mapping": slot,
        "cu_seqlens": cu.astype(np.int32), "seq_start": nc.astype(np.int32),
        "context_lens": (nc + ql).astype(np.int32), "block_tables": tables,
    }
