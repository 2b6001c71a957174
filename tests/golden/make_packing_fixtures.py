#!/usr/bin/env python3
"""Write tests/golden/reference_packing.npz from the reference itself.

BUILD CONTAINER ONLY: imports the reference package from /root/reference
(lite-vllm 0.1.0, pure Python/torch), which does not exist on the GPU host.
The committed .npz is data (schedules and the packed arrays); nothing here
runs at test time.

For each case the script builds a batch the way the reference engine does:
Sequence objects (engine/sequence.py:120-134 SequenceGroup.create) whose
block tables come from the reference's own BlockManager
(cache/block_manager.py:42-62 free-list allocator, 111-131 allocate /
append_slot / free, with allocations and frees of other sequences in
between so the free list is shuffled), then calls the reference's
ModelRunner.prepare_inputs (engine/model_runner.py:180-260) on the CPU and
records its outputs.  Schedules are decode-only (every sequence past its
prompt; block tables padded with 0 to the batch maximum) or prefill-only
(every sequence at a random num_computed_tokens inside its prompt; block
tables and context_lens are None there).  About one sequence in six has a
table one block short of its tokens, which exercises the slot-0 rule
(model_runner.py:211-215, 224-228).  The reference has no mixed batch form
(a prefill in the batch drops the decode tables, 239-241), so none is
written.

Stored per case c (arrays flattened; *_lens give the split points):
  c{n}/block_size, c{n}/is_prefill            scalars
  c{n}/prompt_ids, c{n}/prompt_lens           prompts
  c{n}/output_ids, c{n}/output_lens           generated tokens so far
  c{n}/num_computed                           per sequence
  c{n}/block_ids, c{n}/block_lens             per-sequence physical block ids
  c{n}/input_ids, c{n}/positions, c{n}/slot_mapping       reference outputs
                                              (int64 there, stored as int32)
  c{n}/block_tables, c{n}/context_lens        decode-only cases

Usage: python tests/golden/make_packing_fixtures.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference")
OUT = HERE / "reference_packing.npz"
NUM_DECODE_CASES = 40
NUM_PREFILL_CASES = 40


def _import_reference():
    if not (REFERENCE / "litevllm").is_dir():
        raise SystemExit(f"{REFERENCE} not found: this script runs in the build container only")
    sys.path.insert(0, str(REFERENCE))
    import litevllm  # noqa: F401
    if not Path(litevllm.__file__).resolve().is_relative_to(REFERENCE.resolve()):
        raise SystemExit(f"imported {litevllm.__file__}, not the reference")
    from litevllm.cache.block_manager import BlockManager
    from litevllm.config import CacheConfig, EngineConfig, ModelConfig, SamplingParams
    from litevllm.engine.model_runner import ModelRunner
    from litevllm.engine.sequence import SequenceGroup
    return BlockManager, CacheConfig, EngineConfig, ModelConfig, SamplingParams, ModelRunner, \
        SequenceGroup


def _narrow(t):
    a = t.numpy()
    assert a.dtype == np.int64 and (a.size == 0 or (a.min() >= 0 and a.max() < 2**31))
    return a.astype(np.int32)


def make_case(rng, ref, decode: bool, block_size: int):
    BlockManager, CacheConfig, EngineConfig, ModelConfig, SamplingParams, ModelRunner, \
        SequenceGroup = ref
    n_seqs = int(rng.integers(1, 25))
    bm = BlockManager(block_size, num_gpu_blocks=4096, reserved_blocks=int(rng.integers(0, 2)))
    filler = 10**6                      # seq ids of other requests, allocated and freed
    groups = []
    for i in range(n_seqs):
        # other requests come and go, so this sequence gets scattered ids
        for _ in range(int(rng.integers(0, 4))):
            filler += 1
            bm.allocate(filler, int(rng.integers(1, 6)))
            if rng.random() < 0.6:
                bm.free(filler)
        plen = int(rng.integers(1, 160))
        prompt = rng.integers(0, 151936, plen).tolist()
        sg = SequenceGroup.create(f"r{i}", prompt, SamplingParams(temperature=0.0))
        seq = sg.seqs[0]
        if decode:
            for tok in rng.integers(0, 151936, int(rng.integers(1, 120))).tolist():
                seq.data.append_token(tok)
            seq.num_computed_tokens = plen
        else:
            seq.num_computed_tokens = int(rng.integers(0, plen))
        need = (seq.data.total_len + block_size - 1) // block_size
        short = need > 1 and rng.random() < 1 / 6
        first = (plen + block_size - 1) // block_size
        bm.allocate(seq.seq_id, min(first, need - 1) if short else first)
        while len(bm.get_block_table(seq.seq_id)) < need - (1 if short else 0):
            bm.append_slot(seq.seq_id)     # decode growth, as the scheduler does
        groups.append(sg)
    runner = ModelRunner(EngineConfig(ModelConfig("packing-fixture"),
                                      CacheConfig(block_size=block_size), device="cpu"))
    meta = runner.prepare_inputs(groups, bm)
    assert meta.is_prefill == (not decode)
    seqs = [sg.seqs[0] for sg in groups]
    tables = [bm.get_block_table(s.seq_id).physical_block_ids for s in seqs]
    case = {
        "block_size": np.int64(block_size),
        "is_prefill": np.int64(meta.is_prefill),
        "prompt_ids": np.concatenate([np.asarray(s.data.prompt_token_ids, np.int32)
                                      for s in seqs]),
        "prompt_lens": np.asarray([s.data.prompt_len for s in seqs], np.int64),
        "output_ids": np.asarray([t for s in seqs for t in s.data.output_token_ids], np.int32),
        "output_lens": np.asarray([s.data.output_len for s in seqs], np.int64),
        "num_computed": np.asarray([s.num_computed_tokens for s in seqs], np.int64),
        "block_ids": np.asarray([b for t in tables for b in t], np.int32),
        "block_lens": np.asarray([len(t) for t in tables], np.int64),
        # int64 tensors in the reference; every value fits 32 bits
        "input_ids": _narrow(meta.input_ids),
        "positions": _narrow(meta.positions),
        "slot_mapping": _narrow(meta.slot_mapping),
    }
    if not meta.is_prefill:
        case["block_tables"] = meta.block_tables.numpy().astype(np.int32)
        case["context_lens"] = meta.context_lens.numpy().astype(np.int32)
    return case


def main() -> None:
    ref = _import_reference()
    rng = np.random.default_rng(2024)
    out = {}
    n = 0
    for decode, count in ((True, NUM_DECODE_CASES), (False, NUM_PREFILL_CASES)):
        for k in range(count):
            bs = 16 if k % 4 else int(rng.choice([8, 32]))
            for key, val in make_case(rng, ref, decode, bs).items():
                out[f"c{n}/{key}"] = val
            n += 1
    out["num_cases"] = np.int64(n)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {n} cases, {OUT.stat().st_size} bytes")


if __name__ == "__main__":
    main()
