"""Host-side engine logic (CPU): block manager, scheduler, prefix cache,
config, RoPE, and the packing descriptors.  The first tests of each group
restate what the reference's own tests pin (tests/test_block_manager.py,
test_scheduler.py, test_prefix_cache.py, test_config.py, test_rotary_emb.py);
the rest cover this build's additions (real chunks, chained prefix keys,
descriptor packing)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from litevllm.cache.block_manager import BlockManager
from litevllm.cache.prefix_cache import PrefixCache
from litevllm.config import CacheConfig, SamplingParams, SchedulerConfig
from litevllm.engine.model_runner import build_step
from litevllm.engine.scheduler import Scheduler
from litevllm.engine.sequence import SequenceGroup, SequenceStatus
from litevllm.layers.rotary_emb import RotaryEmbedding, apply_rotary_emb
from oracle.packing import SeqRecord, expand_descriptors, prepare_inputs_literal


# -- block manager ----------------------------------------------------------

def test_allocate_free_counts_and_lifo_order():
    bm = BlockManager(block_size=16, num_gpu_blocks=8)
    t = bm.allocate(1, 3)
    assert bm.num_free_gpu_blocks == 5 and len(bm.get_block_table(1)) == 3
    assert t.ids == [7, 6, 5]          # handed out from the end of the free list
    bm.free(1)
    assert bm.num_free_gpu_blocks == 8 and 1 not in bm.block_tables
    assert bm.allocate(2, 1).ids == [5]  # most recently freed first


def test_can_allocate_append_fork_and_exhaustion():
    bm = BlockManager(block_size=16, num_gpu_blocks=4)
    bm.allocate(1, 1)
    bm.append_slot(1)
    assert len(bm.get_block_table(1)) == 2 and bm.num_free_gpu_blocks == 2
    assert bm.num_forks == 0
    bm.fork(1, 2)
    assert bm.num_forks == 1   # the runner's shared-prefix search looks for sharing again
    assert all(b.ref_count == 2 for b in bm.get_block_table(1).blocks)
    bm.free(1)
    assert bm.num_free_gpu_blocks == 2
    bm.free(2)
    assert bm.num_free_gpu_blocks == 4
    bm.allocate(3, 4)
    assert not bm.can_allocate(1)
    with pytest.raises(RuntimeError):
        bm.allocate(4, 1)


# -- scheduler ----------------------------------------------------------------

def _sched(max_num_seqs=8, tokens=256, chunk=128, blocks=64, bs=16, prefix=False):
    cc = CacheConfig(block_size=bs, num_gpu_blocks=blocks, enable_prefix_caching=prefix)
    sc = SchedulerConfig(max_num_seqs=max_num_seqs, max_num_batched_tokens=tokens,
                         chunked_prefill=True, chunk_size=chunk)
    bm = BlockManager(bs, blocks)
    return Scheduler(sc, cc, bm, PrefixCache(bs, bm) if prefix else None)


def _req(s, rid, n, max_tokens=8, base=0):
    sg = SequenceGroup.create(rid, list(range(base, base + n)), SamplingParams(max_tokens=max_tokens))
    s.add_request(sg)
    return sg


def test_reference_scheduler_behaviours():
    s = _sched()
    _req(s, "r1", 32)
    _req(s, "r2", 64)
    out = s.schedule()
    assert out.num_prefill_groups == 2 and out.num_decode_groups == 0 and not out.is_empty
    s2 = _sched(chunk=64)
    _req(s2, "r1", 200)
    out = s2.schedule()
    assert out.num_prefill_groups == 1 and out.num_batched_tokens <= 256
    s3 = _sched(blocks=8)
    sg = _req(s3, "r1", 16)
    s3.schedule()
    s3.update_running([sg])
    before = s3.block_manager.num_free_gpu_blocks
    for seq in sg.seqs:
        seq.status = SequenceStatus.FINISHED_LENGTH
    assert len(s3.free_finished()) == 1 and s3.block_manager.num_free_gpu_blocks > before
    s4 = _sched()
    _req(s4, "r1", 16)
    _req(s4, "r2", 16)
    s4.abort_request("r1")
    assert [g.request_id for g in s4.waiting] == ["r2"]


def _advance(s, out):
    """Apply a step's progress the way LLMEngine.step does (token 7 sampled)."""
    for sg in out.scheduled_seq_groups:
        for seq in sg.get_unfinished_seqs():
            if seq.is_prefill:
                seq.num_computed_tokens += seq.num_scheduled_tokens
                if seq.num_computed_tokens == seq.data.prompt_len:
                    seq.data.append_token(7)
            else:
                seq.num_computed_tokens = seq.data.total_len
                seq.data.append_token(7)
            seq.num_scheduled_tokens = 0


def test_real_chunks_and_decode_first_order():
    s = _sched(tokens=100, chunk=64)
    a = _req(s, "a", 150)
    out = s.schedule()
    assert [g.request_id for g in out.scheduled_seq_groups] == ["a"]
    assert a.seqs[0].num_scheduled_tokens == 64
    assert len(s.block_manager.get_block_table(a.seqs[0].seq_id)) == 4
    _advance(s, out)
    b = _req(s, "b", 40)
    out = s.schedule()                       # a continues (64), b gets the rest (36)
    assert [g.request_id for g in out.scheduled_seq_groups] == ["a", "b"]
    assert a.seqs[0].num_scheduled_tokens == 64 and b.seqs[0].num_scheduled_tokens == 36
    assert out.num_batched_tokens == 100
    _advance(s, out)
    out = s.schedule()                       # a: last 22 prompt tokens; b: 4 more
    assert a.seqs[0].num_scheduled_tokens == 22 and b.seqs[0].num_scheduled_tokens == 4
    _advance(s, out)
    out = s.schedule()                       # both decode now, decodes first
    assert out.num_decode_groups == 2 and out.num_prefill_groups == 0
    assert all(seq.num_scheduled_tokens == 1 for g in out.scheduled_seq_groups for seq in g.seqs)


def test_prefix_cache_admission_reuses_blocks():
    s = _sched(bs=4, blocks=64, prefix=True)
    a = _req(s, "a", 10)                     # tokens 0..9
    out = s.schedule()
    _advance(s, out)
    s.prefix_cache.insert(a.seqs[0].data.prompt_token_ids, s.block_manager.get_block_table(a.seqs[0].seq_id))
    b = _req(s, "b", 14)                     # shares tokens 0..9 -> 2 full blocks cached
    s.schedule()
    sb = b.seqs[0]
    assert sb.num_computed_tokens == 8 and sb.num_scheduled_tokens == 6
    ta = s.block_manager.get_block_table(a.seqs[0].seq_id).ids
    tb = s.block_manager.get_block_table(sb.seq_id).ids
    assert tb[:2] == ta[:2] and len(tb) == 4


def test_reference_prefix_cache_lookups_and_chained_keys():
    bs = 4
    bm = BlockManager(bs, 8)
    bm.allocate(1, 3)
    pc = PrefixCache(bs)
    pc.insert(list(range(12)), bm.get_block_table(1))
    assert pc.lookup(list(range(12)), bm)[1] == 12
    blocks, n = pc.lookup(list(range(8)) + [99, 100, 101, 102], bm)
    assert n == 8 and len(blocks) == 2
    assert PrefixCache(4).lookup([1, 2, 3, 4], bm) == ([], 0)
    # same block tokens behind a different prefix are not a hit
    assert pc.lookup([50, 51, 52, 53] + list(range(4, 8)), bm)[1] == 0


def test_prefix_cache_evicts_unused_blocks_when_full():
    bs = 4
    bm = BlockManager(bs, 4)
    pc = PrefixCache(bs, bm)
    bm.allocate(1, 4)
    pc.insert(list(range(16)), bm.get_block_table(1))
    bm.free(1)
    assert bm.num_free_gpu_blocks == 0       # the cache still holds them
    assert bm.can_allocate(2) and bm.num_free_gpu_blocks >= 2
    assert len(pc.cache) == 2


# -- config / rope --------------------------------------------------------------

def test_sampling_params_validation():
    sp = SamplingParams()
    assert (sp.temperature, sp.top_p, sp.max_tokens, sp.ignore_eos) == (1.0, 1.0, 256, False)
    for kw in ({"temperature": -0.1}, {"top_p": 0.0}, {"top_p": 1.5}, {"max_tokens": 0}):
        with pytest.raises(ValueError):
            SamplingParams(**kw)


def test_rope_identity_at_zero_and_norm_preserved():
    rope = RotaryEmbedding(head_dim=32, max_position_embeddings=128)
    cos, sin = rope(torch.tensor([0]))
    assert torch.allclose(cos, torch.ones_like(cos)) and torch.allclose(sin, torch.zeros_like(sin))
    x = torch.randn(4, 1, 32)
    cos, sin = rope(torch.arange(4))
    y = apply_rotary_emb(x, cos.unsqueeze(1), sin.unsqueeze(1))
    assert torch.allclose(x.norm(dim=-1), y.norm(dim=-1), atol=1e-5)


# -- packing descriptors vs the literal prepare_inputs restatement -----------

@pytest.mark.parametrize("seed", range(5))
def test_build_step_matches_literal_prepare_inputs(seed):
    rng = np.random.default_rng(seed)
    bs = 16
    bm = BlockManager(bs, 4096)
    groups, recs = [], []
    decode_phase = rng.random() < 0.5      # reference batches are all-decode or prefill
    for i in range(int(rng.integers(1, 9))):
        plen = int(rng.integers(1, 70))
        sg = SequenceGroup.create(f"r{i}", rng.integers(0, 30000, plen).tolist(),
                                  SamplingParams())
        seq = sg.seqs[0]
        if decode_phase:
            seq.num_computed_tokens = plen
            for _ in range(int(rng.integers(1, 20))):
                seq.data.append_token(int(rng.integers(0, 30000)))
        else:
            seq.num_computed_tokens = int(rng.integers(0, plen))
        bm.allocate(seq.seq_id, seq.get_num_blocks(bs))
        groups.append(sg)
        recs.append(SeqRecord(seq.data.prompt_token_ids, seq.data.output_token_ids,
                              seq.num_computed_tokens, bm.get_block_table(seq.seq_id).ids))
    st = build_step(groups, bm)
    lit = prepare_inputs_literal(recs, bs)
    got = expand_descriptors(st.descs, st.block_ids, np.asarray(st.tokens, np.int64), bs,
                             st.max_blocks)
    for k in ("input_ids", "positions", "slot_mapping"):
        assert got[k].tolist() == lit[k], k
    assert st.is_prefill == lit["is_prefill"]
    if not lit["is_prefill"]:
        assert got["block_tables"].tolist() == lit["block_tables"]
        assert got["context_lens"].tolist() == lit["context_lens"]
        assert st.num_decodes == len(groups) and len(st.sample_seqs) == len(groups)
    else:
        assert st.logits_rows == list(np.cumsum([r.total_len - r.num_computed_tokens
                                                 for r in recs]) - 1)


def test_engine_runs_forward_for_chunks_that_sample_nothing():
    """A step whose only work is a non-final prefill chunk still runs the
    forward (its K/V must reach the cache) and advances the sequence."""
    from litevllm.config import EngineConfig, ModelConfig
    from litevllm.engine.llm_engine import LLMEngine

    class StubRunner:
        calls = 0

        def prepare_inputs(self, groups, bm, device_tokens=None):
            st = build_step(groups, bm)
            return type("M", (), {"sample_seqs": st.sample_seqs, "sample_groups": st.sample_groups})

        def execute_model(self, meta):
            StubRunner.calls += 1
            return torch.zeros(len(meta.sample_seqs), 10)

    eng = LLMEngine(EngineConfig(model_config=ModelConfig("x", load_format="dummy")))
    eng.scheduler = _sched(tokens=64, chunk=64)
    eng.block_manager = eng.scheduler.block_manager
    eng.model_runner = StubRunner()
    sg = _req(eng.scheduler, "a", 150)
    eng.step()
    assert StubRunner.calls == 1 and sg.seqs[0].num_computed_tokens == 64
    eng.step()
    assert StubRunner.calls == 2 and sg.seqs[0].num_computed_tokens == 128


def test_build_step_feeds_inflight_tokens_from_the_device():
    """A decode whose last token is still in flight reads it from the
    previous step's sampled ids (token_index = its row) at position
    total_len + num_inflight - 1; the result equals the literal packing of
    the same sequence with that token appended on the host."""
    bs = 16
    bm = BlockManager(bs, 64)
    groups, recs = [], []
    prev_ids = np.array([900, 901, 902, 903], dtype=np.int64)
    for i, (plen, n_out, row) in enumerate([(20, 3, 2), (33, 0, 0), (5, 7, -1)]):
        sg = SequenceGroup.create(f"r{i}", list(range(100 * i, 100 * i + plen)), SamplingParams())
        seq = sg.seqs[0]
        seq.num_computed_tokens = plen
        for t in range(n_out):
            seq.data.append_token(50 + t)
        if row >= 0:
            seq.num_inflight, seq.inflight_row = 1, row
        bm.allocate(seq.seq_id, (seq.data.total_len + seq.num_inflight + bs - 1) // bs)
        groups.append(sg)
        out = seq.data.output_token_ids + ([int(prev_ids[row])] if row >= 0 else [])
        recs.append(SeqRecord(seq.data.prompt_token_ids, out, plen,
                              bm.get_block_table(seq.seq_id).ids))
    st = build_step(groups, bm)
    assert st.uses_device_tokens and st.num_tokens == 3 and len(st.tokens) == 1
    assert st.descs[:, 5].tolist() == [2, 0, -1]
    got = expand_descriptors(st.descs, st.block_ids, np.asarray(st.tokens, np.int64), bs,
                             st.max_blocks, device_tokens=prev_ids)
    lit = prepare_inputs_literal(recs, bs)
    for k in ("input_ids", "positions", "slot_mapping"):
        assert got[k].tolist() == lit[k], k
    assert got["context_lens"].tolist() == lit["context_lens"]


def test_scheduler_counts_inflight_tokens_and_skips_finishing_sequences():
    s = _sched(bs=4, blocks=16)
    sg = _req(s, "a", 4, max_tokens=3)
    out = s.schedule()
    _advance(s, out)                       # prompt done, 1 output token on the host
    seq = sg.seqs[0]
    seq.num_inflight, seq.inflight_row = 1, 0
    out = s.schedule()                     # position total_len + 1 - 1 = 5 -> 2 blocks
    assert out.num_decode_groups == 1
    assert len(s.block_manager.get_block_table(seq.seq_id)) == 2
    seq.num_scheduled_tokens = 0
    seq.num_inflight = 2                   # 1 on host + 2 in flight reach max_tokens=3
    assert s.schedule().is_empty
