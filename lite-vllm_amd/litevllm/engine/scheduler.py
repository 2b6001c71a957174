"""Continuous-batching scheduler with real chunked prefill.

Same interface as the reference (engine/scheduler.py:18-184: SchedulerOutput,
Scheduler.add_request / has_unfinished / abort_request / schedule /
free_finished / update_running) and the same policy: FCFS, a decode-first
token budget, no preemption (a sequence that cannot get a block waits),
head-of-line blocking on admission.  Differences, all so that one mixed
forward per step can run on the GPU:

* a prefill gets a real chunk, min(remaining, chunk_size, budget left), and
  ``Sequence.num_scheduled_tokens`` records it (the reference charges the
  chunk to the budget but feeds the whole prompt, model_runner.py:202-205);
* partially prefilled sequences stay running and continue before new
  admissions;
* with a prefix cache, admission reuses the cached leading blocks and starts
  the sequence at the first uncached token;
* the scheduled list is ordered decodes first, then prefills, which is the
  batch order lv_paged_attention expects.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Optional

from ..cache.block_manager import BlockManager
from ..cache.prefix_cache import PrefixCache
from ..config import CacheConfig, SchedulerConfig
from .sequence import SequenceGroup, SequenceStatus


@dataclass
class SchedulerOutput:
    scheduled_seq_groups: list[SequenceGroup]
    num_prefill_groups: int
    num_decode_groups: int
    blocks_to_swap_in: dict[int, int] = field(default_factory=dict)
    blocks_to_swap_out: dict[int, int] = field(default_factory=dict)
    blocks_to_copy: dict[int, int] = field(default_factory=dict)

    @property
    def is_empty(self) -> bool:
        return not self.scheduled_seq_groups

    @property
    def num_batched_tokens(self) -> int:
        return sum(s.num_scheduled_tokens for sg in self.scheduled_seq_groups
                   for s in sg.get_unfinished_seqs())


class Scheduler:
    def __init__(self, scheduler_config: SchedulerConfig, cache_config: CacheConfig,
                 block_manager: BlockManager, prefix_cache: Optional[PrefixCache] = None) -> None:
        self.config = scheduler_config
        self.cache_config = cache_config
        self.block_manager = block_manager
        self.prefix_cache = prefix_cache
        self.waiting: deque[SequenceGroup] = deque()
        self.running: list[SequenceGroup] = []
        self.swapped: list[SequenceGroup] = []

    def add_request(self, seq_group: SequenceGroup) -> None:
        self.waiting.append(seq_group)

    def has_unfinished(self) -> bool:
        return bool(self.waiting or self.running or self.swapped)

    def abort_request(self, request_id: str) -> None:
        for queue in (self.waiting, self.running, self.swapped):
            for sg in list(queue):
                if sg.request_id == request_id:
                    for seq in sg.seqs:
                        seq.status = SequenceStatus.FINISHED_ABORT
                        self.block_manager.free(seq.seq_id)
                    queue.remove(sg)

    # ------------------------------------------------------------------
    def _blocks_missing(self, seq_id: int, upto_tokens: int) -> int:
        bs = self.cache_config.block_size
        have = len(self.block_manager.block_tables.get(seq_id, ()))
        return (upto_tokens + bs - 1) // bs - have

    def _grow(self, seq_id: int, n: int) -> None:
        for _ in range(n):
            self.block_manager.append_slot(seq_id)

    def schedule(self) -> SchedulerOutput:
        cfg = self.config
        budget_tokens, budget_seqs = cfg.max_num_batched_tokens, cfg.max_num_seqs
        used_tokens = used_seqs = 0
        decodes: list[SequenceGroup] = []
        prefills: list[SequenceGroup] = []

        def chunk_for(remaining: int) -> int:
            left = budget_tokens - used_tokens
            return min(remaining, cfg.chunk_size, left) if cfg.chunked_prefill else \
                min(remaining, left)

        # 1) decodes, then continuing prefill chunks, in running order
        for phase in ("decode", "prefill"):
            for sg in self.running:
                seqs = sg.get_unfinished_seqs()
                if not seqs or any(s.is_prefill for s in seqs) != (phase == "prefill"):
                    continue
                if used_seqs + len(seqs) > budget_seqs or used_tokens >= budget_tokens:
                    continue
                if phase == "decode":
                    # a token still in flight counts: the next position is
                    # total_len + num_inflight - 1; a sequence whose in-flight
                    # tokens already reach max_tokens is finishing, not fed
                    max_tokens = sg.sampling_params.max_tokens
                    if all(s.data.output_len + s.num_inflight >= max_tokens for s in seqs):
                        continue
                    need = sum(self._blocks_missing(s.seq_id, s.data.total_len + s.num_inflight)
                               for s in seqs)
                    if used_tokens + len(seqs) > budget_tokens or \
                            (need > 0 and not self.block_manager.can_allocate(need)):
                        continue
                    for s in seqs:
                        self._grow(s.seq_id, self._blocks_missing(
                            s.seq_id, s.data.total_len + s.num_inflight))
                        s.num_scheduled_tokens = 1
                    used_tokens += len(seqs)
                    decodes.append(sg)
                else:
                    seq = seqs[0]
                    chunk = chunk_for(seq.data.prompt_len - seq.num_computed_tokens)
                    if chunk <= 0:
                        continue
                    need = self._blocks_missing(seq.seq_id, seq.num_computed_tokens + chunk)
                    if need > 0 and not self.block_manager.can_allocate(need):
                        continue
                    self._grow(seq.seq_id, need)
                    seq.num_scheduled_tokens = chunk
                    used_tokens += chunk
                    prefills.append(sg)
                used_seqs += len(seqs)

        # 2) admit waiting requests (FCFS, stop at the first that does not fit)
        bs = self.cache_config.block_size
        while self.waiting and used_seqs < budget_seqs and used_tokens < budget_tokens:
            sg = self.waiting[0]
            seq = sg.seqs[0]
            prompt = seq.data.prompt_token_ids
            cached, n_cached = ([], 0)
            if self.prefix_cache is not None:
                cached, n_cached = self.prefix_cache.lookup(prompt, self.block_manager)
                if n_cached >= len(prompt):      # keep one token to produce logits
                    cached, n_cached = cached[:-1], n_cached - bs
            chunk = chunk_for(len(prompt) - n_cached)
            if chunk <= 0:
                break
            fresh = (n_cached + chunk + bs - 1) // bs - len(cached)
            if fresh > 0 and not self.block_manager.can_allocate(fresh):
                break
            self.waiting.popleft()
            self.block_manager.allocate(seq.seq_id, max(fresh, 0), prefix=cached)
            seq.num_computed_tokens = n_cached
            if n_cached:
                self.prefix_cache.hit_tokens += n_cached
            seq.num_scheduled_tokens = chunk
            seq.status = SequenceStatus.RUNNING
            self.running.append(sg)
            prefills.append(sg)
            used_tokens += chunk
            used_seqs += 1

        return SchedulerOutput(scheduled_seq_groups=decodes + prefills,
                               num_prefill_groups=len(prefills), num_decode_groups=len(decodes))

    def free_finished(self) -> list[SequenceGroup]:
        finished, still = [], []
        for sg in self.running:
            if sg.is_finished:
                for seq in sg.seqs:
                    self.block_manager.free(seq.seq_id)
                finished.append(sg)
            else:
                still.append(sg)
        self.running = still
        return finished

    def update_running(self, scheduled: list[SequenceGroup]) -> None:
        """Scheduled groups are already in `running` (admission moves them);
        kept for interface compatibility."""
        running = set(map(id, self.running))
        for sg in scheduled:
            if id(sg) not in running:
                self.running.append(sg)
