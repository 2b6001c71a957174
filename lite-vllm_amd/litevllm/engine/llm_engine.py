"""LLMEngine: schedule -> one mixed forward -> one fused sampling launch ->
bookkeeping.

Interface of the reference (engine/llm_engine.py:29-245: initialize,
add_request, step, has_unfinished, run_to_completion) and the same stop rules
(EOS, stop_token_ids, max_tokens, stop strings; llm_engine.py:201-229).  A
step runs ONE forward for the whole scheduled batch (the reference runs one
for the decodes plus one per prefill group, llm_engine.py:127-138) and
samples every finished row with one lv_sample call and one device-to-host
copy (the reference calls Sampler.sample and .item() per sequence,
llm_engine.py:197).  Steps overlap: step k is launched before step k-1's
sampled ids are read back, its decodes take their input ids straight from
step k-1's device output, and the host bookkeeping of step k-1 runs while
the GPU computes step k (a sequence that stops on EOS or a stop string thus
computes one extra token, which is dropped; max_tokens is known ahead and
costs nothing).  Text is produced only when somebody reads it: streamed
deltas and stop strings decode only the newest tokens (incremental
detokenization, O(1) per token instead of the reference's full decode per
step, llm_engine.py:151-158, 213-219); a finished request's text is one full
decode, as in the reference.
"""

from __future__ import annotations

import os
import uuid
from dataclasses import dataclass
from typing import Optional

import torch

from .. import ops
from ..cache.block_manager import BlockManager
from ..cache.prefix_cache import PrefixCache
from ..config import EngineConfig, SamplingParams
from ..layers.sampler import Sampler
from ..tokenizer import IncrementalDetokenizer, TokenizerGroup, get_tokenizer
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import Sequence, SequenceGroup, SequenceGroupOutput, SequenceStatus


@dataclass
class _InFlightStep:
    """A launched step whose sampled ids have not been read back yet."""
    groups: list[SequenceGroup]
    sample_seqs: list[Sequence]
    sample_groups: list[SequenceGroup]
    ids_dev: Optional[torch.Tensor]     # sampled ids on the device
    ids_host: Optional[torch.Tensor]    # their pinned host copy (async)
    done: Optional["torch.cuda.Event"]  # recorded after the copy


class LLMEngine:
    def __init__(self, engine_config: EngineConfig) -> None:
        self.config = engine_config
        self.tokenizer: Optional[TokenizerGroup] = None
        self.model_runner: Optional[ModelRunner] = None
        self.scheduler: Optional[Scheduler] = None
        self.block_manager: Optional[BlockManager] = None
        self.prefix_cache: Optional[PrefixCache] = None
        self.sampler = Sampler()
        self.stream_text = False   # AsyncLLM turns this on to get per-step deltas
        self._rng: Optional[torch.Generator] = None
        self._inflight: Optional[_InFlightStep] = None
        # LITEVLLM_CHECK_INDICES=1: check the kernels' index report every step
        # (one device synchronisation per step; otherwise once per generate)
        self._check_every_step = os.environ.get("LITEVLLM_CHECK_INDICES", "0") == "1"

    def initialize(self) -> None:
        self.config.resolve()
        mc = self.config.model_config
        if not self.config.skip_tokenizer_init:
            self.tokenizer = get_tokenizer(mc.model, mc.trust_remote_code, mc.revision)
        self.model_runner = ModelRunner(self.config)
        self.model_runner.load_model()
        cc = self.config.cache_config
        if cc.num_gpu_blocks is None:
            cc.num_gpu_blocks = self.model_runner.profile_num_gpu_blocks()
        self.model_runner.init_kv_cache(cc.num_gpu_blocks)
        use_graphs = (not self.config.enforce_eager and self.config.device != "cpu"
                      and torch.cuda.is_available())
        # graph replays pad the batch with rows that write into block 0
        self.block_manager = BlockManager(cc.block_size, cc.num_gpu_blocks, cc.num_cpu_blocks,
                                          reserved_blocks=1 if use_graphs else 0)
        if cc.enable_prefix_caching:
            self.prefix_cache = PrefixCache(cc.block_size, self.block_manager)
        self.scheduler = Scheduler(self.config.scheduler_config, cc, self.block_manager,
                                   self.prefix_cache)
        if use_graphs:
            self.model_runner.capture_decode_graphs()
        dev = torch.device(self.config.device)
        self._rng = torch.Generator(device=dev)
        self._rng.manual_seed(self.config.seed)

    # ------------------------------------------------------------------
    def add_request(self, prompt: Optional[str], sampling_params: SamplingParams,
                    request_id: Optional[str] = None,
                    prompt_token_ids: Optional[list[int]] = None) -> str:
        if request_id is None:
            request_id = str(uuid.uuid4())
        if prompt_token_ids is None:
            if self.tokenizer is None:
                raise ValueError("no tokenizer: pass prompt_token_ids")
            prompt_token_ids = self.tokenizer.encode(prompt)
        if not prompt_token_ids:
            raise ValueError("empty prompt")
        sg = SequenceGroup.create(request_id, prompt_token_ids, sampling_params,
                                  prompt_text=prompt or "")
        self.scheduler.add_request(sg)
        return request_id

    def has_unfinished(self) -> bool:
        return self.scheduler.has_unfinished() or self._inflight is not None

    def step(self) -> list[SequenceGroupOutput]:
        """Launch this step's forward and sampling, then finish the previous
        step (wait for its sampled ids, append them, apply the stop rules,
        free finished sequences) while the GPU runs this one.  Returns the
        outputs of the step that was finished."""
        sched = self.scheduler.schedule()
        launched = None if sched.is_empty else self._launch(sched)
        prev, self._inflight = self._inflight, launched
        return self._finish(prev) if prev is not None else []

    def run_to_completion(self) -> list[SequenceGroupOutput]:
        finished: list[SequenceGroupOutput] = []
        while self.has_unfinished():
            for out in self.step():
                if out.finished:
                    finished.append(out)
        self.check_device_errors()
        return finished

    def check_device_errors(self) -> None:
        """Raise if a kernel met an out-of-range block id or slot since the
        last check (the kernels clamp them; the reference's indexing would
        have raised).  One device synchronisation."""
        dev = torch.device(self.config.device) if self.model_runner is not None else None
        if dev is not None and dev.type == "cuda":
            ops.check_device_errors(dev)

    # ------------------------------------------------------------------
    def _launch(self, sched) -> "_InFlightStep":
        prev_ids = self._inflight.ids_dev if self._inflight is not None else None
        meta = self.model_runner.prepare_inputs(sched.scheduled_seq_groups, self.block_manager,
                                                device_tokens=prev_ids)
        # the forward runs even when no row is sampled: a chunk that does not
        # finish its prompt still has to write its K/V
        logits = self.model_runner.execute_model(meta)
        ids_dev = ids_host = done = None
        if meta.sample_seqs:
            ids_dev = self._sample(logits, meta)
            ids_host = ids_dev.to("cpu", non_blocking=True)
            done = torch.cuda.Event()
            done.record()
        # progress is booked at launch: later steps are ordered after this
        # one on the stream, so they see its K/V
        for sg in sched.scheduled_seq_groups:
            for seq in sg.get_unfinished_seqs():
                if seq.is_prefill:
                    seq.num_computed_tokens += seq.num_scheduled_tokens or \
                        (seq.data.prompt_len - seq.num_computed_tokens)
                    if self.prefix_cache is not None:
                        self.prefix_cache.insert(
                            seq.data.prompt_token_ids[:seq.num_computed_tokens],
                            self.block_manager.get_block_table(seq.seq_id))
                else:
                    seq.num_computed_tokens = seq.data.total_len + seq.num_inflight
                seq.num_scheduled_tokens = 0
        for row, seq in enumerate(meta.sample_seqs):
            seq.num_inflight += 1
            seq.inflight_row = row
        return _InFlightStep(sched.scheduled_seq_groups, meta.sample_seqs, meta.sample_groups,
                             ids_dev, ids_host, done)

    def _finish(self, step: "_InFlightStep") -> list[SequenceGroupOutput]:
        if self._check_every_step:
            self.check_device_errors()
        if step.ids_host is not None:
            step.done.synchronize()
            for seq, sg, tok in zip(step.sample_seqs, step.sample_groups, step.ids_host.tolist()):
                seq.num_inflight -= 1
                if seq.status.is_finished:      # stopped before this step's token arrived
                    continue
                seq.data.append_token(tok)
                self._check_stop(seq, sg.sampling_params, tok)
        outputs = []
        for sg in step.groups:
            if sg.final_output_sent:
                continue
            out = self._build_step_output(sg)
            sg.final_output_sent = out.finished
            outputs.append(out)
        self.scheduler.update_running(step.groups)
        self.scheduler.free_finished()
        return outputs

    def _sample(self, logits: torch.Tensor, meta) -> torch.Tensor:
        """Sampled ids of meta.sample_seqs as a device tensor (no host sync)."""
        groups = meta.sample_groups
        simple = all(sg.sampling_params.top_k <= 0 and sg.sampling_params.top_p >= 1.0
                     for sg in groups)
        if simple:
            dev = logits.device
            temps = torch.tensor([sg.sampling_params.temperature for sg in groups],
                                 dtype=torch.float32).to(dev, non_blocking=True)
            uni = torch.rand(len(groups), dtype=torch.float32, device=dev, generator=self._rng)
            return self.sampler.sample_batched(logits, temps, uni)
        out = [self.sampler.sample(logits[i], sg.sampling_params, generator=self._rng)
               for i, sg in enumerate(groups)]
        return torch.cat(out)

    def _check_stop(self, seq: Sequence, params: SamplingParams, token_id: int) -> None:
        eos = self.tokenizer.eos_token_id if self.tokenizer is not None else None
        if not params.ignore_eos and eos is not None and token_id == eos:
            seq.status = SequenceStatus.FINISHED_EOS
        elif token_id in params.stop_token_ids:
            seq.status = SequenceStatus.FINISHED_STOPPED
        elif seq.data.output_len >= params.max_tokens:
            seq.status = SequenceStatus.FINISHED_LENGTH
        elif params.stop and self.tokenizer is not None:
            d = seq.stop_detok
            if d is None:
                d = seq.stop_detok = IncrementalDetokenizer(skip_special_tokens=False)
            start = max(0, len(d.text) - max(len(s) for s in params.stop) + 1)
            d.update(self.tokenizer, seq.data.output_token_ids)
            tail = d.text[start:]      # every match that includes new text
            if any(s in tail for s in params.stop):
                seq.status = SequenceStatus.FINISHED_STOPPED

    def _build_step_output(self, sg: SequenceGroup) -> SequenceGroupOutput:
        seq = sg.seqs[0]
        finished = sg.is_finished
        text, delta = seq.emitted_text, ""
        if self.tokenizer is not None and (finished or self.stream_text):
            skip = sg.sampling_params.skip_special_tokens
            if finished:
                text = self.tokenizer.decode(seq.data.output_token_ids, skip_special_tokens=skip)
            else:
                if seq.detok is None:
                    seq.detok = IncrementalDetokenizer(skip_special_tokens=skip)
                seq.detok.update(self.tokenizer, seq.data.output_token_ids)
                text = seq.detok.text
            delta = text[len(seq.emitted_text):]
            seq.emitted_text = text
        return SequenceGroupOutput(request_id=sg.request_id, prompt_text=sg.prompt_text,
                                   prompt_token_ids=seq.data.prompt_token_ids,
                                   output_token_ids=list(seq.data.output_token_ids)
                                   if finished else seq.data.output_token_ids,
                                   output_text=text, finish_reason=seq.status.value,
                                   delta_text=delta, finished=finished)
