"""Request state: SequenceStatus / SequenceData / Sequence / SequenceGroup /
SequenceGroupOutput with the reference's fields and meanings
(engine/sequence.py:17-167).  Additions for real chunked prefill and cheap
per-step packing: ``Sequence.num_scheduled_tokens`` (tokens fed this step)
and ``SequenceData.last_token`` (no prompt+output list concatenation); for
the overlapped step loop, ``Sequence.num_inflight`` / ``inflight_row``: a
token sampled on the device by the step in flight, not yet appended on the
host, and its row in that step's sampled-ids tensor; for text,
``detok`` (streamed output text) and ``stop_detok`` (text for stop strings,
special tokens kept), both incremental."""

from __future__ import annotations

import enum
import itertools
import time
from dataclasses import dataclass, field
from typing import Optional

from litevllm.config import SamplingParams
from litevllm.tokenizer.detokenizer import IncrementalDetokenizer


class SequenceStatus(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    SWAPPED = "swapped"
    FINISHED_STOPPED = "finished_stopped"
    FINISHED_LENGTH = "finished_length"
    FINISHED_EOS = "finished_eos"
    FINISHED_ABORT = "finished_abort"

    @property
    def is_finished(self) -> bool:
        return self in _FINISHED


_FINISHED = {SequenceStatus.FINISHED_STOPPED, SequenceStatus.FINISHED_LENGTH,
             SequenceStatus.FINISHED_EOS, SequenceStatus.FINISHED_ABORT}


@dataclass
class SequenceData:
    prompt_token_ids: list[int]
    output_token_ids: list[int] = field(default_factory=list)

    @property
    def all_token_ids(self) -> list[int]:
        return self.prompt_token_ids + self.output_token_ids

    @property
    def last_token(self) -> int:
        return self.output_token_ids[-1] if self.output_token_ids else self.prompt_token_ids[-1]

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def output_len(self) -> int:
        return len(self.output_token_ids)

    @property
    def total_len(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    def append_token(self, token_id: int) -> None:
        self.output_token_ids.append(token_id)


_seq_ids = itertools.count(1)


@dataclass
class Sequence:
    seq_id: int
    data: SequenceData
    status: SequenceStatus = SequenceStatus.WAITING
    num_computed_tokens: int = 0   # tokens whose KV is in the cache
    emitted_text: str = ""
    num_scheduled_tokens: int = 0  # tokens fed in the current step
    num_inflight: int = 0          # sampled on the device, not yet appended here
    inflight_row: int = -1         # row of the newest such token in its step's ids
    detok: Optional[IncrementalDetokenizer] = None
    stop_detok: Optional[IncrementalDetokenizer] = None

    @classmethod
    def create(cls, prompt_token_ids: list[int]) -> "Sequence":
        return cls(seq_id=next(_seq_ids), data=SequenceData(list(prompt_token_ids)))

    @property
    def is_prefill(self) -> bool:
        return self.num_computed_tokens < self.data.prompt_len

    @property
    def num_new_tokens(self) -> int:
        """Tokens the next step needs: the rest of the prompt, or one."""
        if self.is_prefill:
            return self.data.prompt_len - self.num_computed_tokens
        return 1

    def get_num_blocks(self, block_size: int) -> int:
        return (self.data.total_len + block_size - 1) // block_size


@dataclass
class SequenceGroup:
    request_id: str
    seqs: list[Sequence]
    sampling_params: SamplingParams
    arrival_time: float = field(default_factory=time.time)
    prompt_text: str = ""
    final_output_sent: bool = False   # the finished output was returned once

    @classmethod
    def create(cls, request_id: str, prompt_token_ids: list[int], sampling_params: SamplingParams,
               prompt_text: str = "") -> "SequenceGroup":
        return cls(request_id=request_id, seqs=[Sequence.create(prompt_token_ids)],
                   sampling_params=sampling_params, prompt_text=prompt_text)

    @property
    def is_finished(self) -> bool:
        return all(s.status.is_finished for s in self.seqs)

    def get_unfinished_seqs(self) -> list[Sequence]:
        return [s for s in self.seqs if not s.status.is_finished]


@dataclass
class SequenceGroupOutput:
    request_id: str
    prompt_text: str
    prompt_token_ids: list[int]
    output_token_ids: list[int]
    output_text: str
    finish_reason: str
    delta_text: str = ""
    finished: bool = True

    @property
    def num_prompt_tokens(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def num_output_tokens(self) -> int:
        return len(self.output_token_ids)
